"""CPU oracle for the Qwen3-MoE FP8 expert hot path.

TEST INFRASTRUCTURE ONLY.  This module is the checker the HIP path is compared
against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it; the product package never does.

It restates, in numpy, the algorithm the reference server runs when its
``TorchBackend`` loads a Qwen3-MoE checkpoint.  The reference
(AdvayMonga/inference-server) contains no MoE code of its own: the math lives in
its dependency ``transformers`` (``pyproject.toml:14`` declares
``transformers>=4.51``; the pinned container copy is 5.15.0).  Citations below use
``TF/`` for ``transformers/``.

Conventions fixed here (the reference leaves them implementation-defined):

* bf16 tensors are carried as float32 arrays whose values are exactly
  representable in bf16; ``round_bf16`` is round-to-nearest-even.
* Top-k order: descending bf16 logit, ties broken by the lower expert id.
  Softmax is monotone, so this equals descending probability except where two
  different logits map to the same fp32 probability.
* The expert sort is stable: by expert id, then by flat pair index ``t*k+j``.
* Activation quantisation (absent from the reference's sources, it sits inside
  a hub Triton kernel, see ``TF/integrations/finegrained_fp8.py:191-196``) is
  defined per row and per 128-column group as ``s = amax/448`` (``s = 1`` when
  ``amax == 0``) and ``q = e4m3(clamp(x / s, -448, 448))``.

Parity status per function (how each is pinned is in ``tests/test_oracle.py``):

* ``e4m3_encode`` / ``e4m3_decode``: pinned (OCP value table, brute-force
  nearest-even search, torch's float8_e4m3fn cast).
* ``round_bf16``: pinned (torch's bfloat16 cast).
* ``quantize_act_fp8``, ``quantize_weight_fp8``, ``dequantize_weight_fp8``:
  pinned (closed forms and error bounds, amax code = 448, zero groups).
* ``route``: pinned (brute-force sort, crafted ties, golden vectors written by
  the transformers router on CPU).
* ``align``: pinned (brute-force loops on tiny inputs, invariants).
* ``experts_fp8`` / ``experts_bf16``: pinned (token-major brute force; the bf16
  variant against golden vectors from ``Qwen3MoeSparseMoeBlock`` on CPU).
"""

from __future__ import annotations

import numpy as np

FP8_MAX = 448.0
GROUP = 128

# ----------------------------------------------------------------------------
# bf16
# ----------------------------------------------------------------------------


def round_bf16(a) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), returned as float32."""
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    bits = a.view(np.uint32)
    # finite inputs cannot overflow 32 bits here; NaNs are restored below
    rounded = (bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    out = rounded.view(np.float32).reshape(a.shape)
    nan = np.isnan(a)
    if nan.any():
        out = np.where(nan, np.float32(np.nan), out)
    return out


def bf16_bits(a) -> np.ndarray:
    """uint16 bit patterns of bf16-representable float32 values."""
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    return (a.view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(bits) -> np.ndarray:
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------
# FP8 E4M3 (OCP "fn" variant: no infinities, 0x7F/0xFF are NaN, max 448)
# ----------------------------------------------------------------------------


def e4m3_table() -> np.ndarray:
    """Value of each of the 256 e4m3fn codes, straight from the OCP FP8 definition."""
    vals = np.zeros(256, dtype=np.float32)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> 3) & 0xF
        man = code & 0x7
        if exp == 0xF and man == 0x7:
            vals[code] = np.nan
        elif exp == 0:
            vals[code] = sign * (man / 8.0) * 2.0 ** (-6)
        else:
            vals[code] = sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)
    return vals


_E4M3 = e4m3_table()


def e4m3_decode(codes) -> np.ndarray:
    return _E4M3[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(v) -> np.ndarray:
    """Round float32 values already clamped to [-448, 448] to e4m3fn codes (RNE)."""
    v = np.asarray(v, dtype=np.float32)
    sign = np.signbit(v)
    a = np.abs(v).astype(np.float32)
    if np.any(a > FP8_MAX) or np.any(np.isnan(a)):
        raise ValueError("e4m3_encode expects finite inputs clamped to +-448")
    code = np.zeros(a.shape, dtype=np.int32)
    sub = a < np.float32(2.0 ** -6)
    # Subnormal range: value = m * 2^-9 with m in [0, 8]; scaling by 2^9 is exact.
    m = np.rint(a[sub] * np.float32(512.0)).astype(np.int32)
    code[sub] = m  # m == 8 lands on the smallest normal code 0x08, as it should
    nrm = ~sub
    # Normal range: round the fp32 mantissa to 3 bits, ties to even, on the bit pattern.
    bits = a[nrm].view(np.uint32).astype(np.uint64)
    lsb = (bits >> 20) & 1
    rb = (bits + 0x7FFFF + lsb) >> 20  # exponent and 3 mantissa bits; carries roll into the exponent
    exp = (rb >> 3).astype(np.int64) - 127
    code[nrm] = (((exp + 7) << 3) | (rb & 7).astype(np.int64)).astype(np.int32)
    code = np.where(sign, code | 0x80, code)
    return code.astype(np.uint8)


def quantize_act_fp8(x, group: int = GROUP):
    """Dynamic per-row, per-``group``-column quantisation of activations.

    The reference's FP8 grouped GEMM quantises its bf16 input inline
    (``TF/integrations/finegrained_fp8.py:191-196``, kernel source not shipped).
    Returns (codes uint8 [R, C], scales float32 [R, C/group]).
    """
    x = np.asarray(x, dtype=np.float32)
    R, C = x.shape
    if C % group:
        raise ValueError("columns must be a multiple of the group size")
    xg = x.reshape(R, C // group, group)
    amax = np.abs(xg).max(axis=-1)
    s = (amax / np.float32(FP8_MAX)).astype(np.float32)
    s = np.where(amax > 0, s, np.float32(1.0)).astype(np.float32)
    y = (xg / s[..., None]).astype(np.float32)
    y = np.clip(y, -FP8_MAX, FP8_MAX)
    return e4m3_encode(y).reshape(R, C), s


def dequantize_act_fp8(codes, scales, group: int = GROUP) -> np.ndarray:
    R, C = codes.shape
    v = e4m3_decode(codes).reshape(R, C // group, group)
    return (v * scales[..., None]).reshape(R, C).astype(np.float32)


def quantize_weight_fp8(w, block: int = GROUP):
    """Per 128x128 tile weight quantiser, ``Fp8Quantize._quantize_one``
    (``TF/integrations/finegrained_fp8.py:903-941``).

    ``scale = 448 / amax`` (1 where amax == 0), ``q = e4m3(clamp(w * scale))``,
    stored inverse ``scale_inv = 1 / scale`` in fp32.  w: [..., N, K].
    Returns (codes uint8 [..., N, K], scale_inv float32 [..., N/128, K/128]).
    """
    w = np.asarray(w, dtype=np.float32)
    *lead, N, K = w.shape
    if N % block or K % block:
        raise ValueError("weight dims must be multiples of the block size")
    t = w.reshape(*lead, N // block, block, K // block, block)
    amax = np.abs(t).max(axis=(-3, -1))
    safe = np.where(amax > 0, amax, np.float32(1.0)).astype(np.float32)
    scale = (np.float32(FP8_MAX) / safe).astype(np.float32)
    scale = np.where(amax > 0, scale, np.float32(1.0)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    y = (t * scale[..., :, None, :, None]).astype(np.float32)
    y = np.clip(y, -FP8_MAX, FP8_MAX)
    return e4m3_encode(y).reshape(w.shape), inv


def dequantize_weight_fp8(codes, scale_inv, block: int = GROUP) -> np.ndarray:
    """``Fp8Dequantize._dequantize_one`` (``TF/integrations/finegrained_fp8.py:1005-1048``)."""
    codes = np.asarray(codes, dtype=np.uint8)
    *lead, N, K = codes.shape
    v = e4m3_decode(codes).reshape(*lead, N // block, block, K // block, block)
    s = np.asarray(scale_inv, dtype=np.float32)[..., :, None, :, None]
    return (v * s).reshape(codes.shape).astype(np.float32)


# ----------------------------------------------------------------------------
# Routing: Qwen3MoeTopKRouter.forward (TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267)
# ----------------------------------------------------------------------------


def router_logits(x, w_router) -> np.ndarray:
    """``F.linear(hidden, weight)`` in bf16 (``modeling_qwen3_moe.py:260``): exact-ish
    fp64 accumulation, one rounding to fp32 then to bf16."""
    acc = np.asarray(x, np.float64) @ np.asarray(w_router, np.float64).T
    return round_bf16(acc.astype(np.float32))


def topk_from_logits(logits, k: int, renorm: bool = True):
    """softmax(fp32) -> top-k -> optional renormalise -> bf16 (``modeling_qwen3_moe.py:261-266``).

    Returns (ids int32 [T,k], weights float32 (bf16 values) [T,k], probs float32 [T,E]).
    """
    lg = np.asarray(logits, dtype=np.float32)
    T, E = lg.shape
    m = lg.max(axis=1, keepdims=True)
    e = np.exp((lg - m).astype(np.float32)).astype(np.float32)
    z = e.sum(axis=1, keepdims=True, dtype=np.float32)
    p = (e / z).astype(np.float32)
    ids = np.empty((T, k), dtype=np.int32)
    for t in range(T):
        order = np.lexsort((np.arange(E), -lg[t].astype(np.float64)))
        ids[t] = order[:k]
    top = np.take_along_axis(p, ids.astype(np.int64), axis=1)
    if renorm:
        s = np.zeros((T, 1), dtype=np.float32)
        for j in range(k):  # sequential fp32 sum in top-k order
            s = (s + top[:, j : j + 1]).astype(np.float32)
        top = (top / s).astype(np.float32)
    return ids, round_bf16(top), p


def route(x, w_router, k: int, renorm: bool = True):
    """Whole router: returns (logits bf16-as-f32 [T,E], ids int32 [T,k], weights [T,k])."""
    lg = router_logits(x, w_router)
    ids, w, _ = topk_from_logits(lg, k, renorm)
    return lg, ids, w


# ----------------------------------------------------------------------------
# Sort / align: TF/integrations/moe.py:389-403
# ----------------------------------------------------------------------------


def align(ids, num_experts: int):
    """Stable expert sort of the flat (token, slot) pairs.

    ``torch.sort(expert_ids)`` + ``histc`` + ``cumsum`` (``moe.py:393-403``), with the
    stable tie rule.  Returns (perm int32 [S], counts int32 [E], offsets int32 [E+1])
    where ``offsets`` is exclusive (``offsets[1:]`` equals the reference's inclusive
    ``cumsum``).
    """
    flat = np.asarray(ids, dtype=np.int64).reshape(-1)
    perm = np.argsort(flat, kind="stable").astype(np.int32)
    counts = np.bincount(flat, minlength=num_experts).astype(np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    return perm, counts, offsets


def tile_list(counts, block_m: int):
    """(expert, first sorted row, rows) for every ``block_m``-row tile of every expert."""
    out = []
    start = 0
    for e, c in enumerate(np.asarray(counts)):
        for r in range(0, int(c), block_m):
            out.append((e, start + r, min(block_m, int(c) - r)))
        start += int(c)
    return np.asarray(out, dtype=np.int32).reshape(-1, 3)


# ----------------------------------------------------------------------------
# Experts
# ----------------------------------------------------------------------------


def silu_mul_bf16(gate, up) -> np.ndarray:
    """``act_fn(gate) * up`` on bf16 tensors (``moe.py:509-520``): silu is evaluated in
    fp32 and rounded to bf16, then the bf16 product is rounded again."""
    g = np.asarray(gate, np.float32)
    sg = round_bf16((g / (np.float32(1.0) + np.exp(-g.astype(np.float64)).astype(np.float32))).astype(np.float32))
    return round_bf16((sg * np.asarray(up, np.float32)).astype(np.float32))


def _matmul(a, b_t, acc):
    return (np.asarray(a, acc) @ np.asarray(b_t, acc).T).astype(np.float32)


def experts_fp8(x, ids, weights, w13_q, s13, w2_q, s2, acc=np.float64, return_intermediates=False):
    """FP8 grouped experts forward, ``fp8_grouped_mm_experts_forward``
    (``TF/integrations/finegrained_fp8.py:498-589``), with the FP8 GEMM restated as
    dequantise-then-matmul (``finegrained_fp8.py:1005-1048``) and the dynamic
    activation quantisation defined in the module docstring.

    x bf16 [T,H]; ids [T,k]; weights bf16 [T,k]; w13_q uint8 [E,2I,H]; s13 [E,2I/128,H/128];
    w2_q uint8 [E,H,I]; s2 [E,H/128,I/128].  Returns bf16-valued float32 [T,H].
    """
    x = np.asarray(x, np.float32)
    T, H = x.shape
    ids = np.asarray(ids)
    k = ids.shape[1]
    E, I2, _ = w13_q.shape
    I = I2 // 2
    perm, counts, offsets = align(ids, E)
    xq, sx = quantize_act_fp8(x)
    xd = dequantize_act_fp8(xq, sx)  # per token; every pair of a token sees the same row
    wflat = np.asarray(weights, np.float32).reshape(-1)
    S = T * k
    h_sorted = np.zeros((S, I), np.float32)
    z_pairs = np.zeros((S, H), np.float32)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if lo == hi:
            continue
        rows = perm[lo:hi]
        a = xd[rows // k]
        wd = dequantize_weight_fp8(w13_q[e], s13[e])
        y = round_bf16(_matmul(a, wd, acc))  # grouped_matmul returns bf16
        h = silu_mul_bf16(y[:, :I], y[:, I:])
        h_sorted[lo:hi] = h
        hq, sh = quantize_act_fp8(h)
        hd = dequantize_act_fp8(hq, sh)
        w2d = dequantize_weight_fp8(w2_q[e], s2[e])
        z = round_bf16(_matmul(hd, w2d, acc))
        z_pairs[rows] = round_bf16(z * wflat[rows][:, None])  # bf16 * bf16
    out = np.zeros((T, H), np.float32)
    zp = z_pairs.reshape(T, k, H)
    for j in range(k):  # view(T,k,H).sum(1): fp32 accumulation in slot order
        out = (out + zp[:, j]).astype(np.float32)
    out = round_bf16(out)
    if return_intermediates:
        return out, dict(perm=perm, counts=counts, offsets=offsets, xq=xq, sx=sx,
                         h_sorted=h_sorted, z_pairs=z_pairs)
    return out


def experts_bf16(x, ids, weights, w13, w2, acc=np.float64):
    """bf16 grouped experts forward, ``grouped_mm_experts_forward`` (``TF/integrations/moe.py:377-478``):
    each grouped GEMM returns bf16, ``silu(gate) * up`` in bf16, bf16 routing-weight product,
    then the fp32 ``view(T,k,H).sum(1)`` and a final bf16 cast."""
    x = np.asarray(x, np.float32)
    T, H = x.shape
    ids = np.asarray(ids)
    k = ids.shape[1]
    E, I2, _ = w13.shape
    I = I2 // 2
    perm, counts, offsets = align(ids, E)
    wflat = np.asarray(weights, np.float32).reshape(-1)
    z_pairs = np.zeros((T * k, H), np.float32)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if lo == hi:
            continue
        rows = perm[lo:hi]
        y = round_bf16(_matmul(x[rows // k], w13[e], acc))
        h = silu_mul_bf16(y[:, :I], y[:, I:])
        z = round_bf16(_matmul(h, w2[e], acc))
        z_pairs[rows] = round_bf16(z * wflat[rows][:, None])
    out = np.zeros((T, H), np.float32)
    zp = z_pairs.reshape(T, k, H)
    for j in range(k):
        out = (out + zp[:, j]).astype(np.float32)
    return round_bf16(out)


def moe_block_fp8(x, w_router, k, w13_q, s13, w2_q, s2, renorm=True, acc=np.float64):
    """``Qwen3MoeSparseMoeBlock.forward`` (``modeling_qwen3_moe.py:276-281``) with FP8 experts."""
    lg, ids, w = route(x, w_router, k, renorm)
    return experts_fp8(x, ids, w, w13_q, s13, w2_q, s2, acc=acc), (lg, ids, w)


# ----------------------------------------------------------------------------
# Synthetic inputs for the benchmark configurations (seeded, numpy PCG64)
# ----------------------------------------------------------------------------


def gen_normal_bf16(rng, shape, std=1.0) -> np.ndarray:
    return round_bf16((rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32))


def uniform_routing(rng, T, E, k):
    """k distinct uniformly random experts per token; weights = renormalised softmax of
    N(0,1) logits at those ids, rounded to bf16, ordered by descending weight."""
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    lg = rng.standard_normal((T, k)).astype(np.float32)
    order = np.argsort(-lg, axis=1, kind="stable")
    ids = np.take_along_axis(ids, order, axis=1)
    lg = np.take_along_axis(lg, order, axis=1)
    e = np.exp(lg - lg.max(axis=1, keepdims=True)).astype(np.float32)
    w = round_bf16(e / e.sum(axis=1, keepdims=True))
    return ids, w


def zipf_bias(E, s=1.1, beta=1.0, seed=0):
    """Router-logit bias ``b_e = beta * (-s * ln r_e)`` with r a seeded permutation of 1..E."""
    r = np.random.default_rng(seed).permutation(E) + 1
    return (beta * (-s * np.log(r))).astype(np.float32)
