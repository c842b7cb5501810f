"""HIP path vs the CPU oracle, through the C ABI (via the torch wrappers).

Integer / byte / index outputs must be bit-exact; bf16 layer outputs must be within
max-abs 2e-2 and mean-relative 1e-2 of the dequantise-then-fp32 oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc
from tests.helpers import (TOL_MAX_ABS, TOL_MEAN_REL, bf16_ulp_diff, errors, f8_codes, gpu_weights, np_f32,
                           to_bf16, to_dev, to_f8)

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------------------
# quantisers (bit-exact)
# ---------------------------------------------------------------------------


def test_quant_act_bit_exact(pkg, dev):
    rng = np.random.default_rng(1)
    R, C = 96, 2048
    x = orc.gen_normal_bf16(rng, (R, C))
    x[3, 128:256] = 0.0                                   # zero group -> scale 1, codes 0
    x[4] = orc.round_bf16(x[4] * 1e-6)                    # tiny values: fp8 subnormals
    x[5] = orc.round_bf16(x[5] * 3e4)                     # large values
    x[6, :128] = orc.round_bf16(np.linspace(-1, 1, 128, dtype=np.float32))
    x[7, 5] = -0.0
    q, s = pkg.quantize_act_fp8(to_bf16(x, dev))
    q_ref, s_ref = orc.quantize_act_fp8(x)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(f8_codes(q), q_ref)


@pytest.mark.parametrize("dtype", ["bf16", "fp32"])
def test_quant_weight_bit_exact(pkg, dev, dtype):
    rng = np.random.default_rng(2)
    w = rng.standard_normal((3, 256, 384), dtype=np.float32) * np.float32(0.02)
    w[1, :128, :128] = 0.0
    w[2, 128:, 256:] *= np.float32(1e-5)
    if dtype == "bf16":
        w = orc.round_bf16(w)
        wt = to_bf16(w, dev)
    else:
        wt = to_dev(w.astype(np.float32), dev)
    q, s = pkg.quantize_weight_fp8(wt)
    q_ref, s_ref = orc.quantize_weight_fp8(w)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(f8_codes(q), q_ref)


# ---------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------


def _crafted_logits(T, E, rng):
    lg = orc.gen_normal_bf16(rng, (T, E))
    lg[0, :] = 0.5                                        # all tied: ids 0..k-1
    lg[1, ::2] = 1.0                                      # ties inside and at the k boundary
    lg[2, 100:] = 3.0
    lg[3, 7] = -0.0
    lg[3, 9] = 0.0
    lg[4, :] = orc.round_bf16(np.float32(-1e-30) * np.arange(E, dtype=np.float32))
    return lg


@pytest.mark.parametrize("E,k", [(128, 8), (64, 4), (256, 8), (100, 6)])
@pytest.mark.parametrize("index_dtype", [torch.int32, torch.int64])
def test_topk_softmax_bit_exact(pkg, dev, E, k, index_dtype):
    rng = np.random.default_rng(3)
    T = 333
    lg = _crafted_logits(T, E, rng)
    w, ids = pkg.topk_softmax(to_bf16(lg, dev), k, True, index_dtype=index_dtype)
    ids_ref, w_ref, _ = orc.topk_from_logits(lg, k, True)
    assert ids.dtype == index_dtype
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    assert bf16_ulp_diff(np_f32(w), w_ref).max() <= 1
    w_nr, ids_nr = pkg.topk_softmax(to_bf16(lg, dev), k, False)
    ids_ref_nr, w_ref_nr, _ = orc.topk_from_logits(lg, k, False)
    np.testing.assert_array_equal(ids_nr.cpu().numpy(), ids_ref_nr)
    assert bf16_ulp_diff(np_f32(w_nr), w_ref_nr).max() <= 1


@pytest.mark.parametrize("T,H,E,k", [(1, 2048, 128, 8), (16, 2048, 128, 8), (257, 2048, 128, 8),
                                     (4096, 2048, 128, 8), (64, 4096, 128, 8), (33, 256, 48, 3)])
def test_route(pkg, dev, T, H, E, k):
    rng = np.random.default_rng(4)
    x = orc.gen_normal_bf16(rng, (T, H))
    wr = orc.gen_normal_bf16(rng, (E, H), 0.02)
    lg, w, ids = pkg.route(to_bf16(x, dev), to_bf16(wr, dev), k)
    lg_ref = orc.router_logits(x, wr)
    lg_gpu = np_f32(lg)
    # one bf16 rounding of the fp32 sum, plus the fp32 accumulation error, which is
    # bounded by a small multiple of eps * sum|x_i w_i| (it matters for logits near 0)
    abs_sum = np.abs(x.astype(np.float64)) @ np.abs(wr.astype(np.float64)).T
    ulp_ref = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(lg_ref), 1e-30))) - 7)
    assert np.all(np.abs(lg_gpu - lg_ref) <= ulp_ref + 1e-5 * abs_sum)
    assert (bf16_ulp_diff(lg_gpu, lg_ref) > 0).mean() <= 2e-3
    ids_ref, w_ref, _ = orc.topk_from_logits(lg_gpu, k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    assert bf16_ulp_diff(np_f32(w), w_ref).max() <= 1


# ---------------------------------------------------------------------------
# sort / align (bit-exact)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("T,k,E,block_m", [(1, 8, 128, 16), (16, 8, 128, 16), (64, 8, 128, 16),
                                           (256, 8, 128, 128), (257, 8, 128, 128),  # one WG / chunked
                                           (512, 8, 128, 16), (513, 8, 128, 64), (4096, 8, 128, 64),
                                           (3000, 4, 60, 32), (4096, 8, 128, 256), (0, 8, 128, 16)])
@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_align_bit_exact(pkg, dev, T, k, E, block_m, index_dtype):
    rng = np.random.default_rng(5 + T)
    ids = np.array([rng.permutation(E)[:k] for _ in range(T)], dtype=index_dtype).reshape(T, k)
    if T >= 16:
        ids[: T // 2, 0] = 3  # skew: one hot expert
    out = pkg.align(to_dev(ids, dev), E, block_m)
    perm, counts, offsets = orc.align(ids, E)
    np.testing.assert_array_equal(out["perm"].cpu().numpy(), perm)
    np.testing.assert_array_equal(out["counts"].cpu().numpy(), counts)
    np.testing.assert_array_equal(out["offsets"].cpu().numpy(), offsets)
    tl = orc.tile_list(counts, block_m)
    n = int(out["n_tiles"].cpu().item())
    assert n == len(tl)
    np.testing.assert_array_equal(out["tiles"].cpu().numpy()[:n, :3], tl)


def test_align_sentinels(pkg, dev):
    """Ids outside [0, E) are left out of counts and go, stably, to the tail of perm."""
    rng = np.random.default_rng(6)
    T, k, E = 700, 8, 128
    ids = rng.integers(0, E, size=(T, k)).astype(np.int64)
    ids[rng.random((T, k)) < 0.1] = E + 5
    ids[5, 2] = -1
    out = pkg.align(to_dev(ids, dev), E, 16)
    flat = ids.reshape(-1)
    valid = (flat >= 0) & (flat < E)
    key = np.where(valid, flat, E)
    perm_ref = np.argsort(key, kind="stable")
    np.testing.assert_array_equal(out["perm"].cpu().numpy(), perm_ref)
    np.testing.assert_array_equal(out["counts"].cpu().numpy(), np.bincount(flat[valid], minlength=E))
    assert int(out["offsets"][E].item()) == int(valid.sum())


# ---------------------------------------------------------------------------
# experts / block
# ---------------------------------------------------------------------------


def _check_experts(pkg, dev, x, ids, w, q13, s13, q2, s2, idx_subset=None):
    out = pkg.experts_fp8(to_bf16(x, dev), to_dev(ids, dev), to_bf16(w, dev), q13, s13, q2, s2)
    o = np_f32(out)
    q13n, s13n, q2n, s2n = f8_codes(q13), s13.cpu().numpy(), f8_codes(q2), s2.cpu().numpy()
    sel = slice(None) if idx_subset is None else idx_subset
    ref = orc.experts_fp8(x[sel], ids[sel], w[sel], q13n, s13n, q2n, s2n, acc=np.float32)
    max_abs, mean_rel = errors(o[sel], ref)
    assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL, (max_abs, mean_rel)
    return out, max_abs, mean_rel


@pytest.fixture(scope="module")
def w30b(dev):
    return gpu_weights(128, 2048, 768, dev, seed=0)


@pytest.mark.parametrize("T", [1, 8, 32, 64, 128, 256])
def test_experts_decode_30b(pkg, dev, w30b, T):
    rng = np.random.default_rng(10 + T)
    x = orc.gen_normal_bf16(rng, (T, 2048))
    ids, w = orc.uniform_routing(rng, T, 128, 8)
    _check_experts(pkg, dev, x, ids, w, *w30b)


@pytest.mark.parametrize("R", [8, 512])
def test_experts_ep_share_30b(pkg, dev, R):
    """One GPU's share of 8-way expert parallelism (bench.py's ep_share entry): 16 local experts at
    the 30B H / I, R received rows with one local expert each (k = 1); 8 rows take the 16-row
    tiles, 512 rows the 128-row prefill tiles (S > 8 E)."""
    E = 16
    rng = np.random.default_rng(20 + R)
    x = orc.gen_normal_bf16(rng, (R, 2048))
    ids = rng.integers(0, E, size=(R, 1)).astype(np.int32)
    w = orc.round_bf16(rng.uniform(0.25, 1.0, size=(R, 1)).astype(np.float32))
    _check_experts(pkg, dev, x, ids, w, *gpu_weights(E, 2048, 768, dev, seed=3),
                   idx_subset=np.arange(0, R, max(1, R // 128)))


def test_experts_prefill_skewed_30b(pkg, dev, w30b):
    """4096-token chunk with Zipf-skewed routing; 96 random tokens checked (tokens are independent;
    tests/test_gpu_configs.py checks a token of every tile)."""
    T, H, E, k = 4096, 2048, 128, 8
    rng = np.random.default_rng(11)
    x = orc.gen_normal_bf16(rng, (T, H))
    lg = orc.gen_normal_bf16(rng, (T, E)) + orc.zipf_bias(E, 1.1, beta=1.5)
    ids, w, _ = orc.topk_from_logits(orc.round_bf16(lg), k)
    sub = np.sort(rng.choice(T, 96, replace=False))
    _check_experts(pkg, dev, x, ids, w, *w30b, idx_subset=sub)


@pytest.mark.parametrize("T", [300, 1024])
def test_experts_prefill_uniform_30b(pkg, dev, w30b, T):
    """128-row LDS-tiled path (S > 16 E) with ragged last tiles per expert."""
    rng = np.random.default_rng(20 + T)
    x = orc.gen_normal_bf16(rng, (T, 2048))
    ids, w = orc.uniform_routing(rng, T, 128, 8)
    sub = np.sort(rng.choice(T, min(T, 80), replace=False))
    _check_experts(pkg, dev, x, ids, w, *w30b, idx_subset=sub)


def test_experts_64row_path_odd_hidden(pkg, dev):
    """H % 256 != 0 takes the 64-row register-tiled path for prefill-sized batches."""
    E, H, I, k, T = 4, 384, 256, 2, 96
    q13, s13, q2, s2 = gpu_weights(E, H, I, dev, seed=5)
    rng = np.random.default_rng(21)
    x = orc.gen_normal_bf16(rng, (T, H))
    ids, w = orc.uniform_routing(rng, T, E, k)
    _check_experts(pkg, dev, x, ids, w, q13, s13, q2, s2)


def test_experts_deterministic(pkg, dev, w30b):
    rng = np.random.default_rng(12)
    T = 300
    x = to_bf16(orc.gen_normal_bf16(rng, (T, 2048)), dev)
    ids, w = orc.uniform_routing(rng, T, 128, 8)
    a = pkg.experts_fp8(x, to_dev(ids, dev), to_bf16(w, dev), *w30b)
    b = pkg.experts_fp8(x, to_dev(ids, dev), to_bf16(w, dev), *w30b)
    assert torch.equal(a, b)


def test_experts_235b_shape(pkg, dev):
    E, H, I, k, T = 16, 4096, 1536, 8, 64  # 235B per-expert shape, a 16-expert slice
    q13, s13, q2, s2 = gpu_weights(E, H, I, dev, seed=3)
    rng = np.random.default_rng(13)
    x = orc.gen_normal_bf16(rng, (T, H))
    ids, w = orc.uniform_routing(rng, T, E, k)
    _check_experts(pkg, dev, x, ids, w, q13, s13, q2, s2)


def test_block_matches_oracle(pkg, dev):
    T, H, I, E, k = 48, 512, 256, 32, 4
    rng = np.random.default_rng(14)
    x = orc.gen_normal_bf16(rng, (T, H))
    wr = orc.gen_normal_bf16(rng, (E, H), 0.02)
    w13 = orc.gen_normal_bf16(rng, (E, 2 * I, H), 0.02)
    w2 = orc.gen_normal_bf16(rng, (E, H, I), 0.02)
    q13, s13 = orc.quantize_weight_fp8(w13)
    q2, s2 = orc.quantize_weight_fp8(w2)
    out, (lg, w, ids) = pkg.moe_block_fp8(to_bf16(x, dev).reshape(2, 24, H), to_bf16(wr, dev), k, to_f8(q13, dev),
                                          to_dev(s13, dev), to_f8(q2, dev), to_dev(s2, dev), return_routing=True)
    assert out.shape == (2, 24, H)
    ids_ref, _, _ = orc.topk_from_logits(np_f32(lg), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    ref = orc.experts_fp8(x, ids.cpu().numpy(), np_f32(w), q13, s13, q2, s2)
    max_abs, mean_rel = errors(np_f32(out).reshape(T, H), ref)
    assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL


@pytest.fixture(scope="module")
def router30b(dev):
    g = torch.Generator(device=dev).manual_seed(7)
    return (torch.randn((128, 2048), generator=g, device=dev) * 0.02).to(torch.bfloat16)


@pytest.mark.parametrize("T", [1, 3, 4, 5, 8, 16, 17, 64, 600])
def test_block_30b_routing_paths(pkg, dev, w30b, router30b, T):
    """Block forward across the routing variants: routing inside the gate_up GEMM (T <= 4),
    top-k + sort fused in one workgroup (T <= 16), separate top-k then single-workgroup sort (T*k <= 4096), and the
    multi-block sort."""
    rng = np.random.default_rng(30 + T)
    x = orc.gen_normal_bf16(rng, (T, 2048))
    out, (lg, w, ids) = pkg.moe_block_fp8(to_bf16(x, dev), router30b, 8, *w30b, return_routing=True)
    lg_n = np_f32(lg)
    lg_ref = orc.router_logits(x, np_f32(router30b))
    abs_sum = np.abs(x.astype(np.float64)) @ np.abs(np_f32(router30b).astype(np.float64)).T
    ulp_ref = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(lg_ref), 1e-30))) - 7)
    assert np.all(np.abs(lg_n - lg_ref) <= ulp_ref + 1e-5 * abs_sum)
    ids_ref, w_ref, _ = orc.topk_from_logits(lg_n, 8)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    assert bf16_ulp_diff(np_f32(w), w_ref).max() <= 1
    sub = np.sort(rng.choice(T, min(T, 48), replace=False))
    q13, s13, q2, s2 = w30b
    ref = orc.experts_fp8(x[sub], ids_ref[sub], w_ref[sub], f8_codes(q13), s13.cpu().numpy(), f8_codes(q2),
                          s2.cpu().numpy(), acc=np.float32)
    max_abs, mean_rel = errors(np_f32(out)[sub], ref)
    assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL


@pytest.mark.parametrize("T", [40, 600])  # 16-row decode tiles; 128-row prefill tiles
def test_sentinel_pairs_contribute_zero(pkg, dev, w30b, T):
    """Expert-parallel sentinels (ids outside [0, E), moe.py:405-419) add nothing: the output
    equals, bit for bit, the same routing with those slots' weights set to zero (every pair
    row is computed independently of the other rows of its tile)."""
    rng = np.random.default_rng(15 + T)
    x = orc.gen_normal_bf16(rng, (T, 2048))
    ids, w = orc.uniform_routing(rng, T, 128, 8)
    ids_s = ids.astype(np.int64).copy()
    ids_s[:, 7] = 128  # every token's last slot routed off-device
    ids_s[::3, 2] = -1  # and a third of the tokens' third slot
    out = pkg.experts_fp8(to_bf16(x, dev), to_dev(ids_s, dev), to_bf16(w, dev), *w30b)
    w0 = w.copy()
    w0[:, 7] = 0.0
    w0[::3, 2] = 0.0
    ref = pkg.experts_fp8(to_bf16(x, dev), to_dev(ids.copy(), dev), to_bf16(w0, dev), *w30b)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 8, 64, 600, 1024])
def test_block_fused_quant_is_bit_exact(pkg, dev, w30b, router30b, T):
    """The block path quantises x inside the router GEMM; the experts path quantises it in
    its own kernel.  Fed the block's routing, the experts path must reproduce the block's
    output bit for bit (same e4m3 codes and scales, same deterministic GEMMs).  Up to 4 tokens
    the block's gate_up routes its own one-row slots with no sort; the experts path sorts."""
    rng = np.random.default_rng(70 + T)
    x = to_bf16(orc.gen_normal_bf16(rng, (T, 2048)), dev)
    out, (_, w, ids) = pkg.moe_block_fp8(x, router30b, 8, *w30b, return_routing=True)
    ref = pkg.experts_fp8(x, ids, w, *w30b)
    assert torch.equal(out, ref)


# (T, H, I, E, k) chosen so that each GEMM tiling of the block runs (tile rows from S = T k:
# 16 while S <= 8 E, 32 while S <= 16 E, then 128 when H % 256 == 0 and H, I >= 512, else 64),
# with expert counts that are not powers of two, odd token counts and k = E.
SHAPE_SWEEP = [
    (5, 256, 128, 8, 2),       # 16-row tiles, 10 pairs
    (20, 512, 1024, 16, 4),    # 16-row tiles, 4 K blocks per down wave (the unrolled K loop)
    (12, 256, 768, 32, 8),     # 16-row tiles, 3 K blocks per down wave, 8 pairs per token
    (9, 256, 128, 64, 32),     # the largest top-k
    (50, 256, 128, 256, 8),    # the largest expert count
    (1, 768, 256, 3, 3),       # k = E, one token
    (2, 256, 128, 3, 3),       # 6 pairs on 3 experts: expert buckets (the routed path needs S <= E)
    (2, 256, 128, 8, 3),       # routed one-row slots, two of them may name one expert
    (4, 256, 128, 3, 3),       # 4 tokens on 3 experts: expert buckets
    (2, 1536, 256, 16, 4),     # routed one-row slots, gate_up with 3 K blocks per wave unrolled
    (30, 512, 256, 10, 4),     # 32-row tiles
    (40, 384, 256, 6, 3),      # 64-row tiles (H % 256 != 0)
    (77, 1024, 384, 20, 5),    # 64-row tiles (I < 512)
    (300, 512, 512, 16, 4),    # 128-row prefill tiles, 4 K blocks per GEMM
    (257, 1024, 640, 12, 6),   # 128-row prefill tiles, 5 K blocks in the down GEMM
    (24, 256, 4096, 2, 1),     # the largest intermediate size: 32 K blocks in the down GEMM
    (600, 512, 4096, 4, 2),    # the same on the 128-row prefill tiles
    (2, 256, 1536, 16, 4),     # routed one-row slots, h quantised in gate_up's hand-off (I > 1024)
    (6, 256, 1536, 32, 4),     # expert buckets, S <= 2 E: h quantised in gate_up's hand-off
    (2, 256, 2048, 16, 4),     # the same two at I = 2048
    (6, 256, 2048, 32, 4),
    (3, 256, 1024, 16, 4),     # the down GEMM quantises h itself with 4 K blocks per wave (NKW = 4)
    (10, 256, 384, 16, 4),     # 16-row tiles, h quantised by the down GEMM, no K split: 3 K blocks
    (10, 256, 512, 16, 4),     # the same with 4 K blocks
    (4, 4096, 768, 8, 2),      # the same with 6 K blocks and exact accumulation (routed slots)
    (5, 4096, 256, 8, 2),      # H > 2048: exact bf16 MFMAs on widened e4m3, 16-row tiles
    (30, 4096, 256, 10, 4),    # exact, 32-row tiles
    (60, 4096, 256, 10, 4),    # exact, 64-row tiles
    (300, 4096, 512, 8, 4),    # exact, 128-row prefill tiles
]


@pytest.mark.parametrize("T,H,I,E,k", SHAPE_SWEEP)
def test_block_shape_sweep(pkg, dev, T, H, I, E, k):
    """Block output within the layer tolerance of the oracle on its own routing; routing
    bit-exact given the kernel's logits; the experts path fed that routing reproduces the
    block bit for bit."""
    rng = np.random.default_rng(1000 + T + H + E)
    x = orc.gen_normal_bf16(rng, (T, H))
    wr = orc.gen_normal_bf16(rng, (E, H), 0.02)
    w13 = orc.gen_normal_bf16(rng, (E, 2 * I, H), 0.02)
    w2 = orc.gen_normal_bf16(rng, (E, H, I), 0.02)
    q13, s13 = orc.quantize_weight_fp8(w13)
    q2, s2 = orc.quantize_weight_fp8(w2)
    dq13, ds13, dq2, ds2 = to_f8(q13, dev), to_dev(s13, dev), to_f8(q2, dev), to_dev(s2, dev)
    xd = to_bf16(x, dev)
    out, (lg, w, ids) = pkg.moe_block_fp8(xd, to_bf16(wr, dev), k, dq13, ds13, dq2, ds2, return_routing=True)
    ids_ref, w_ref, _ = orc.topk_from_logits(np_f32(lg), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    assert bf16_ulp_diff(np_f32(w), w_ref).max() <= 1
    ref = orc.experts_fp8(x, ids.cpu().numpy(), np_f32(w), q13, s13, q2, s2)
    max_abs, mean_rel = errors(np_f32(out), ref)
    assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL, (max_abs, mean_rel)
    again = pkg.experts_fp8(xd, ids, w, dq13, ds13, dq2, ds2)
    assert torch.equal(out, again)
