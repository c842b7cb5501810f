"""Pins the attention oracle (oracle/attn_oracle.py) without a GPU: golden vectors that
transformers' decoder-layer functions wrote on CPU (tests/golden/make_golden_attn.py), a
pure-Python brute force on tiny shapes, and closed forms."""

from __future__ import annotations

import math
import os
import sys

import numpy as np
import pytest

from oracle import attn_oracle as att
from oracle import moe_oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden_attn as mga  # noqa: E402

SCALE = 128 ** -0.5


def ulps(a, b):
    def ordered(x):
        bits = orc.bf16_bits(x).astype(np.int32)
        return np.where(bits & 0x8000, -(bits & 0x7FFF), bits)
    return np.abs(ordered(a) - ordered(b))


@pytest.mark.parametrize("case", list(mga.CASES))
def test_golden_decoder_pieces(case):
    cfg = mga.CASES[case]
    g = np.load(os.path.join(GOLDEN, f"{case}.npz"))
    q, k, v, x, w = mga.make_inputs(**cfg)
    assert [mga.digest(a) for a in (q, k, v, x, w)] == list(g["digests"]), "input generator drifted"
    gold = {n: orc.from_bf16_bits(g[n]) for n in g.files if n.endswith("_bf16")}

    # RMSNorm: fp32 variance, rsqrt, bf16 casts
    d = ulps(att.rms_norm(x, w, eps=mga.EPS), gold["rmsnorm_bf16"])
    assert d.max() <= 1 and (d == 0).mean() >= 0.99

    # rotary cos / sin and their application to q (position L-1) and every k
    L = cfg["L"]
    inv = g["inv_freq"]
    # numpy and torch evaluate the fp32 pow and divide with different libm code: <= 2 ulps apart
    assert np.abs(att.default_inv_freq(mga.HEAD_DIM, mga.THETA).view(np.int32) - inv.view(np.int32)).max() <= 2
    cos, sin = att.rope_cos_sin(np.arange(L), mga.HEAD_DIM, mga.THETA, inv_freq=inv)
    assert ulps(cos, gold["cos_bf16"]).max() <= 1 and ulps(sin, gold["sin_bf16"]).max() <= 1
    # with the reference's own cos / sin the application is bit-exact
    q_rot = att.rotary(q[None], gold["cos_bf16"][L - 1:], gold["sin_bf16"][L - 1:])[0]
    assert np.array_equal(orc.bf16_bits(q_rot), g["q_rot_bf16"])
    k_rot = att.rotary(k, gold["cos_bf16"], gold["sin_bf16"])
    assert np.array_equal(orc.bf16_bits(k_rot), g["k_rot_bf16"])

    # eager attention of the new token over the whole context
    out = att.decode_attention(gold["q_rot_bf16"], gold["k_rot_bf16"], v, SCALE)
    d = ulps(out, gold["attn_bf16"])
    assert d.max() <= 2 and (d == 0).mean() >= 0.95, (d.max(), (d == 0).mean())


def _rb(x) -> float:
    return float(orc.round_bf16(np.float32(x)).reshape(-1)[0])


def brute_attention(q, keys, values, scale):
    """Scalar loops, one rounding per reference op."""
    Hq, dh = q.shape
    L, Hkv, _ = keys.shape
    G = Hq // Hkv
    out = np.zeros((Hq, dh), np.float32)
    for h in range(Hq):
        g = h // G
        s = []
        for t in range(L):
            dot = math.fsum(float(q[h, i]) * float(keys[t, g, i]) for i in range(dh))
            s.append(_rb(np.float32(_rb(dot)) * np.float32(scale)))
        m = max(s)
        e = [np.float32(math.exp(x - m)) for x in s]
        tot = np.float32(sum(np.float64(x) for x in e))
        p = [_rb(x / tot) for x in e]
        for i in range(dh):
            out[h, i] = _rb(math.fsum(p[t] * float(values[t, g, i]) for t in range(L)))
    return out


def test_brute_force_tiny():
    rng = np.random.default_rng(3)
    for Hq, Hkv, L, dh in [(2, 1, 5, 4), (4, 2, 9, 8), (3, 3, 1, 4)]:
        q = orc.round_bf16(rng.standard_normal((Hq, dh)).astype(np.float32))
        k = orc.round_bf16(rng.standard_normal((L, Hkv, dh)).astype(np.float32))
        v = orc.round_bf16(rng.standard_normal((L, Hkv, dh)).astype(np.float32))
        a = att.decode_attention(q, k, v, 0.5)
        b = brute_attention(q, k, v, 0.5)
        assert ulps(a, b).max() <= 1


def test_identical_keys_average_values():
    # equal scores -> p = 1/L exactly for L a power of two -> mean of V, one bf16 rounding
    rng = np.random.default_rng(4)
    L, dh = 16, 128
    q = orc.round_bf16(rng.standard_normal((2, dh)).astype(np.float32))
    krow = orc.round_bf16(rng.standard_normal(dh).astype(np.float32))
    k = np.broadcast_to(krow, (L, 1, dh)).copy()
    v = orc.round_bf16(rng.standard_normal((L, 1, dh)).astype(np.float32))
    out = att.decode_attention(q, k, v, SCALE)
    assert np.array_equal(out, orc.round_bf16(v[:, 0, :].astype(np.float64).mean(0).astype(np.float32))[None].repeat(2, 0))


def test_dominant_key_selects_its_value():
    dh, L = 128, 40
    q = np.zeros((1, dh), np.float32)
    q[0, 0] = 8.0
    k = np.zeros((L, 1, dh), np.float32)
    k[17, 0, 0] = 64.0  # score 64*8/sqrt(128) ~ 45 above the rest: exp(-45) ~ 3e-20
    v = orc.round_bf16(np.random.default_rng(5).standard_normal((L, 1, dh)).astype(np.float32))
    out = att.decode_attention(q, k, v, SCALE)
    assert np.array_equal(out[0], v[17, 0])


def test_kv_head_mapping():
    # kv head g holds constant value rows g+1: query head h must return h // G + 1 everywhere
    Hq, Hkv, L, dh = 8, 4, 20, 128
    rng = np.random.default_rng(6)
    q = orc.round_bf16(rng.standard_normal((Hq, dh)).astype(np.float32))
    k = orc.round_bf16(rng.standard_normal((L, Hkv, dh)).astype(np.float32))
    v = np.zeros((L, Hkv, dh), np.float32)
    for g in range(Hkv):
        v[:, g, :] = g + 1
    out = att.decode_attention(q, k, v, SCALE)
    for h in range(Hq):
        # sum of bf16 probabilities times a constant: within a few bf16 ulps of the constant
        assert np.allclose(out[h], h // (Hq // Hkv) + 1, rtol=2 ** -6)


def test_paged_round_trip():
    rng = np.random.default_rng(7)
    L, Hkv, dh = 53, 2, 128
    k = rng.standard_normal((L, Hkv, dh)).astype(np.float32)
    v = rng.standard_normal((L, Hkv, dh)).astype(np.float32)
    pages = [5, 0, 9, 2]
    kc, vc = att.scatter_paged(k, v, pages)
    k2, v2 = att.gather_paged(kc, vc, np.array(pages + [0, 0]), L)
    assert np.array_equal(k, k2) and np.array_equal(v, v2)


def test_rope_position_zero_is_identity_and_preserves_norms():
    cos, sin = att.rope_cos_sin(np.array([0, 1000]), 128, 1e6)
    x = orc.round_bf16(np.random.default_rng(8).standard_normal((2, 3, 128)).astype(np.float32))
    y = att.rotary(x, cos, sin)
    assert np.array_equal(y[0], x[0])
    n0 = np.hypot(x[1, :, :64], x[1, :, 64:])
    n1 = np.hypot(y[1, :, :64], y[1, :, 64:])
    assert np.allclose(n0, n1, rtol=2e-2, atol=1e-2)


def test_product_inv_freq_is_the_references():
    """The decode path's inv_freq (computed like transformers' rotary embedding) equals the
    reference's golden inv_freq bit for bit."""
    import torch

    import __graft_entry__

    dec = __graft_entry__.load_package().decode
    g = np.load(os.path.join(GOLDEN, "attn_g8_l300.npz"))
    got = dec.default_inv_freq(dec.DecoderConfig(), torch.device("cpu")).numpy()
    assert np.array_equal(got, g["inv_freq"])
