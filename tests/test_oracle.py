"""Pins the CPU oracle (CPU only).

Every oracle function is checked against something independent of its own formula:
the OCP e4m3 value table and brute-force nearest-even search, torch's dtype casts as
library routines, closed forms, token-major brute force, and golden vectors that
transformers' Qwen3-MoE block wrote on CPU (tests/golden/make_golden.py).
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden  # noqa: E402


# ---------------------------------------------------------------------------
# number formats
# ---------------------------------------------------------------------------


def test_e4m3_table_known_codes():
    t = orc.e4m3_table()
    assert t[0x00] == 0.0 and t[0x80] == 0.0 and np.signbit(t[0x80])
    assert t[0x01] == 2.0 ** -9            # smallest subnormal
    assert t[0x07] == 7 * 2.0 ** -9        # largest subnormal
    assert t[0x08] == 2.0 ** -6            # smallest normal
    assert t[0x38] == 1.0
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert np.all(np.diff(t[:0x7F]) > 0)   # positive codes are ordered by value
    np.testing.assert_array_equal(t[0x80:0xFF], -t[0x00:0x7F])


def _brute_force_e4m3(v):
    """Nearest table value, ties to the even code (the code's mantissa LSB is 0)."""
    t = orc.e4m3_table()[:0x7F].astype(np.float64)
    out = np.empty(v.shape, np.uint8)
    for i, x in enumerate(v.astype(np.float64)):
        a = abs(x)
        d = np.abs(t - a)
        best = np.flatnonzero(d == d.min())
        code = best[0] if len(best) == 1 else [c for c in best if c % 2 == 0][0]
        out[i] = code | (0x80 if np.signbit(x) else 0)
    return out


def test_e4m3_encode_matches_brute_force_on_ties_and_neighbours():
    t = orc.e4m3_table()[:0x7F].astype(np.float32)
    mids = ((t[:-1].astype(np.float64) + t[1:]) / 2).astype(np.float32)  # exact in fp32
    vals = np.concatenate([t, mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1000)),
                           np.random.default_rng(0).uniform(0, 448, 3000).astype(np.float32),
                           np.random.default_rng(1).uniform(0, 2 ** -5, 2000).astype(np.float32)])
    vals = np.concatenate([vals, -vals])
    np.testing.assert_array_equal(orc.e4m3_encode(vals), _brute_force_e4m3(vals))


def test_e4m3_encode_matches_torch_cast():
    rng = np.random.default_rng(2)
    v = np.concatenate([rng.standard_normal(200000).astype(np.float32) * 60,
                        rng.standard_normal(200000).astype(np.float32) * 1e-3])
    v = np.clip(v, -448, 448).astype(np.float32)
    ref = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(orc.e4m3_encode(v), ref)
    np.testing.assert_array_equal(orc.e4m3_decode(ref), torch.from_numpy(ref).view(torch.float8_e4m3fn).float())


def test_round_bf16_matches_torch_cast():
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.standard_normal(300000).astype(np.float32) * 1e3,
                        rng.standard_normal(1000).astype(np.float32) * 1e-38,
                        np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38], np.float32)])
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(orc.round_bf16(v), ref)
    assert np.isnan(orc.round_bf16(np.array([np.nan], np.float32)))[0]


# ---------------------------------------------------------------------------
# quantisers
# ---------------------------------------------------------------------------


def test_quantize_act_invariants():
    rng = np.random.default_rng(4)
    x = orc.gen_normal_bf16(rng, (12, 512))
    x[1, 128:256] = 0.0
    x[2] *= np.float32(1e-4)
    q, s = orc.quantize_act_fp8(x)
    assert q.dtype == np.uint8 and s.shape == (12, 4)
    assert s[1, 1] == 1.0 and np.all(q[1, 128:256] == 0)
    g = np.abs(x).reshape(12, 4, 128)
    # the group's absolute maximum maps onto +-448 exactly
    amax_pos = g.argmax(-1)
    codes = q.reshape(12, 4, 128)
    for r in range(12):
        for j in range(4):
            if g[r, j].max() > 0:
                assert codes[r, j, amax_pos[r, j]] & 0x7F == 0x7E
                assert s[r, j] == np.float32(g[r, j].max() / np.float32(448.0))
    # error bound: half an e4m3 ulp (2^-4 relative for normals, 2^-10 * s for subnormals)
    d = orc.dequantize_act_fp8(q, s)
    bound = np.maximum(np.abs(x) * 2.0 ** -4, np.repeat(s, 128, axis=1) * 2.0 ** -10) * (1 + 1e-6)
    assert np.all(np.abs(d - x) <= bound)
    # sign and position are preserved (catches a transposed or mis-strided quantiser)
    assert np.all(np.sign(d[np.abs(x) > np.repeat(s, 128, axis=1) * 2.0 ** -9]) ==
                  np.sign(x[np.abs(x) > np.repeat(s, 128, axis=1) * 2.0 ** -9]))


def test_quantize_weight_invariants():
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((2, 256, 384), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    w[0, :128, 128:256] = 0.0
    q, inv = orc.quantize_weight_fp8(w)
    assert inv.shape == (2, 2, 3)
    assert inv[0, 0, 1] == 1.0 and np.all(q[0, :128, 128:256] == 0)
    t = np.abs(w).reshape(2, 2, 128, 3, 128).max(axis=(2, 4))
    nz = t > 0
    # stored inverse scale is 1/(448/amax): within one fp32 ulp of amax/448
    np.testing.assert_allclose(inv[nz], t[nz] / 448.0, rtol=2.5e-7)
    d = orc.dequantize_weight_fp8(q, inv)
    inv_full = np.repeat(np.repeat(inv, 128, axis=1), 128, axis=2)
    bound = np.maximum(np.abs(w) * 2.0 ** -4, inv_full * 2.0 ** -10) * (1 + 1e-5)
    assert np.all(np.abs(d - w) <= bound)


# ---------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------


def test_topk_brute_force_with_ties():
    rng = np.random.default_rng(6)
    T, E, k = 64, 32, 6
    lg = orc.round_bf16(rng.integers(-3, 4, size=(T, E)).astype(np.float32) * np.float32(0.25))  # many ties
    lg[0] = 0.0
    lg[1, 5] = -0.0
    ids, w, p = orc.topk_from_logits(lg, k, True)
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-float(lg[t, e]), e))
        assert list(ids[t]) == order[:k]
    np.testing.assert_allclose(p.sum(1), 1.0, rtol=1e-6)
    np.testing.assert_allclose(w.astype(np.float64).sum(1), 1.0, atol=k * 2.0 ** -8)
    assert list(ids[0]) == list(range(k))


def test_router_logits_brute_force():
    rng = np.random.default_rng(7)
    x = orc.gen_normal_bf16(rng, (5, 64))
    wr = orc.gen_normal_bf16(rng, (8, 64), 0.02)
    lg = orc.router_logits(x, wr)
    for t in range(5):
        for e in range(8):
            exact = sum(float(x[t, i]) * float(wr[e, i]) for i in range(64))
            assert lg[t, e] == orc.round_bf16(np.float32(exact))


# ---------------------------------------------------------------------------
# sort / align
# ---------------------------------------------------------------------------


def test_align_brute_force():
    rng = np.random.default_rng(8)
    T, k, E = 37, 3, 9
    ids = rng.integers(0, E, size=(T, k))
    perm, counts, offsets = orc.align(ids, E)
    flat = ids.reshape(-1)
    expect = [i for e in range(E) for i in range(T * k) if flat[i] == e]
    assert list(perm) == expect
    assert list(counts) == [int((flat == e).sum()) for e in range(E)]
    assert offsets[0] == 0 and offsets[-1] == T * k
    assert all(offsets[e + 1] - offsets[e] == counts[e] for e in range(E))
    tl = orc.tile_list(counts, 4)
    assert tl[:, 2].sum() == T * k and np.all(tl[:, 2] <= 4)


@pytest.mark.parametrize("block_m", [1, 4, 16, 128])
def test_tile_list_brute_force(block_m):
    """tile_list against a sequential scan of the sorted expert column: a new tile starts where the
    expert changes or the current tile is full.  Pins every tile's expert, start row and length."""
    rng = np.random.default_rng(9 + block_m)
    for T, k, E in ((37, 3, 9), (300, 8, 16), (5, 2, 40), (0, 4, 3)):
        ids = rng.integers(0, E, size=(T, k))
        if T > 10:
            ids[: T // 2, 0] = 2  # a hot expert: several full tiles then a remainder
        _, counts, _ = orc.align(ids, E)
        sorted_e = np.sort(ids.reshape(-1), kind="stable")
        expect = []
        for row, e in enumerate(sorted_e):
            if expect and expect[-1][0] == e and expect[-1][2] < block_m:
                expect[-1][2] += 1
            else:
                expect.append([int(e), row, 1])
        got = orc.tile_list(counts, block_m)
        assert got.shape == (len(expect), 3)
        np.testing.assert_array_equal(got, np.array(expect, dtype=np.int32).reshape(-1, 3))


# ---------------------------------------------------------------------------
# experts
# ---------------------------------------------------------------------------


def _token_major_fp8(x, ids, w, q13, s13, q2, s2):
    """Per token and slot, no sort: the same chain written the other way round."""
    T, H = x.shape
    k = ids.shape[1]
    I = q13.shape[1] // 2
    out = np.zeros((T, H), np.float32)
    for t in range(T):
        xq, sx = orc.quantize_act_fp8(x[t:t + 1])
        a = orc.dequantize_act_fp8(xq, sx)[0].astype(np.float64)
        acc = np.float32(0.0) * np.zeros(H, np.float32)
        for j in range(k):
            e = int(ids[t, j])
            wd = orc.dequantize_weight_fp8(q13[e], s13[e]).astype(np.float64)
            y = orc.round_bf16((wd @ a).astype(np.float32))
            h = orc.silu_mul_bf16(y[:I], y[I:])
            hq, sh = orc.quantize_act_fp8(h[None])
            hd = orc.dequantize_act_fp8(hq, sh)[0].astype(np.float64)
            w2d = orc.dequantize_weight_fp8(q2[e], s2[e]).astype(np.float64)
            z = orc.round_bf16((w2d @ hd).astype(np.float32))
            acc = (acc + orc.round_bf16(z * np.float32(w[t, j]))).astype(np.float32)
        out[t] = orc.round_bf16(acc)
    return out


def test_experts_fp8_matches_token_major_brute_force():
    rng = np.random.default_rng(9)
    T, H, I, E, k = 11, 256, 128, 6, 3
    x = orc.gen_normal_bf16(rng, (T, H))
    q13, s13 = orc.quantize_weight_fp8(orc.gen_normal_bf16(rng, (E, 2 * I, H), 0.02))
    q2, s2 = orc.quantize_weight_fp8(orc.gen_normal_bf16(rng, (E, H, I), 0.02))
    ids, w = orc.uniform_routing(rng, T, E, k)
    got = orc.experts_fp8(x, ids, w, q13, s13, q2, s2)
    np.testing.assert_array_equal(got, _token_major_fp8(x, ids, w, q13, s13, q2, s2))


def test_experts_fp8_closed_form_gate_then_up():
    """Gate = 2*Id, up = Id, down = Id on one expert: out = w * q(silu(2 q(x)) * q(x))."""
    H = I = 128
    x = orc.round_bf16(np.linspace(-2, 2, H, dtype=np.float32))[None]
    eye = np.eye(H, dtype=np.float32)
    q13, s13 = orc.quantize_weight_fp8(np.concatenate([2 * eye, eye])[None])
    q2, s2 = orc.quantize_weight_fp8(eye[None])
    ids = np.zeros((1, 1), np.int32)
    wt = orc.round_bf16(np.array([[0.75]], np.float32))
    out = orc.experts_fp8(x, ids, wt, q13, s13, q2, s2)[0]
    xd = orc.dequantize_act_fp8(*orc.quantize_act_fp8(x))[0]
    g, u = orc.round_bf16(2 * xd), orc.round_bf16(xd)
    h = orc.round_bf16(orc.round_bf16(g / (1 + np.exp(-g.astype(np.float64))).astype(np.float32)) * u)
    hd = orc.dequantize_act_fp8(*orc.quantize_act_fp8(h[None]))[0]
    np.testing.assert_array_equal(out, orc.round_bf16(orc.round_bf16(hd) * np.float32(0.75)))
    swapped = orc.round_bf16(orc.round_bf16(u / (1 + np.exp(-u.astype(np.float64))).astype(np.float32)) * g)
    assert not np.allclose(h, swapped)


def test_silu_closed_form():
    g = np.array([0.0, 20.0, -20.0, 1.0], np.float32)
    h = orc.silu_mul_bf16(g, np.ones(4, np.float32))
    assert h[0] == 0.0 and h[1] == 20.0 and abs(h[2]) < 1e-7
    assert h[3] == orc.round_bf16(np.float32(1 / (1 + np.exp(-1.0))))


# ---------------------------------------------------------------------------
# golden vectors from transformers' Qwen3MoeSparseMoeBlock on CPU
# ---------------------------------------------------------------------------


def _has_ties_near_boundary(row, k):
    s = np.sort(row)[::-1]
    return np.any(s[: k + 1][1:] == s[: k + 1][:-1])


@pytest.mark.parametrize("case", list(make_golden.CASES))
def test_golden_reference_block(case):
    cfg = make_golden.CASES[case]
    g = np.load(os.path.join(GOLDEN, f"{case}.npz"))
    x, wr, w13, w2 = make_golden.make_inputs(**cfg)
    assert [make_golden.digest(a) for a in (x, wr, w13, w2)] == list(g["digests"]), "input generator drifted"
    T, E, k, H = cfg["T"], cfg["E"], cfg["k"], cfg["H"]
    lg_ref = orc.from_bf16_bits(g["logits_bf16"]).reshape(T, E)
    # router logits: fp32-accumulated bf16 linear, bit-exact on these inputs
    np.testing.assert_array_equal(orc.router_logits(x, wr), lg_ref)
    ids, w, _ = orc.topk_from_logits(lg_ref, k)
    gi = g["indices"]
    gw = orc.from_bf16_bits(g["scores_bf16"]).reshape(T, k)
    # same expert sets everywhere except where an exact tie straddles the k-th place
    for t in range(T):
        if not _has_ties_near_boundary(lg_ref[t], k):
            assert set(ids[t]) == set(gi[t])
        if not _has_ties_near_boundary(lg_ref[t], k - 1) and np.all(np.diff(np.sort(lg_ref[t])[::-1][:k + 1]) != 0):
            np.testing.assert_array_equal(ids[t], gi[t])
            np.testing.assert_array_equal(w[t], gw[t])
    # experts: the reference's own routing fed to the oracle's bf16 grouped chain
    out_ref = orc.from_bf16_bits(g["out_bf16"]).reshape(T, H)
    out = orc.experts_bf16(x, gi, gw, w13, w2)
    d = np.abs(out - out_ref)
    assert (d == 0).mean() >= 0.99
    assert d.max() <= 2.0 ** -8 * max(float(np.abs(out_ref).max()), 1e-3) * 2
