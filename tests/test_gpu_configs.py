"""Every BASELINE configuration at its own workload, on the GPU, against the oracle and the
reference's golden vectors.

* C1: the Qwen3-30B-A3B layer at 16 tokens, seed 0: the HIP router against the logits and
  top-k ids that transformers' ``Qwen3MoeSparseMoeBlock`` wrote on CPU
  (tests/golden/make_golden.py), and the FP8 block on the same inputs against the oracle.
* C2: decode batches including 128 and 129 tokens, the 8 E pair count where the expert GEMMs
  switch from 16-row streaming tiles to the 128-row LDS-tiled kernel, and 256 tokens
  (tests/test_gpu_parity.py covers 1, 8, 32, 64, 256).
* C3: the 4096-token Zipf-skewed prefill chunk, checked on a tile-stratified token sample: the
  first, the last and a random row of every M tile of the expert GEMMs (ragged remainders of the
  cold experts included) belong to a checked token.
* C4: the full 128-expert Qwen3-235B-A22B layer at decode 64 (every token) and prefill 2048
  (tile-stratified).

Layer outputs: max-abs <= 2e-2 and mean-relative <= 1e-2 against the dequantise-then-fp32
oracle on the kernel's own routing; routing bit-exact given the kernel's logits.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc
from tests.helpers import (TOL_MAX_ABS, TOL_MEAN_REL, bf16_ulp_diff, errors, f8_codes, gpu_weights, np_f32,
                           to_bf16, to_dev)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden  # noqa: E402

pytestmark = pytest.mark.gpu


def block_m_of(pkg, T, H, I, E, k):
    """Tile height the library picks for T tokens (low 16 bits of the numerics key)."""
    return int(pkg._lib.load().moe_mi355x_block_numerics_key(T, H, I, E, k, 1)) & 0xFFFF


def tile_stratified_tokens(ids, E, block_m, rng):
    """Tokens owning the first, the last and a random row of every block_m-row tile of the
    stable expert sort (oracle align + tile_list), so every tile the GEMMs run is checked."""
    k = ids.shape[1]
    perm, counts, _ = orc.align(ids, E)
    toks = set()
    tiles = orc.tile_list(counts, block_m)
    for _, r0, rows in tiles:
        for r in (r0, r0 + rows - 1, r0 + int(rng.integers(rows))):
            toks.add(int(perm[r]) // k)
    return np.array(sorted(toks)), len(tiles)


def check_experts(pkg, dev, x, ids, w, weights_dev, weights_np, sub=None):
    """Layer output against the oracle at the absolute bar: max-abs <= 2e-2, mean-rel <= 1e-2."""
    out = pkg.experts_fp8(to_bf16(x, dev), to_dev(ids, dev), to_bf16(w, dev), *weights_dev)
    o = np_f32(out)
    sel = slice(None) if sub is None else sub
    ref = orc.experts_fp8(x[sel], ids[sel], w[sel], *weights_np, acc=np.float32)
    max_abs, mean_rel = errors(o[sel], ref)
    bar = TOL_MAX_ABS
    print(f"max_abs {max_abs:.4g} (bar {bar:.4g}), mean_rel {mean_rel:.3g}, |ref| max {np.abs(ref).max():.3g}")
    assert max_abs <= bar and mean_rel <= TOL_MEAN_REL, (max_abs, mean_rel)
    return out


def host_weights(wd):
    q13, s13, q2, s2 = wd
    return f8_codes(q13), s13.cpu().numpy(), f8_codes(q2), s2.cpu().numpy()


# ---------------------------------------------------------------------------
# C1: golden vectors of transformers' block (30B shape, 16 tokens, seed 0)
# ---------------------------------------------------------------------------


def _boundary_tie(row, k):
    """An exact tie between the k-th and the (k+1)-th largest logit: the expert set itself is
    then up to the reference's CPU topk, which orders ties arbitrarily."""
    s = np.sort(row)[::-1]
    return bool(s[k - 1] == s[k])


def test_c1_router_matches_transformers_golden(pkg, dev):
    cfg = make_golden.CASES["c1_30b_t16"]
    g = np.load(os.path.join(GOLDEN, "c1_30b_t16.npz"))
    x, wr, w13, w2 = make_golden.make_inputs(**cfg)
    assert [make_golden.digest(a) for a in (x, wr, w13, w2)] == list(g["digests"]), "input generator drifted"
    T, E, k = cfg["T"], cfg["E"], cfg["k"]
    lg, w, ids = pkg.route(to_bf16(x, dev), to_bf16(wr, dev), k)
    lg_gpu = np_f32(lg)
    lg_ref = orc.from_bf16_bits(g["logits_bf16"]).reshape(T, E)
    ulps = bf16_ulp_diff(lg_gpu, lg_ref)
    assert (ulps > 0).mean() <= 2e-3 and ulps.max() <= 1, (int((ulps > 0).sum()), int(ulps.max()))
    gi = g["indices"]
    gids = ids.cpu().numpy()
    checked = 0
    for t in range(T):
        if _boundary_tie(lg_ref[t], k):
            continue  # the reference's CPU topk orders exact ties arbitrarily
        assert set(gids[t]) == set(gi[t]), t
        checked += 1
    assert checked >= T - 2  # 6% of tokens of this data have a boundary tie
    # the expert order and weights where the whole top-k+1 has no tie
    gw = orc.from_bf16_bits(g["scores_bf16"]).reshape(T, k)
    for t in range(T):
        top = np.sort(lg_ref[t])[::-1][: k + 1]
        if np.all(np.diff(top) != 0):
            np.testing.assert_array_equal(gids[t], gi[t])
            assert bf16_ulp_diff(np_f32(w)[t], gw[t]).max() <= 1


def test_c1_fp8_block_matches_oracle(pkg, dev):
    cfg = make_golden.CASES["c1_30b_t16"]
    x, wr, w13, w2 = make_golden.make_inputs(**cfg)
    k = cfg["k"]
    q13, s13 = pkg.quantize_weight_fp8(to_bf16(w13, dev))
    q2, s2 = pkg.quantize_weight_fp8(to_bf16(w2, dev))
    del w13, w2
    out, (lg, w, ids) = pkg.moe_block_fp8(to_bf16(x, dev), to_bf16(wr, dev), k, q13, s13, q2, s2,
                                          return_routing=True)
    ids_ref, w_ref, _ = orc.topk_from_logits(np_f32(lg), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    assert bf16_ulp_diff(np_f32(w), w_ref).max() <= 1
    ref = orc.experts_fp8(x, ids_ref, w_ref, *host_weights((q13, s13, q2, s2)), acc=np.float32)
    max_abs, mean_rel = errors(np_f32(out), ref)
    assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL, (max_abs, mean_rel)


# ---------------------------------------------------------------------------
# C2 / C3: the 30B FP8 layer
# ---------------------------------------------------------------------------


@pytest.fixture(scope="module")
def w30b(dev):
    wd = gpu_weights(128, 2048, 768, dev, seed=0)
    return wd, host_weights(wd)


@pytest.mark.parametrize("T", [127, 128, 129, 256])
def test_c2_decode_tile_switch(pkg, dev, w30b, T):
    """Around S = 8 E = 1024 pairs: 16-row tiles up to 128 tokens, the 128-row LDS-tiled kernel
    from 129 (every token checked)."""
    assert block_m_of(pkg, T, 2048, 768, 128, 8) == (16 if T <= 128 else 128)
    rng = np.random.default_rng(200 + T)
    x = orc.gen_normal_bf16(rng, (T, 2048))
    ids, w = orc.uniform_routing(rng, T, 128, 8)
    check_experts(pkg, dev, x, ids, w, *w30b)


def test_c3_prefill_zipf_every_tile(pkg, dev, w30b):
    T, H, E, k = 4096, 2048, 128, 8
    rng = np.random.default_rng(11)
    x = orc.gen_normal_bf16(rng, (T, H))
    lg = orc.gen_normal_bf16(rng, (T, E)) + orc.zipf_bias(E, 1.1, beta=1.5)
    ids, w, _ = orc.topk_from_logits(orc.round_bf16(lg), k)
    counts = np.bincount(ids.reshape(-1), minlength=E)
    assert np.sort(counts)[::-1][:10].sum() / (T * k) > 0.4  # skewed: a few hot experts
    bm = block_m_of(pkg, T, H, 768, E, k)
    assert bm == 128
    sub, n_tiles = tile_stratified_tokens(ids, E, bm, rng)
    assert n_tiles > 200
    check_experts(pkg, dev, x, ids, w, *w30b, sub=sub)


# ---------------------------------------------------------------------------
# C4: the full 128-expert 235B layer
# ---------------------------------------------------------------------------


@pytest.fixture(scope="module")
def w235b(dev):
    wd = gpu_weights(128, 4096, 1536, dev, seed=3)
    return wd, host_weights(wd)


@pytest.mark.timeout(600)
def test_c4_235b_decode_64_all_tokens(pkg, dev, w235b):
    T = 64
    rng = np.random.default_rng(301)
    x = orc.gen_normal_bf16(rng, (T, 4096))
    ids, w = orc.uniform_routing(rng, T, 128, 8)
    assert block_m_of(pkg, T, 4096, 1536, 128, 8) == 16
    check_experts(pkg, dev, x, ids, w, *w235b)


@pytest.mark.timeout(600)
def test_c4_235b_prefill_2048_every_tile(pkg, dev, w235b):
    T = 2048
    rng = np.random.default_rng(302)
    x = orc.gen_normal_bf16(rng, (T, 4096))
    ids, w = orc.uniform_routing(rng, T, 128, 8)
    bm = block_m_of(pkg, T, 4096, 1536, 128, 8)
    assert bm == 128
    sub, n_tiles = tile_stratified_tokens(ids, 128, bm, rng)
    assert n_tiles >= 128
    check_experts(pkg, dev, x, ids, w, *w235b, sub=sub)


@pytest.mark.timeout(600)
def test_c4_235b_block_with_router(pkg, dev, w235b):
    """The whole block (router + experts) at the 235B shape, decode 64."""
    T, H, E, k = 64, 4096, 128, 8
    g = torch.Generator(device=dev).manual_seed(5)
    wr = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    rng = np.random.default_rng(303)
    x = orc.gen_normal_bf16(rng, (T, H))
    wd, wn = w235b
    out, (lg, w, ids) = pkg.moe_block_fp8(to_bf16(x, dev), wr, k, *wd, return_routing=True)
    ids_ref, w_ref, _ = orc.topk_from_logits(np_f32(lg), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    ref = orc.experts_fp8(x, ids_ref, w_ref, *wn, acc=np.float32)
    max_abs, mean_rel = errors(np_f32(out), ref)
    print(f"max_abs {max_abs:.4g}, mean_rel {mean_rel:.3g}, |ref| max {np.abs(ref).max():.3g}")
    assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL, (max_abs, mean_rel)
