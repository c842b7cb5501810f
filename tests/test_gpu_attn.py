"""Paged decode attention and KV append on the GPU, through the C ABI, against the oracle
(oracle/attn_oracle.py, pinned in tests/test_oracle_attn.py).

Tolerance: the kernel applies unnormalised bf16 probabilities and divides once in fp32,
the reference rounds the normalised probabilities to bf16 first, so outputs agree to
bf16 rounding noise.  The bar is the layer tolerance of the MoE path: max-abs <= 2e-2 (one
bf16 ulp of an output of magnitude 2-4 is 1.6e-2) and mean relative error <= 1e-2."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attn_oracle as att
from oracle import moe_oracle as orc
from tests.helpers import errors, to_bf16

pytestmark = pytest.mark.gpu

PAGE, D = 16, 128
SCALE = D ** -0.5


def build_cache(rng, lens, Hkv, q_std=1.0, n_spare=3, poison=True):
    """Random keys / values per sequence scattered over shuffled pages; unused slots NaN."""
    n_pages = [(L + PAGE - 1) // PAGE for L in lens]
    total = sum(n_pages) + n_spare
    order = rng.permutation(total)
    kc = np.full((total, Hkv, PAGE, D), np.nan if poison else 0.0, np.float32)
    vc = np.full((total, Hkv, D, PAGE), np.nan if poison else 0.0, np.float32)
    max_pages = max(n_pages) + 2
    tables = np.zeros((len(lens), max_pages), np.int32)
    seqs = []
    used = 0
    for b, L in enumerate(lens):
        pages = order[used:used + n_pages[b]]
        used += n_pages[b]
        tables[b, :n_pages[b]] = pages
        k = orc.round_bf16(rng.standard_normal((L, Hkv, D)).astype(np.float32))
        v = orc.round_bf16(rng.standard_normal((L, Hkv, D)).astype(np.float32))
        for t in range(L):
            kc[pages[t // PAGE], :, t % PAGE, :] = k[t]
            vc[pages[t // PAGE], :, :, t % PAGE] = v[t]
        seqs.append((k, v))
    return kc, vc, tables, seqs


def run_case(pkg, dev, lens, Hq, Hkv, seed, q_std=1.0):
    rng = np.random.default_rng(seed)
    kc, vc, tables, seqs = build_cache(rng, lens, Hkv)
    q = orc.round_bf16((rng.standard_normal((len(lens), Hq, D)) * q_std).astype(np.float32))
    out = pkg.paged_attention_decode(to_bf16(q, dev), to_bf16(kc, dev), to_bf16(vc, dev),
                                     torch.from_numpy(tables).to(dev), torch.tensor(lens, dtype=torch.int32, device=dev),
                                     SCALE)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    # an empty context attends to nothing: the kernel writes zeros
    ref = np.stack([att.decode_attention(q[b], k, v, SCALE) if len(k) else np.zeros((Hq, D), np.float32)
                    for b, (k, v) in enumerate(seqs)])
    return got, ref


@pytest.mark.parametrize("lens,Hq,Hkv", [
    ([1, 2, 15, 16, 17, 33], 32, 4),          # one token, partial and exact pages
    ([300, 511, 512, 1000], 32, 4),           # the Qwen3-30B-A3B grouping, several splits
    ([4096, 8192], 32, 4),                    # BASELINE config 5's longest contexts
    ([77, 130], 8, 8),                        # no grouping
    ([200, 64], 16, 1),                       # 16 query heads on one kv head
])
def test_paged_attention_matches_oracle(pkg, dev, lens, Hq, Hkv):
    got, ref = run_case(pkg, dev, lens, Hq, Hkv, seed=sum(lens))
    max_abs, mean_rel = errors(got, ref)
    assert max_abs <= 2e-2 and mean_rel <= 1e-2, (max_abs, mean_rel)


def test_paged_attention_many_sequences(pkg, dev):
    """600 sequences: the item scan runs in three chunks of 256 (a totals pass, then the locating
    pass); full 64-page splits, partial last splits of every length and empty contexts, so every
    dispatch phase is populated."""
    rng = np.random.default_rng(600)
    lens = rng.integers(1, 1300, size=600)
    lens[rng.random(600) < 0.05] = 0
    lens[:63] = 16 * (64 + np.arange(1, 64)) - 5  # one full split, then a partial one of 1..63 pages
    lens = [int(x) for x in lens]
    got, ref = run_case(pkg, dev, lens, 32, 4, seed=600)
    assert (got[np.array(lens) == 0] == 0).all()
    max_abs, mean_rel = errors(got, ref)
    assert max_abs <= 2e-2 and mean_rel <= 1e-2, (max_abs, mean_rel)


def test_paged_attention_peaked_scores(pkg, dev):
    # large q: softmax concentrated on few keys (exercises the running max / rescale path)
    got, ref = run_case(pkg, dev, [700, 1500], 32, 4, seed=9, q_std=8.0)
    max_abs, mean_rel = errors(got, ref)
    assert max_abs <= 2e-2 and mean_rel <= 1e-2, (max_abs, mean_rel)


def test_paged_attention_deterministic(pkg, dev):
    rng = np.random.default_rng(10)
    lens = [900, 3000, 40]
    kc, vc, tables, _ = build_cache(rng, lens, 4, poison=False)
    q = to_bf16(rng.standard_normal((3, 32, D)).astype(np.float32), dev)
    args = (to_bf16(kc, dev), to_bf16(vc, dev), torch.from_numpy(tables).to(dev),
            torch.tensor(lens, dtype=torch.int32, device=dev), SCALE)
    a = pkg.paged_attention_decode(q, *args)
    b = pkg.paged_attention_decode(q, *args)
    assert torch.equal(a, b)


def test_kv_append_places_rows(pkg, dev):
    rng = np.random.default_rng(11)
    B, Hkv, n_pages = 3, 4, 7
    kc = torch.zeros((n_pages, Hkv, PAGE, D), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros((n_pages, Hkv, D, PAGE), dtype=torch.bfloat16, device=dev)
    tables = np.array([[3, 1, 0], [6, 2, 0], [5, 4, 0]], np.int32)
    pos = np.array([0, 17, 31], np.int32)
    k = orc.round_bf16(rng.standard_normal((B, Hkv, D)).astype(np.float32))
    v = orc.round_bf16(rng.standard_normal((B, Hkv, D)).astype(np.float32))
    pkg.kv_append(to_bf16(k, dev), to_bf16(v, dev), kc, vc, torch.from_numpy(tables).to(dev),
                  torch.from_numpy(pos).to(dev))
    torch.cuda.synchronize()
    kcn, vcn = kc.float().cpu().numpy(), vc.float().cpu().numpy()
    expect_k = np.zeros_like(kcn)
    expect_v = np.zeros_like(vcn)
    for b in range(B):
        pg, slot = tables[b, pos[b] // PAGE], pos[b] % PAGE
        expect_k[pg, :, slot, :] = k[b]
        expect_v[pg, :, :, slot] = v[b]
    assert np.array_equal(kcn, expect_k) and np.array_equal(vcn, expect_v)


def test_paged_attention_rejects_bad_shapes(pkg, dev):
    q = torch.zeros((2, 32, 64), dtype=torch.bfloat16, device=dev)
    kc = torch.zeros((4, 4, PAGE, 64), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros((4, 4, 64, PAGE), dtype=torch.bfloat16, device=dev)
    t = torch.zeros((2, 2), dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        pkg.paged_attention_decode(q, kc, vc, t, t[:, 0].contiguous(), 0.1)


def test_cache_writers_reject_mismatched_pools(pkg, dev):
    """A V pool that is not the K pool's [pages, Hkv, 128, 16] counterpart is refused before
    any kernel could write past it."""
    kc = torch.zeros((4, 2, PAGE, D), dtype=torch.bfloat16, device=dev)
    bad_v = [torch.zeros((2, 2, D, PAGE), dtype=torch.bfloat16, device=dev),   # fewer pages
             torch.zeros((4, 2, PAGE, D), dtype=torch.bfloat16, device=dev)]   # K's layout
    k = torch.zeros((1, 2, D), dtype=torch.bfloat16, device=dev)
    t = torch.zeros((1, 4), dtype=torch.int32, device=dev)
    pos = torch.zeros(1, dtype=torch.int32, device=dev)
    qkv = torch.zeros((1, 8 * D), dtype=torch.bfloat16, device=dev)
    nw = torch.ones(D, dtype=torch.bfloat16, device=dev)
    inv = torch.ones(D // 2, dtype=torch.float32, device=dev)
    for vc in bad_v:
        with pytest.raises(ValueError, match="v_cache"):
            pkg.kv_append(k, k, kc, vc, t, pos)
        with pytest.raises(ValueError, match="v_cache"):
            pkg.qk_norm_rope_append(qkv, nw, nw, inv, pos, 4, 2, 1e-6, kc, vc, t)


def test_paged_attention_out_of_table_contexts(pkg, dev):
    """Context lengths are device data the host cannot check: a length past the block table
    attends to the table's pages only, and an empty context gives zeros (never NaN, never a
    read beyond the table)."""
    rng = np.random.default_rng(12)
    lens = [40, 70]
    kc, vc, tables, seqs = build_cache(rng, lens, 4, poison=False)
    tables = tables[:, :3]  # room for 48 tokens: the second sequence overflows it
    q = orc.round_bf16(rng.standard_normal((3, 32, D)).astype(np.float32))
    tab3 = np.concatenate([tables, tables[:1]], 0)
    ctx = torch.tensor([40, 70, 0], dtype=torch.int32, device=dev)
    out = pkg.paged_attention_decode(to_bf16(q, dev), to_bf16(kc, dev), to_bf16(vc, dev),
                                     torch.from_numpy(np.ascontiguousarray(tab3)).to(dev), ctx, SCALE)
    got = out.float().cpu().numpy()
    k1, v1 = seqs[1]
    ref = np.stack([att.decode_attention(q[0], *seqs[0], SCALE), att.decode_attention(q[1], k1[:48], v1[:48], SCALE)])
    max_abs, mean_rel = errors(got[:2], ref)
    assert max_abs <= 2e-2 and mean_rel <= 1e-2, (max_abs, mean_rel)
    assert np.array_equal(got[2], np.zeros_like(got[2]))


def test_kv_append_skips_positions_outside_the_table(pkg, dev):
    rng = np.random.default_rng(13)
    B, Hkv, n_pages = 3, 4, 5
    kc = torch.zeros((n_pages, Hkv, PAGE, D), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros((n_pages, Hkv, D, PAGE), dtype=torch.bfloat16, device=dev)
    tables = np.array([[3, 1], [4, 2], [0, 1]], np.int32)
    pos = np.array([20, -1, 32], np.int32)  # only the first is inside its 2-page table
    k = orc.round_bf16(rng.standard_normal((B, Hkv, D)).astype(np.float32))
    v = orc.round_bf16(rng.standard_normal((B, Hkv, D)).astype(np.float32))
    pkg.kv_append(to_bf16(k, dev), to_bf16(v, dev), kc, vc, torch.from_numpy(tables).to(dev),
                  torch.from_numpy(pos).to(dev))
    torch.cuda.synchronize()
    kcn, vcn = kc.float().cpu().numpy(), vc.float().cpu().numpy()
    expect_k, expect_v = np.zeros_like(kcn), np.zeros_like(vcn)
    expect_k[1, :, 4, :] = k[0]
    expect_v[1, :, :, 4] = v[0]
    assert np.array_equal(kcn, expect_k) and np.array_equal(vcn, expect_v)


def test_paged_attention_skips_table_entries_outside_the_pools(pkg, dev):
    """A block-table entry outside [0, pages) (a -1 pad, a stale id) inside a context is an empty
    page: never read (its descriptor covers no bytes), its keys left out of the softmax.  The
    output equals the attention over the valid pages' keys; a context whose every page is
    invalid gives zeros, never NaN."""
    rng = np.random.default_rng(14)
    lens = [100, 700, 50]
    Hq, Hkv = 32, 4
    kc, vc, tables, seqs = build_cache(rng, lens, Hkv, poison=False)
    n_pool = kc.shape[0]
    tables = tables.copy()
    # sequence 0 (7 pages): pages 1 and 5 invalid, so wave 1 of the split sees only empty pages
    tables[0, 1] = -1
    tables[0, 5] = n_pool + 3
    # sequence 1 (44 pages, several splits): a run of invalid pages filling one whole split
    tables[1, 8:24] = -7
    tables[1, 30] = n_pool
    # sequence 2: every page invalid
    tables[2, :4] = -1
    q = orc.round_bf16(rng.standard_normal((3, Hq, D)).astype(np.float32))
    out = pkg.paged_attention_decode(to_bf16(q, dev), to_bf16(kc, dev), to_bf16(vc, dev),
                                     torch.from_numpy(tables).to(dev), torch.tensor(lens, dtype=torch.int32, device=dev),
                                     SCALE)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    refs = []
    for b in range(2):
        k, v = seqs[b]
        keep = np.array([0 <= tables[b, t // PAGE] < n_pool for t in range(lens[b])])
        refs.append(att.decode_attention(q[b], k[keep], v[keep], SCALE))
    max_abs, mean_rel = errors(got[:2], np.stack(refs))
    assert max_abs <= 2e-2 and mean_rel <= 1e-2, (max_abs, mean_rel)
    assert np.array_equal(got[2], np.zeros_like(got[2]))


def test_cache_writers_skip_table_entries_outside_the_pools(pkg, dev):
    """kv_append and qk_norm_rope_append write nothing through a table entry outside the pools:
    every pool byte is unchanged except the rows of the valid writes; q is still written."""
    rng = np.random.default_rng(15)
    B, Hq, Hkv, n_pages = 4, 8, 2, 6
    kc0 = to_bf16(rng.standard_normal((n_pages, Hkv, PAGE, D)).astype(np.float32), dev)
    vc0 = to_bf16(rng.standard_normal((n_pages, Hkv, D, PAGE)).astype(np.float32), dev)
    tables = torch.tensor([[2, -1], [n_pages, 3], [5, 1], [-100, 4]], dtype=torch.int32, device=dev)
    pos = torch.tensor([20, 3, 17, 0], dtype=torch.int32, device=dev)  # pages: -1, n_pages, 1, -100
    k = to_bf16(rng.standard_normal((B, Hkv, D)).astype(np.float32), dev)
    v = to_bf16(rng.standard_normal((B, Hkv, D)).astype(np.float32), dev)
    kc, vc = kc0.clone(), vc0.clone()
    pkg.kv_append(k, v, kc, vc, tables, pos)
    ek, ev = kc0.clone(), vc0.clone()
    ek[1, :, 1, :] = k[2]
    ev[1, :, :, 1] = v[2]
    torch.cuda.synchronize()
    assert torch.equal(kc.view(torch.int16), ek.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), ev.view(torch.int16))

    qkv = to_bf16(rng.standard_normal((B, (Hq + 2 * Hkv) * D)).astype(np.float32), dev)
    nw = torch.ones(D, dtype=torch.bfloat16, device=dev)
    inv = torch.from_numpy(att.default_inv_freq()).to(dev)
    kc, vc = kc0.clone(), vc0.clone()
    q = pkg.qk_norm_rope_append(qkv, nw, nw, inv, pos, Hq, Hkv, 1e-6, kc, vc, tables)
    torch.cuda.synchronize()
    changed_k = (kc.view(torch.int16) != kc0.view(torch.int16)).any(dim=(1, 3))  # [pages, slot]
    changed_v = (vc.view(torch.int16) != vc0.view(torch.int16)).any(dim=(1, 2))
    allowed = torch.zeros((n_pages, PAGE), dtype=torch.bool, device=dev)
    allowed[1, 1] = True
    assert not (changed_k & ~allowed).any() and not (changed_v & ~allowed).any()
    assert changed_v[1, 1]
    assert torch.isfinite(q.float()).all() and q.abs().sum() > 0
