"""Fused decoder-layer pieces on the GPU, through the C ABI, against the oracle
(oracle/attn_oracle.py: RMSNorm and rotary pinned by transformers golden vectors).

* RMSNorm: within 1 bf16 ulp of the oracle, >= 99% bit-identical (the fp32 sum of squares
  is accumulated in another order).
* q/k norm + rotary + KV append: q and k within 1 bf16 ulp of the oracle's norm-then-rotary
  chain given the same inv_freq, >= 98% bit-identical (the fp32 sum of squares is accumulated
  in another order; the device's fp32 cos / sin are within one ulp of the float64-rounded
  ones); v placed bit-exactly.
* MoE sublayer: bit-identical to RMSNorm, the MoE block and a bf16 residual add run as
  separate calls.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attn_oracle as att
from oracle import moe_oracle as orc
from tests.helpers import gpu_weights, to_bf16

pytestmark = pytest.mark.gpu

D, PAGE = 128, 16


def ulps(a, b):
    def ordered(x):
        bits = orc.bf16_bits(x).astype(np.int32)
        return np.where(bits & 0x8000, -(bits & 0x7FFF), bits)
    return np.abs(ordered(a) - ordered(b))


@pytest.mark.parametrize("rows,cols", [(64, 2048), (300, 128), (5, 4096), (1, 8)])
def test_rms_norm(pkg, dev, rows, cols):
    rng = np.random.default_rng(rows + cols)
    x = orc.round_bf16((rng.standard_normal((rows, cols)) * 3).astype(np.float32))
    w = orc.round_bf16((1 + 0.1 * rng.standard_normal(cols)).astype(np.float32))
    out = pkg.rms_norm(to_bf16(x, dev), to_bf16(w, dev), 1e-6).float().cpu().numpy()
    d = ulps(out, att.rms_norm(x, w, 1e-6))
    assert d.max() <= 1 and (d == 0).mean() >= 0.99


@pytest.mark.parametrize("Hq,Hkv,B", [(32, 4, 7), (4, 2, 3)])
def test_qk_norm_rope_append(pkg, dev, Hq, Hkv, B):
    from inference_server_amd import decode as dec

    rng = np.random.default_rng(B)
    nh = Hq + 2 * Hkv
    qkv = orc.round_bf16(rng.standard_normal((B, nh * D)).astype(np.float32))
    qw = orc.round_bf16((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    kw = orc.round_bf16((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    pos = rng.integers(0, 8000, size=B).astype(np.int32)
    max_pages = 8000 // PAGE + 1
    n_pages = B * max_pages
    tables = rng.permutation(n_pages).astype(np.int32).reshape(B, max_pages)
    kc = torch.zeros((n_pages, Hkv, PAGE, D), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros((n_pages, Hkv, D, PAGE), dtype=torch.bfloat16, device=dev)
    inv_freq = dec.default_inv_freq(dec.DecoderConfig(), dev)
    q = pkg.qk_norm_rope_append(to_bf16(qkv, dev), to_bf16(qw, dev), to_bf16(kw, dev), inv_freq,
                                torch.from_numpy(pos).to(dev), Hq, Hkv, 1e-6, kc, vc, torch.from_numpy(tables).to(dev))
    torch.cuda.synchronize()
    cos, sin = att.rope_cos_sin(pos, D, 1e6, inv_freq=inv_freq.cpu().numpy())
    heads = qkv.reshape(B, nh, D)
    q_ref = att.rotary(att.rms_norm(heads[:, :Hq], qw, 1e-6), cos, sin)
    k_ref = att.rotary(att.rms_norm(heads[:, Hq:Hq + Hkv], kw, 1e-6), cos, sin)
    d = ulps(q.float().cpu().numpy(), q_ref)
    assert d.max() <= 1 and (d == 0).mean() >= 0.98, (d.max(), (d == 0).mean())
    kcn, vcn = kc.float().cpu().numpy(), vc.float().cpu().numpy()
    for b in range(B):
        pg, slot = tables[b, pos[b] // PAGE], pos[b] % PAGE
        dk = ulps(kcn[pg, :, slot, :], k_ref[b])
        assert dk.max() <= 1 and (dk == 0).mean() >= 0.95
        assert np.array_equal(vcn[pg, :, :, slot], heads[b, Hq + Hkv:])



def test_qk_norm_rope_append_position_outside_the_table(pkg, dev):
    """q is still produced; the cache is left untouched for a position with no page."""
    from inference_server_amd import decode as dec

    rng = np.random.default_rng(5)
    Hq, Hkv, B = 4, 2, 2
    nh = Hq + 2 * Hkv
    qkv = orc.round_bf16(rng.standard_normal((B, nh * D)).astype(np.float32))
    qw = orc.round_bf16((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
    pos = np.array([40, 5], np.int32)  # the first is past its 2-page table
    tables = np.array([[0, 1], [2, 3]], np.int32)
    kc = torch.zeros((4, Hkv, PAGE, D), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros((4, Hkv, D, PAGE), dtype=torch.bfloat16, device=dev)
    inv_freq = dec.default_inv_freq(dec.DecoderConfig(), dev)
    q = pkg.qk_norm_rope_append(to_bf16(qkv, dev), to_bf16(qw, dev), to_bf16(qw, dev), inv_freq,
                                torch.from_numpy(pos).to(dev), Hq, Hkv, 1e-6, kc, vc, torch.from_numpy(tables).to(dev))
    torch.cuda.synchronize()
    cos, sin = att.rope_cos_sin(pos, D, 1e6, inv_freq=inv_freq.cpu().numpy())
    q_ref = att.rotary(att.rms_norm(qkv.reshape(B, nh, D)[:, :Hq], qw, 1e-6), cos, sin)
    assert ulps(q.float().cpu().numpy(), q_ref).max() <= 1
    kcn, vcn = kc.float().cpu().numpy(), vc.float().cpu().numpy()
    assert not kcn[[0, 1]].any() and not vcn[[0, 1]].any()  # sequence 0: nothing written
    assert kcn[2, :, 5, :].any() and vcn[2, :, :, 5].any()  # sequence 1: its slot

@pytest.mark.parametrize("M,N,K", [(128, 5120, 2048), (128, 2048, 4096), (1, 1024, 256), (3, 256, 512),
                                   (300, 64, 128), (129, 640, 1024), (1, 5120, 2048), (5, 1024, 4096),
                                   (24, 2048, 4096), (40, 512, 2048), (64, 5120, 2048), (0, 64, 128)])
def test_linear_bf16(pkg, dev, M, N, K):
    """y = bf16(x @ w^T) against the exact product rounded once (fp64 sum of the exact bf16
    products): the kernel accumulates in fp32 (the MFMA sums its products exactly, the K blocks are
    added in fp32), so an output differs only where that fp32 sum sits within a few fp32 ulps of a
    bf16 rounding boundary: at most 1 bf16 ulp (or 2^-20 of sum |x w| near zero), >= 99.9%
    identical.  (128, 5120, 2048) and (128, 2048, 4096) are the decode step's q/k/v and o_proj at
    batch 128; the shapes cover every row-tile count (1, 2, 4, 8 per wave), partial row blocks,
    the K split (1 to 8 chunks and none) and an empty batch."""
    rng = np.random.default_rng(M + N + K)
    x = orc.round_bf16(rng.standard_normal((M, K)).astype(np.float32))
    w = orc.round_bf16((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    y = pkg.linear_bf16(to_bf16(x, dev), to_bf16(w, dev)).float().cpu().numpy()
    if M == 0:
        assert y.shape == (0, N)
        return
    ref = orc.round_bf16((x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32))
    d = ulps(y, ref)
    # near zero (cancellation) a few fp32 ulps of the summed magnitudes are many bf16 ulps of the
    # result: there the bound is 2^-20 of sum |x w| (the fp32 accumulation's error)
    mag = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T
    ok = (d <= 1) | (np.abs(y.astype(np.float64) - ref) <= 2.0 ** -20 * mag)
    assert ok.all() and (d == 0).mean() >= 0.999, (int(d.max()), float((d == 0).mean()))


@pytest.mark.parametrize("T", [1, 64, 600])
def test_moe_sublayer_equals_separate_calls(pkg, dev, T):
    E, H, I, k = 32, 512, 256, 4
    q13, s13, q2, s2 = gpu_weights(E, H, I, dev, seed=T)
    g = torch.Generator(device=dev).manual_seed(T)
    h = (torch.randn((T, H), generator=g, device=dev) * 2).to(torch.bfloat16)
    ln = (1 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
    wr = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    fused = pkg.moe_sublayer_fp8(h, ln, 1e-6, wr, k, q13, s13, q2, s2)
    x = pkg.rms_norm(h, ln, 1e-6)
    sep = h + pkg.moe_block_fp8(x, wr, k, q13, s13, q2, s2)
    torch.cuda.synchronize()
    assert torch.equal(fused, sep)


@pytest.mark.parametrize("T", [1, 64, 600])
def test_moe_sublayer_with_attention_residual(pkg, dev, T):
    """With ``add`` the sublayer forms ``h' = bf16(h + add)`` itself (the residual add after the
    attention): bit-identical to torch's bf16 add followed by the sublayer on ``h'``."""
    E, H, I, k = 32, 512, 256, 4
    q13, s13, q2, s2 = gpu_weights(E, H, I, dev, seed=T + 1)
    g = torch.Generator(device=dev).manual_seed(T + 1)
    h = (torch.randn((T, H), generator=g, device=dev) * 2).to(torch.bfloat16)
    o = (torch.randn((T, H), generator=g, device=dev) * 0.5).to(torch.bfloat16)
    ln = (1 + 0.1 * torch.randn(H, generator=g, device=dev)).to(torch.bfloat16)
    wr = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    fused = pkg.moe_sublayer_fp8(h, ln, 1e-6, wr, k, q13, s13, q2, s2, add=o)
    sep = pkg.moe_sublayer_fp8(h + o, ln, 1e-6, wr, k, q13, s13, q2, s2)
    torch.cuda.synchronize()
    assert torch.equal(fused, sep)


@pytest.mark.parametrize("T", [1, 8, 64, 128])
def test_moe_sublayer_prologue_matches_oracle(pkg, dev, T):
    """The MoE sublayer at the Qwen3-30B-A3B shape (residual add + post-attention RMSNorm in one
    launch, router GEMM + x quantisation in the next) against the oracle:
    hs = bf16(h + o), x = attn_oracle.rms_norm(hs, w_ln), moe_oracle's router and FP8 experts
    on x, then bf16(hs + block).  Tokens whose oracle logits have a near-tie at the top-k
    boundary (the 8th and 9th logits within 1 bf16 ulp) are left out: one ulp of RMSNorm or
    router rounding may route them to the other expert.  With 128 experts whose logits are
    ~N(0, 0.9), the 8th / 9th gap is within one ulp for about a fifth of the tokens."""
    E, H, I, k = 128, 2048, 768, 8
    q13, s13, q2, s2 = gpu_weights(E, H, I, dev, seed=50 + T)
    rng = np.random.default_rng(60 + T)
    h = orc.gen_normal_bf16(rng, (T, H), 2.0)
    o = orc.gen_normal_bf16(rng, (T, H), 0.5)
    ln = orc.round_bf16((1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
    wr = orc.gen_normal_bf16(rng, (E, H), 0.02)
    out = pkg.moe_sublayer_fp8(to_bf16(h, dev), to_bf16(ln, dev), 1e-6, to_bf16(wr, dev), k, q13, s13, q2, s2,
                               add=to_bf16(o, dev))
    got = out.float().cpu().numpy()
    hs = orc.round_bf16(h + o)
    x = att.rms_norm(hs, ln, 1e-6)
    lg = orc.router_logits(x, wr)
    ids, w, _ = orc.topk_from_logits(lg, k)
    blk = orc.experts_fp8(x, ids, w, q13.view(torch.uint8).cpu().numpy(), s13.cpu().numpy(),
                          q2.view(torch.uint8).cpu().numpy(), s2.cpu().numpy(), acc=np.float32)
    ref = orc.round_bf16(hs + blk)
    srt = np.sort(lg, axis=1)[:, ::-1]
    gap_ulps = ulps(srt[:, k - 1], srt[:, k])
    keep = gap_ulps > 1
    assert keep.sum() >= max(1, T // 2)
    d = np.abs(got[keep].astype(np.float64) - ref[keep])
    mean_rel = d.mean() / np.abs(blk[keep]).mean()  # relative to the block's contribution
    # the output is bf16(hs + block): a block within 2e-2 of the oracle's moves it by at most 2e-2
    # plus one bf16 ulp of the output (the residual add's own rounding can fall the other way;
    # hs ~ N(0, 2) reaches ~8, where one ulp is 6.3e-2)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref[keep]), 2.0 ** -126))) - 7)
    assert np.all(d <= 2e-2 + ulp) and mean_rel <= 1e-2, (float((d - ulp).max()), mean_rel)
