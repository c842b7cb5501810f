"""BASELINE config 5 at its own workload (GPU): one Qwen3-30B-A3B-shaped decoder layer of the
48-layer decode step at batch 128, contexts uniform in [512, 8192], against the oracle
(oracle/attn_oracle.py + oracle/moe_oracle.py), not against transformers.

The layer is ``Qwen3MoeDecoderLayer.forward`` (TF/models/qwen3_moe/modeling_qwen3_moe.py:319-348):
input RMSNorm, fused q/k/v projection, q/k RMSNorm + rotary + KV append, paged GQA attention
(32 q heads, 4 kv heads, head_dim 128, 16-token pages), o_proj, residual add, post-attention
RMSNorm, the FP8 MoE block, residual add.  Checked stage by stage at the layer tolerance
(max-abs <= 2e-2, mean-rel <= 1e-2):

* paged attention on the kernel's q and cache, every sequence, every split count (1-8 splits
  of <= 64 pages) present;
* the attention sublayer (RMSNorm -> q/k/v -> norms + rotary -> attention -> o_proj) against the
  oracle's own chain from the same hidden states;
* the MoE block on the kernel's post-attention RMSNorm output: routing bit-exact given the
  kernel's logits, output at the bar;
* the decode step's layer output equals bf16(h + attn) + block bit for bit, so the stages above
  bound it.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attn_oracle as att
from oracle import moe_oracle as orc
from tests.helpers import TOL_MAX_ABS, TOL_MEAN_REL, bf16_ulp_diff, errors, f8_codes, np_f32

pytestmark = pytest.mark.gpu

PAGE, D = 16, 128
B = 128
SPLIT_PAGES = 64  # pages per attention split of the kernel


def _bf16_matmul_t(a, w):
    """``F.linear`` on bf16 operands: exact products, one bf16 rounding of the fp32-accumulated sum."""
    return orc.round_bf16((np.asarray(a, np.float64) @ np.asarray(w, np.float64).T).astype(np.float32))


@pytest.fixture(scope="module")
def c5_layer(pkg, dev):
    from inference_server_amd import decode as dec

    cfg = dec.DecoderConfig()
    g = torch.Generator(device=dev).manual_seed(55)
    w = dec.DecoderLayerWeights.random(cfg, dev, g)
    with torch.no_grad():  # non-trivial norm weights, so that a mixed-up norm shows
        for t in (w.ln1, w.q_norm, w.k_norm, w.ln2):
            t.copy_((1.0 + 0.2 * torch.randn(t.shape, generator=g, device=dev)).to(torch.bfloat16))
    rng = np.random.default_rng(5)
    ctx = rng.integers(512, 8193, size=B).astype(np.int32)
    n_pages = (ctx + PAGE - 1) // PAGE
    total = int(n_pages.sum()) + 4
    order = rng.permutation(total).astype(np.int32)
    tables = np.zeros((B, int(n_pages.max())), np.int32)
    used = 0
    for b in range(B):
        tables[b, :n_pages[b]] = order[used:used + n_pages[b]]
        used += n_pages[b]
    kc = torch.randn((total, cfg.kv_heads, PAGE, D), generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn((total, cfg.kv_heads, D, PAGE), generator=g, device=dev).to(torch.bfloat16)
    h = torch.randn((B, cfg.hidden), generator=g, device=dev).to(torch.bfloat16)
    return dict(cfg=cfg, w=w, ctx=ctx, tables=tables, kc=kc, vc=vc, h=h)


def _sequence_kv(kc, vc, table, length):
    """Keys / values [length, Hkv, d] of one sequence, gathered on the GPU and read back."""
    n = (length + PAGE - 1) // PAGE
    idx = torch.from_numpy(np.ascontiguousarray(table[:n], np.int64)).to(kc.device)
    return att.gather_paged(np_f32(kc.index_select(0, idx)), np_f32(vc.index_select(0, idx)), np.arange(n), length)


@pytest.mark.timeout(900)
def test_c5_decoder_layer_batch128(pkg, dev, c5_layer):
    from inference_server_amd import decode as dec
    from inference_server_amd import kernels

    L = c5_layer
    cfg, w, ctx, tables, kc, vc, h = L["cfg"], L["w"], L["ctx"], L["tables"], L["kc"], L["vc"], L["h"]
    Hq, Hkv, H = cfg.heads, cfg.kv_heads, cfg.hidden
    scale = D ** -0.5
    splits = (ctx + PAGE * SPLIT_PAGES - 1) // (PAGE * SPLIT_PAGES)
    assert set(splits.tolist()) == set(range(1, 9)), sorted(set(splits.tolist()))
    pos_d = torch.from_numpy(ctx - 1).to(dev)
    ctx_d = torch.from_numpy(ctx).to(dev)
    tab_d = torch.from_numpy(tables).to(dev)
    inv_freq = dec.default_inv_freq(cfg, dev)

    # ---- GPU: the layer's stages, then the decode step itself ----
    x1 = kernels.rms_norm(h, w.ln1, cfg.rms_eps)
    qkv = torch.nn.functional.linear(x1, w.wqkv)
    q = kernels.qk_norm_rope_append(qkv, w.q_norm, w.k_norm, inv_freq, pos_d, Hq, Hkv, cfg.rms_eps, kc, vc, tab_d)
    a = kernels.paged_attention_decode(q, kc, vc, tab_d, ctx_d, scale)
    o = dec.attention_sublayer(w, h, pos_d, ctx_d, tab_d, inv_freq, kc, vc)  # appends the same k, v again
    hs = h + o
    x2 = kernels.rms_norm(hs, w.ln2, cfg.rms_eps)
    blk, (lg, wts, ids) = kernels.moe_block_fp8(x2, w.router, cfg.top_k, w.q13, w.s13, w.q2, w.s2,
                                                return_routing=True)
    model = dec.DecodeModel(cfg, [w], dec.PagedKVCache(1, 1, Hkv, dev))
    model.cache.k[0], model.cache.v[0] = kc, vc
    out = model.step(h, pos_d, ctx_d, tab_d)
    torch.cuda.synchronize()
    assert torch.equal(out, hs + blk), "the decode step's layer output is not bf16(h + attn) + block"

    # ---- 1. paged attention on the kernel's q and cache: every sequence ----
    qn = np_f32(q)
    kv = [_sequence_kv(kc, vc, tables[b], int(ctx[b])) for b in range(B)]
    a_ref = np.stack([att.decode_attention(qn[b], kv[b][0], kv[b][1], scale) for b in range(B)])
    an = np_f32(a)
    for s in range(1, 9):  # per split count
        sel = splits == s
        ma, mr = errors(an[sel], a_ref[sel])
        assert ma <= TOL_MAX_ABS and mr <= TOL_MEAN_REL, (s, ma, mr)
    ma, mr = errors(an, a_ref)
    print(f"attention: max_abs {ma:.3g} mean_rel {mr:.3g}")

    # ---- 2. the attention sublayer against the oracle's own chain from h ----
    hn = np_f32(h)
    x1_ref = att.rms_norm(hn, np_f32(w.ln1), cfg.rms_eps)
    assert bf16_ulp_diff(np_f32(x1), x1_ref).max() <= 1
    qkv_ref = _bf16_matmul_t(x1_ref, np_f32(w.wqkv)).reshape(B, Hq + 2 * Hkv, D)
    cos, sin = att.rope_cos_sin(ctx - 1, D, cfg.rope_theta, inv_freq=inv_freq.cpu().numpy())
    q_ref = att.rotary(att.rms_norm(qkv_ref[:, :Hq], np_f32(w.q_norm), cfg.rms_eps), cos, sin)
    k_ref = att.rotary(att.rms_norm(qkv_ref[:, Hq:Hq + Hkv], np_f32(w.k_norm), cfg.rms_eps), cos, sin)
    v_ref = qkv_ref[:, Hq + Hkv:]
    a_chain = np.empty_like(a_ref)
    for b in range(B):
        keys, vals = kv[b][0].copy(), kv[b][1].copy()
        keys[-1], vals[-1] = k_ref[b], v_ref[b]  # the oracle's own new token
        a_chain[b] = att.decode_attention(q_ref[b], keys, vals, scale)
    o_ref = _bf16_matmul_t(a_chain.reshape(B, Hq * D), np_f32(w.wo))
    ma, mr = errors(np_f32(o), o_ref)
    print(f"attention sublayer: max_abs {ma:.3g} mean_rel {mr:.3g} |ref| max {np.abs(o_ref).max():.3g}")
    assert ma <= TOL_MAX_ABS and mr <= TOL_MEAN_REL, (ma, mr)

    # ---- 3. the MoE block on the kernel's post-attention RMSNorm output ----
    x2n = np_f32(x2)
    hs_ref = orc.round_bf16(hn + o_ref)
    x2_ref = att.rms_norm(hs_ref, np_f32(w.ln2), cfg.rms_eps)
    assert errors(x2n, x2_ref)[1] <= TOL_MEAN_REL
    ids_ref, w_ref, _ = orc.topk_from_logits(np_f32(lg), cfg.top_k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    assert bf16_ulp_diff(np_f32(wts), w_ref).max() <= 1
    blk_ref = orc.experts_fp8(x2n, ids_ref, np_f32(wts), f8_codes(w.q13), w.s13.cpu().numpy(), f8_codes(w.q2),
                              w.s2.cpu().numpy(), acc=np.float32)
    ma, mr = errors(np_f32(blk), blk_ref)
    print(f"moe block: max_abs {ma:.3g} mean_rel {mr:.3g} |ref| max {np.abs(blk_ref).max():.3g}")
    assert ma <= TOL_MAX_ABS and mr <= TOL_MEAN_REL, (ma, mr)
