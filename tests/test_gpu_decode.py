"""The decode step of ``inference_server_amd.decode`` against transformers' own decoder layers (GPU).

A tiny Qwen3-MoE causal LM (eager attention, MoE blocks swapped for ``MI355XSparseMoeBlock``) runs
a prefill with a ``DynamicCache`` and then one batched decode step, the way the reference backend
drives it (src/inference_server/backends/torch_backend.py:283-322).  Its prefill keys / values are
copied into the paged cache, and ``DecodeModel.step`` on the same new-token embeddings must give the
hidden state that transformers' last decoder layer returns for the decode step
(TF/models/qwen3_moe/modeling_qwen3_moe.py:319-348): max-abs <= 2e-2 of the hidden-state scale and
mean relative error <= 2e-2.  The mean bound is twice the single-kernel one: the hidden states of
this tiny model are ~0.05 in magnitude, and two layers of bf16 rounding chains (norms, rotary,
projections, the attention's weighted sum, whose terms cancel) put the measured agreement at
0.4-1.4%, the same with and without left padding.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.helpers import errors, np_f32

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")

PAGE = 16


def _model(dev, n_layers=2, heads=4, kv_heads=2):
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeForCausalLM

    cfg = Qwen3MoeConfig(vocab_size=128, hidden_size=256, intermediate_size=256, num_hidden_layers=n_layers,
                         num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=128, num_experts=16,
                         num_experts_per_tok=4, moe_intermediate_size=128, norm_topk_prob=True,
                         max_position_embeddings=512, rope_theta=1e6)
    cfg._attn_implementation = "eager"
    torch.manual_seed(0)
    model = Qwen3MoeForCausalLM(cfg).to(torch.bfloat16).to(dev).eval()
    with torch.no_grad():
        for layer in model.model.layers:
            layer.mlp.gate.weight.normal_(0, 0.02)
            layer.mlp.experts.gate_up_proj.normal_(0, 0.02)
            layer.mlp.experts.down_proj.normal_(0, 0.02)
            # non-trivial norm weights, so that a mixed-up norm shows
            for w in (layer.input_layernorm.weight, layer.post_attention_layernorm.weight,
                      layer.self_attn.q_norm.weight, layer.self_attn.k_norm.weight):
                w.copy_(1.0 + 0.2 * torch.randn_like(w.float()))
    return cfg, model


@pytest.mark.parametrize("lens", [[23], [40, 17, 5]])
def test_decode_step_matches_transformers(pkg, dev, lens):
    from transformers import DynamicCache

    from inference_server_amd import decode as dec

    cfg, model = _model(dev)
    assert pkg.swap_moe_blocks(model) == cfg.num_hidden_layers
    B, S = len(lens), max(lens)
    ids = torch.randint(0, cfg.vocab_size, (B, S), device=dev)
    # left padding, as the reference's batched decode does; the padded keys are masked out
    attn_mask = torch.zeros((B, S), dtype=torch.long, device=dev)
    for b, L in enumerate(lens):
        attn_mask[b, S - L:] = 1
    nxt = torch.randint(0, cfg.vocab_size, (B, 1), device=dev)
    outs = {}

    def hook(mod, inp, out):
        outs["last"] = out.detach().clone()

    model.model.layers[-1].register_forward_hook(hook)
    cache = DynamicCache()
    with torch.no_grad():
        pos = (attn_mask.cumsum(-1) - 1).clamp(min=0)
        model(input_ids=ids, attention_mask=attn_mask, position_ids=pos, past_key_values=cache, use_cache=True)
        full_mask = torch.cat([attn_mask, torch.ones((B, 1), dtype=torch.long, device=dev)], dim=1)
        new_pos = torch.tensor(lens, device=dev).view(B, 1)
        model(input_ids=nxt, attention_mask=full_mask, position_ids=new_pos, past_key_values=cache, use_cache=True)
        ref = outs["last"].view(B, cfg.hidden_size)
        emb = model.model.embed_tokens(nxt).view(B, cfg.hidden_size)

    dcfg = dec.DecoderConfig(hidden=cfg.hidden_size, heads=cfg.num_attention_heads, kv_heads=cfg.num_key_value_heads,
                             head_dim=128, experts=cfg.num_experts, top_k=cfg.num_experts_per_tok,
                             moe_intermediate=cfg.moe_intermediate_size, rms_eps=cfg.rms_norm_eps, rope_theta=1e6)
    layers = [dec.DecoderLayerWeights.from_hf_layer(l, dcfg) for l in model.model.layers]
    max_pages = (S + 1 + PAGE - 1) // PAGE + 1
    n_pages = B * max_pages + 2
    kv = dec.PagedKVCache(cfg.num_hidden_layers, n_pages, cfg.num_key_value_heads, dev)
    # scattered page assignment
    perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(1)).to(torch.int32)
    tables = perm[: B * max_pages].view(B, max_pages).contiguous().to(dev)
    for i in range(cfg.num_hidden_layers):
        k_all, v_all = cache.layers[i].keys, cache.layers[i].values  # [B, Hkv, S + 1, d], post-rotary
        for b, L in enumerate(lens):
            rows = torch.arange(S - L, S, device=dev)  # this sequence's prefill tokens (left padded)
            k = k_all[b, :, rows].transpose(0, 1).contiguous()  # [L, Hkv, d]
            v = v_all[b, :, rows].transpose(0, 1).contiguous()
            pkg.kv_append(k, v, kv.k[i], kv.v[i], tables[b:b + 1].expand(L, -1).contiguous(),
                          torch.arange(L, dtype=torch.int32, device=dev))
    model_dec = dec.DecodeModel(dcfg, layers, kv)
    positions = torch.tensor(lens, dtype=torch.int32, device=dev)
    with torch.no_grad():
        got = model_dec.step(emb.contiguous(), positions, positions + 1, tables)
    torch.cuda.synchronize()
    g, r = np_f32(got), np_f32(ref)
    scale = float(np.abs(r).max())
    max_abs, mean_rel = errors(g, r)
    assert max_abs <= 2e-2 * max(scale, 1.0) and mean_rel <= 2e-2, (max_abs, mean_rel, scale)


def test_decode_step_graph_replays_match_eager(pkg, dev):
    from inference_server_amd import decode as dec

    dcfg = dec.DecoderConfig(hidden=256, heads=8, kv_heads=2, experts=16, top_k=4, moe_intermediate=128)
    gen = torch.Generator(device=dev).manual_seed(3)
    layers = [dec.DecoderLayerWeights.random(dcfg, dev, gen) for _ in range(3)]
    B, max_pages = 5, 8
    kv = dec.PagedKVCache(len(layers), B * max_pages, dcfg.kv_heads, dev)
    for t in kv.k + kv.v:
        t.copy_(torch.randn(t.shape, generator=gen, device=dev).to(torch.bfloat16))
    tables = torch.arange(B * max_pages, dtype=torch.int32, device=dev).view(B, max_pages)
    lens = torch.tensor([1, 16, 17, 60, 127], dtype=torch.int32, device=dev)
    h = torch.randn((B, dcfg.hidden), generator=gen, device=dev).to(torch.bfloat16)
    model = dec.DecodeModel(dcfg, layers, kv)
    with torch.no_grad():
        eager = model.step(h, lens - 1, lens, tables)
        graph, statics, out = model.capture(h, lens - 1, lens, tables)
        for _ in range(3):
            graph.replay()
            torch.cuda.synchronize()
            # eager work between replays
            junk = torch.randn((1024, 1024), device=dev) @ torch.randn((1024, 1024), device=dev)
            del junk
            assert torch.equal(out, eager)
