"""The HIP path behind the reference's own call sites (GPU).

* transformers' FP8 experts module dispatching to the ``"mi355x"`` experts implementation
  (TF/integrations/moe.py:567-570, finegrained_fp8.py:757-768);
* a tiny Qwen3-MoE causal LM whose sparse blocks were swapped for ``MI355XSparseMoeBlock``,
  driven the way the reference backend drives it: a prefill forward with a KV cache, then
  a batched one-token decode step (src/inference_server/backends/torch_backend.py:283-322).
  Every swapped block's output is checked against the oracle on the block's captured input.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc
from tests.helpers import TOL_MAX_ABS, TOL_MEAN_REL, errors, f8_codes, np_f32

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def _tiny_config(**kw):
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig

    base = dict(vocab_size=128, hidden_size=256, intermediate_size=256, num_hidden_layers=2, num_attention_heads=2,
                num_key_value_heads=1, head_dim=128, num_experts=16, num_experts_per_tok=4, moe_intermediate_size=128,
                norm_topk_prob=True, max_position_embeddings=256)
    base.update(kw)
    return Qwen3MoeConfig(**base)


def test_fp8_experts_interface_dispatch(pkg, dev):
    from transformers.integrations.finegrained_fp8 import ALL_FP8_EXPERTS_FUNCTIONS, FP8Experts
    from transformers.integrations.moe import use_experts_implementation

    assert pkg.register()
    cfg = _tiny_config()
    cfg._experts_implementation = pkg.IMPLEMENTATION_KEY
    cls = use_experts_implementation(experts_class=FP8Experts, experts_interface=ALL_FP8_EXPERTS_FUNCTIONS)
    mod = cls(cfg, block_size=(128, 128)).to(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    E, I, H = 16, 128, 256
    w13 = (torch.randn((E, 2 * I, H), generator=g, device=dev) * 0.02)
    w2 = (torch.randn((E, H, I), generator=g, device=dev) * 0.02)
    q13, s13 = pkg.quantize_weight_fp8(w13)
    q2, s2 = pkg.quantize_weight_fp8(w2)
    with torch.no_grad():
        mod.gate_up_proj.copy_(q13)
        mod.gate_up_proj_scale_inv.copy_(s13)
        mod.down_proj.copy_(q2)
        mod.down_proj_scale_inv.copy_(s2)
    T, k = 40, 4
    x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, device=dev)[:k] for _ in range(T)])  # int64, like torch.topk
    w = torch.softmax(torch.randn((T, k), generator=g, device=dev), -1).to(torch.bfloat16)
    out = mod(x, ids, w)
    assert out.shape == (T, H) and out.dtype == torch.bfloat16
    ref = orc.experts_fp8(np_f32(x), ids.cpu().numpy(), np_f32(w), f8_codes(q13), s13.cpu().numpy(),
                          f8_codes(q2), s2.cpu().numpy())
    max_abs, mean_rel = errors(np_f32(out), ref)
    assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL


def test_swapped_model_prefill_and_decode(pkg, dev):
    from transformers import DynamicCache
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeForCausalLM

    torch.manual_seed(0)
    cfg = _tiny_config()
    model = Qwen3MoeForCausalLM(cfg).to(torch.bfloat16).to(dev).eval()
    with torch.no_grad():
        for layer in model.model.layers:
            layer.mlp.gate.weight.normal_(0, 0.02)
            layer.mlp.experts.gate_up_proj.normal_(0, 0.02)
            layer.mlp.experts.down_proj.normal_(0, 0.02)
    assert pkg.swap_moe_blocks(model, quantize_fp8=True) == cfg.num_hidden_layers
    captured = []

    def hook(mod, inp, out):
        captured.append((mod, inp[0].detach().clone(), out.detach().clone()))

    for layer in model.model.layers:
        assert isinstance(layer.mlp, pkg.MI355XSparseMoeBlock)
        layer.mlp.register_forward_hook(hook)

    B, S = 3, 24
    ids = torch.randint(0, cfg.vocab_size, (B, S), device=dev)
    cache = DynamicCache()
    with torch.no_grad():
        out = model(input_ids=ids, past_key_values=cache, use_cache=True)
        nxt = out.logits[:, -1].argmax(-1, keepdim=True)
        out2 = model(input_ids=nxt, past_key_values=out.past_key_values, use_cache=True)
    assert out.logits.shape == (B, S, cfg.vocab_size)
    assert out2.logits.shape == (B, 1, cfg.vocab_size)
    assert torch.isfinite(out2.logits.float()).all()
    assert len(captured) == 2 * cfg.num_hidden_layers  # prefill + decode per layer

    for mod, x, y in captured:
        xs = np_f32(x.reshape(-1, cfg.hidden_size))
        e = mod.experts
        # feed the GPU's own routing to the oracle experts: bit-exact ids are tested elsewhere
        _, (glg, gw, gids) = pkg.moe_block_fp8(x, mod.gate.weight, cfg.num_experts_per_tok, e.gate_up_proj,
                                               e.gate_up_proj_scale_inv, e.down_proj, e.down_proj_scale_inv,
                                               return_routing=True)
        ids_from_gpu_logits, _, _ = orc.topk_from_logits(np_f32(glg), cfg.num_experts_per_tok)
        np.testing.assert_array_equal(gids.cpu().numpy(), ids_from_gpu_logits)
        ref = orc.experts_fp8(xs, gids.cpu().numpy(), np_f32(gw), f8_codes(e.gate_up_proj),
                              e.gate_up_proj_scale_inv.cpu().numpy(), f8_codes(e.down_proj),
                              e.down_proj_scale_inv.cpu().numpy())
        max_abs, mean_rel = errors(np_f32(y).reshape(ref.shape), ref)
        assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL


def _tiny_model(dev, **kw):
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeForCausalLM

    torch.manual_seed(0)
    cfg = _tiny_config(**kw)
    model = Qwen3MoeForCausalLM(cfg).to(torch.bfloat16).to(dev).eval()
    with torch.no_grad():
        for layer in model.model.layers:
            layer.mlp.gate.weight.normal_(0, 0.02)
            layer.mlp.experts.gate_up_proj.normal_(0, 0.02)
            layer.mlp.experts.down_proj.normal_(0, 0.02)
    return cfg, model


def test_graphed_swap_replays_match_oracle(pkg, dev):
    """swap_moe_blocks(graphed=True): decode batches replay a captured graph per bucket.  Every
    replayed block output is checked against the oracle on the block's own routing, and equals the
    eager block bit for bit."""
    from transformers import DynamicCache

    cfg, model = _tiny_model(dev)
    assert pkg.swap_moe_blocks(model, quantize_fp8=True, graphed=True) == cfg.num_hidden_layers
    captured = []

    def hook(mod, inp, out):
        captured.append((mod, inp[0].detach().clone(), out.detach().clone()))

    for layer in model.model.layers:
        assert isinstance(layer.mlp, pkg.MI355XGraphedMoeBlock)
        layer.mlp.register_forward_hook(hook)
    B, S = 5, 12  # decode batch 5 pads to the 8-token bucket
    ids = torch.randint(0, cfg.vocab_size, (B, S), device=dev)
    cache = DynamicCache()
    with torch.no_grad():
        out = model(input_ids=ids, past_key_values=cache, use_cache=True)  # 60 tokens: bucket 64
        nxt = out.logits[:, -1].argmax(-1, keepdim=True)
        for _ in range(2):  # two decode steps: the second replays the graphs captured by the first
            out = model(input_ids=nxt, past_key_values=cache, use_cache=True)
            nxt = out.logits[:, -1].argmax(-1, keepdim=True)
    torch.cuda.synchronize()
    assert len(captured) == 3 * cfg.num_hidden_layers
    assert all(8 in m._graphs and 64 in m._graphs for m in {id(m): m for m, _, _ in captured}.values())
    for mod, x, y in captured:
        blk = mod.block
        xs = x.reshape(-1, cfg.hidden_size)
        eager, (glg, gw, gids) = pkg.moe_block_fp8(xs, blk.gate.weight, cfg.num_experts_per_tok,
                                                   blk.experts.gate_up_proj, blk.experts.gate_up_proj_scale_inv,
                                                   blk.experts.down_proj, blk.experts.down_proj_scale_inv,
                                                   return_routing=True)
        assert torch.equal(y.reshape(eager.shape), eager)
        ids_ref, w_ref, _ = orc.topk_from_logits(np_f32(glg), cfg.num_experts_per_tok)
        np.testing.assert_array_equal(gids.cpu().numpy(), ids_ref)
        e = blk.experts
        ref = orc.experts_fp8(np_f32(xs), ids_ref, w_ref, f8_codes(e.gate_up_proj),
                              e.gate_up_proj_scale_inv.cpu().numpy(), f8_codes(e.down_proj),
                              e.down_proj_scale_inv.cpu().numpy())
        max_abs, mean_rel = errors(np_f32(y).reshape(ref.shape), ref)
        assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL


def test_graphed_block_crossing_tile_switch(pkg, dev):
    """E = 100, k = 6: the tile height changes at 8 E / k = 133.3 tokens, inside the default
    (128, 256] bucket.  The bucket list gains an edge at 133, so 129..133 tokens (16-row tiles)
    and 134 tokens (32-row tiles) each replay a graph of their own tiling, bit-equal to eager."""
    E, H, I, k = 100, 512, 256, 6
    block = pkg.MI355XSparseMoeBlock(E, H, I, k, device=dev)
    g = torch.Generator(device=dev).manual_seed(21)
    with torch.no_grad():
        block.gate.weight.copy_((torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16))
        from tests.helpers import gpu_weights

        for name, t in zip(("gate_up_proj", "gate_up_proj_scale_inv", "down_proj", "down_proj_scale_inv"),
                           gpu_weights(E, H, I, dev, seed=22)):
            getattr(block.experts, name).copy_(t)
    graphed = pkg.MI355XGraphedMoeBlock(block)
    assert 133 in graphed.buckets
    for T in (130, 133, 134, 200):
        x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
        want = block(x)
        got = graphed(x)
        torch.cuda.synchronize()
        assert torch.equal(got, want), T


def test_compiled_swapped_model_matches_eager(pkg, dev):
    """The reference compiles the whole model when COMPILE_MODEL is set (torch_backend.py:44-47).
    The swapped blocks call torch.ops.moe_mi355x.*, so Dynamo traces through them: the prefill and a
    decode step of torch.compile(model, fullgraph=True) equal the eager model bit for bit."""
    from transformers import DynamicCache

    cfg, model = _tiny_model(dev)
    assert pkg.swap_moe_blocks(model, quantize_fp8=True) == cfg.num_hidden_layers
    B, S = 2, 10
    ids = torch.randint(0, cfg.vocab_size, (B, S), device=dev)

    def step(input_ids, cache):
        return model(input_ids=input_ids, past_key_values=cache, use_cache=True).logits

    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    with torch.no_grad():
        cache_e, cache_c = DynamicCache(), DynamicCache()
        want = step(ids, cache_e)
        got = compiled(ids, cache_c)
        assert torch.equal(got, want)
        nxt = want[:, -1].argmax(-1, keepdim=True)  # one decode step on the KV cache
        want1 = step(nxt, cache_e)
        got1 = compiled(nxt, cache_c)
        assert got1.shape == (B, 1, cfg.vocab_size)
        assert torch.equal(got1, want1)
    torch.cuda.synchronize()


def test_graphed_bf16_block_across_tile_heights(pkg, dev):
    """bf16 experts, E = 16, k = 4: 16-row tiles up to 32 tokens, then the LDS-tiled 128-row
    kernel.  Each tiling gets bucket edges of its own, and every replay equals the eager block bit
    for bit."""
    E, H, I, k = 16, 512, 256, 4
    block = pkg.MI355XSparseMoeBlock(E, H, I, k, device=dev, experts_dtype=torch.bfloat16)
    g = torch.Generator(device=dev).manual_seed(31)
    with torch.no_grad():
        block.gate.weight.copy_((torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16))
        block.experts.gate_up_proj.copy_((torch.randn((E, 2 * I, H), generator=g, device=dev) * 0.02).to(torch.bfloat16))
        block.experts.down_proj.copy_((torch.randn((E, H, I), generator=g, device=dev) * 0.02).to(torch.bfloat16))
    graphed = pkg.MI355XGraphedMoeBlock(block)
    heights = {t: int(pkg._lib.load().moe_mi355x_block_numerics_key(t, H, I, E, k, 0)) & 0xFFFF
               for t in (30, 33, 64, 65, 100)}
    assert heights == {30: 16, 33: 128, 64: 128, 65: 128, 100: 128}, heights
    assert 32 in graphed.buckets
    for T in (3, 30, 33, 64, 65, 100):
        x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
        want = block(x)
        got = graphed(x)
        torch.cuda.synchronize()
        assert torch.equal(got, want), T


def test_compiled_bf16_swapped_model_matches_eager(pkg, dev):
    """The same with the default bf16 checkpoint kept in bf16 (torch.ops.moe_mi355x.moe_block_bf16):
    a compiled prefill and decode step of the model equal eager bit for bit, and the swapped block
    compiled on its own equals eager on an 80-token chunk, which runs the 128-row bf16 tiles.  (The
    whole model is compared at 10 tokens: at 40 transformers' own compiled attention path already
    differs from eager in the last bits, with FP8 blocks as with bf16 ones.)"""
    from transformers import DynamicCache

    cfg, model = _tiny_model(dev, moe_intermediate_size=256)
    assert pkg.swap_moe_blocks(model) == cfg.num_hidden_layers
    mlp = model.model.layers[0].mlp
    assert not mlp.is_fp8
    B, S = 2, 10
    ids = torch.randint(0, cfg.vocab_size, (B, S), device=dev)

    def step(input_ids, cache):
        return model(input_ids=input_ids, past_key_values=cache, use_cache=True).logits

    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    with torch.no_grad():
        cache_e, cache_c = DynamicCache(), DynamicCache()
        want = step(ids, cache_e)
        got = compiled(ids, cache_c)
        assert torch.equal(got, want)
        nxt = want[:, -1].argmax(-1, keepdim=True)
        want1 = step(nxt, cache_e)
        got1 = compiled(nxt, cache_c)
        assert torch.equal(got1, want1)
        # 80 tokens x 4 slots > 16 E: the 128-row bf16 tiles
        key = pkg._lib.load().moe_mi355x_block_numerics_key(80, 256, 256, 16, 4, 0)
        assert int(key) & 0xFFFF == 128
        x = torch.randn((2, 40, 256), device=dev).to(torch.bfloat16)
        block_c = torch.compile(lambda t: mlp(t), backend="aot_eager", fullgraph=True)
        assert torch.equal(block_c(x), mlp(x))
    torch.cuda.synchronize()
