"""The bf16-expert path (the reference's default bf16 checkpoints, no FP8 requantisation) on the
GPU, through the C ABI.

* C1 golden vectors: transformers' own ``Qwen3MoeSparseMoeBlock`` wrote, on CPU, the bf16 output
  of the Qwen3-30B-A3B layer at 16 tokens (tests/golden/make_golden.py).  Fed the reference's
  own routing, the GPU's bf16 experts reproduce it >= 99% bit-identical, the rest within 2 bf16
  ulps of the output scale (the
  bf16 MFMA accumulates exactly in fp32; only the order of fp32 additions differs).
* the block (router + bf16 experts) against the oracle's bf16 grouped chain on the kernel's
  routing, at every tile height (16-, 32-, 64- and the LDS-tiled 128-row tiles);
* the 4096-token Zipf-skewed prefill chunk (C3's routing) on bf16 experts, one token of every
  128-row tile checked;
* a tiny Qwen3-MoE LM swapped with bf16 blocks, and one dispatching its bf16 experts through
  transformers' ``ExpertsInterface`` under the ``"mi355x"`` key, against transformers' own
  ``grouped_mm`` experts on the same GPU.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc
from tests.helpers import TOL_MAX_ABS, TOL_MEAN_REL, bf16_ulp_diff, errors, np_f32, to_bf16, to_dev

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", list(make_golden.CASES))
def test_bf16_experts_reproduce_transformers_golden(pkg, dev, case):
    cfg = make_golden.CASES[case]
    g = np.load(os.path.join(GOLDEN, f"{case}.npz"))
    x, wr, w13, w2 = make_golden.make_inputs(**cfg)
    T, k, H = cfg["T"], cfg["k"], cfg["H"]
    gi = g["indices"]
    gw = orc.from_bf16_bits(g["scores_bf16"]).reshape(T, k)
    out = pkg.experts_bf16(to_bf16(x, dev), to_dev(gi, dev), to_bf16(gw, dev), to_bf16(w13, dev), to_bf16(w2, dev))
    got = np_f32(out)
    ref = orc.from_bf16_bits(g["out_bf16"]).reshape(T, H)
    u = bf16_ulp_diff(got, ref)
    assert (u == 0).mean() >= 0.99, (u == 0).mean()
    # the rest within 2 bf16 ulps of the output's scale (the CPU oracle's bar on the same vectors)
    d = np.abs(got - ref)
    assert d.max() <= 2.0 ** -8 * max(float(np.abs(ref).max()), 1e-3) * 2, d.max()


def bf16_block_m(pkg, T, H, I, E, k):
    """Tile height of the bf16 path for T tokens (low 16 bits of the numerics key)."""
    return int(pkg._lib.load().moe_mi355x_block_numerics_key(T, H, I, E, k, 0)) & 0xFFFF


@pytest.mark.parametrize("T,H,I,E,k,bm", [(1, 2048, 768, 128, 8, 16), (16, 2048, 768, 128, 8, 16),
                                          (64, 2048, 768, 128, 8, 16), (200, 2048, 768, 128, 8, 128),
                                          (600, 2048, 768, 128, 8, 128), (37, 384, 256, 20, 5, 32),
                                          (100, 384, 256, 8, 2, 64), (257, 1024, 640, 12, 6, 128),
                                          (600, 4096, 1536, 16, 8, 128), (40, 512, 256, 4, 2, 128),
                                          (2, 384, 256, 20, 5, 16)])
def test_bf16_block_matches_oracle(pkg, dev, T, H, I, E, k, bm):
    """16-row tiles (S <= 8 E; from 2 tokens on the down GEMM combines each token itself), above the 128-row LDS-tiled kernel; where H % 256 != 0, 32-row
    tiles (S <= 16 E) and 64-row tiles.  128-row cases at the 30B and 235B widths, with 5 K blocks
    of 128 in the down GEMM's h (I = 640) and with the minimum of 4 bf16 K blocks (I = 256)."""
    assert bf16_block_m(pkg, T, H, I, E, k) == bm
    rng = np.random.default_rng(400 + T + H)
    x = orc.gen_normal_bf16(rng, (T, H))
    wr = orc.gen_normal_bf16(rng, (E, H), 0.02)
    w13 = orc.gen_normal_bf16(rng, (E, 2 * I, H), 0.02)
    w2 = orc.gen_normal_bf16(rng, (E, H, I), 0.02)
    out, (lg, w, ids) = pkg.moe_block_bf16(to_bf16(x, dev), to_bf16(wr, dev), k, to_bf16(w13, dev), to_bf16(w2, dev),
                                           return_routing=True)
    lg_n = np_f32(lg)
    lg_ref = orc.router_logits(x, wr)
    assert (bf16_ulp_diff(lg_n, lg_ref) > 1).mean() == 0
    ids_ref, w_ref, _ = orc.topk_from_logits(lg_n, k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    assert bf16_ulp_diff(np_f32(w), w_ref).max() <= 1
    sub = np.sort(rng.choice(T, min(T, 64), replace=False))
    ref = orc.experts_bf16(x[sub], ids_ref[sub], w_ref[sub], w13, w2, acc=np.float32)
    got = np_f32(out)[sub]
    max_abs, mean_rel = errors(got, ref)
    assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL, (max_abs, mean_rel)
    # the GEMMs accumulate exactly in fp32: nearly every output is the oracle's bf16 value
    assert (bf16_ulp_diff(got, ref) == 0).mean() >= 0.95
    # the experts entry point (sorted tiles, separate combine) fed the block's routing gives the
    # same bits as the block (expert-bucket tiles on 16-row tiles, combine inside the down GEMM)
    again = pkg.experts_bf16(to_bf16(x, dev), ids, w, to_bf16(w13, dev), to_bf16(w2, dev))
    assert torch.equal(out, again)


def test_bf16_prefill_zipf_every_tile(pkg, dev):
    """C3's routing (4096 tokens, Zipf-skewed: a few hot experts with many tiles, ragged last
    tiles) on bf16 30B experts, 128-row tiles; the first, the last and a random row of every tile
    are checked against the oracle's bf16 chain."""
    from tests.test_gpu_configs import tile_stratified_tokens

    T, H, I, E, k = 4096, 2048, 768, 128, 8
    assert bf16_block_m(pkg, T, H, I, E, k) == 128
    rng = np.random.default_rng(12)
    x = orc.gen_normal_bf16(rng, (T, H))
    lg = orc.gen_normal_bf16(rng, (T, E)) + orc.zipf_bias(E, 1.1, beta=1.5)
    ids, w, _ = orc.topk_from_logits(orc.round_bf16(lg), k)
    g = torch.Generator(device=dev).manual_seed(9)
    w13 = (torch.randn((E, 2 * I, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn((E, H, I), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    out = pkg.experts_bf16(to_bf16(x, dev), to_dev(ids, dev), to_bf16(w, dev), w13, w2)
    sub, n_tiles = tile_stratified_tokens(ids, E, 128, rng)
    assert n_tiles > 200
    ref = orc.experts_bf16(x[sub], ids[sub], w[sub], np_f32(w13), np_f32(w2), acc=np.float32)
    got = np_f32(out)[sub]
    max_abs, mean_rel = errors(got, ref)
    assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL, (max_abs, mean_rel)
    assert (bf16_ulp_diff(got, ref) == 0).mean() >= 0.95


def test_bf16_experts_deterministic(pkg, dev):
    rng = np.random.default_rng(7)
    T, H, I, E, k = 300, 512, 256, 16, 4
    x = to_bf16(orc.gen_normal_bf16(rng, (T, H)), dev)
    ids, w = orc.uniform_routing(rng, T, E, k)
    w13 = to_bf16(orc.gen_normal_bf16(rng, (E, 2 * I, H), 0.02), dev)
    w2 = to_bf16(orc.gen_normal_bf16(rng, (E, H, I), 0.02), dev)
    a = pkg.experts_bf16(x, to_dev(ids, dev), to_bf16(w, dev), w13, w2)
    b = pkg.experts_bf16(x, to_dev(ids, dev), to_bf16(w, dev), w13, w2)
    assert torch.equal(a, b)


transformers = pytest.importorskip("transformers")


def _tiny_lm(dev, impl=None):
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeForCausalLM

    cfg = Qwen3MoeConfig(vocab_size=128, hidden_size=256, intermediate_size=256, num_hidden_layers=2,
                         num_attention_heads=2, num_key_value_heads=1, head_dim=128, num_experts=16,
                         num_experts_per_tok=4, moe_intermediate_size=128, norm_topk_prob=True,
                         max_position_embeddings=256)
    if impl is not None:
        cfg._experts_implementation = impl
    torch.manual_seed(0)
    model = Qwen3MoeForCausalLM(cfg).to(torch.bfloat16).to(dev).eval()
    with torch.no_grad():
        for layer in model.model.layers:
            layer.mlp.gate.weight.normal_(0, 0.02)
            layer.mlp.experts.gate_up_proj.normal_(0, 0.02)
            layer.mlp.experts.down_proj.normal_(0, 0.02)
    return cfg, model


def test_swapped_bf16_blocks_match_transformers(pkg, dev):
    """Every swapped bf16 block, on the input transformers' own block saw, against that block's
    output (grouped_mm experts on this GPU), for a prefill and a decode step."""
    from transformers import DynamicCache

    cfg, model = _tiny_lm(dev)
    originals = [layer.mlp for layer in model.model.layers]
    captured = []

    def hook(mod, inp, out):
        captured.append((mod, inp[0].detach().clone(), out.detach().clone()))

    for m in originals:
        m.register_forward_hook(hook)
    ids = torch.randint(0, cfg.vocab_size, (3, 20), device=dev)
    with torch.no_grad():
        cache = DynamicCache()
        out = model(input_ids=ids, past_key_values=cache, use_cache=True)
        nxt = out.logits[:, -1].argmax(-1, keepdim=True)
        model(input_ids=nxt, past_key_values=cache, use_cache=True)
    assert len(captured) == 2 * cfg.num_hidden_layers
    for m in originals:
        m._forward_hooks.clear()
    swapped = {id(m): pkg.MI355XSparseMoeBlock.from_hf_block(m) for m in originals}
    for mod, x, y in captured:
        blk = swapped[id(mod)]
        assert not blk.is_fp8
        with torch.no_grad():
            got = blk(x)
        max_abs, mean_rel = errors(np_f32(got), np_f32(y))
        assert max_abs <= TOL_MAX_ABS and mean_rel <= TOL_MEAN_REL, (max_abs, mean_rel)


def test_experts_interface_dispatch_bf16(pkg, dev):
    """A model loaded with experts_implementation="mi355x" sends its bf16 experts to this path
    (TF/integrations/moe.py:567-570): same logits as the grouped_mm implementation within bf16 noise."""
    assert pkg.register()
    _, ref_model = _tiny_lm(dev, impl="grouped_mm")
    _, model = _tiny_lm(dev, impl=pkg.IMPLEMENTATION_KEY)
    ids = torch.randint(0, 128, (2, 12), device=dev)
    with torch.no_grad():
        want = ref_model(input_ids=ids).logits
        got = model(input_ids=ids).logits
    max_abs, mean_rel = errors(np_f32(got), np_f32(want))
    assert max_abs <= 5e-2 * max(1.0, float(want.abs().max())) and mean_rel <= 2e-2, (max_abs, mean_rel)
