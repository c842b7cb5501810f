"""Host-side logic of the drop-in layer (CPU only): validation, the plugin registration and
the parameter layout the transformers FP8 experts module uses."""

from __future__ import annotations

import pytest
import torch


def test_wrappers_reject_cpu_tensors(pkg):
    x = torch.zeros(4, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm GPU"):
        pkg.quantize_act_fp8(x)
    with pytest.raises(ValueError, match="ROCm GPU"):
        pkg.route(x, torch.zeros(16, 256, dtype=torch.bfloat16), 4)


def test_wrappers_reject_bad_dtypes_and_shapes(pkg):
    with pytest.raises(TypeError):
        pkg.kernels._need(torch.zeros(2, 2, dtype=torch.float32), "x", torch.bfloat16)
    with pytest.raises(ValueError, match="2-D"):
        pkg.kernels._need(torch.zeros(2, 2, 2, dtype=torch.bfloat16), "x", torch.bfloat16, 2)


def test_experts_forward_rejects_static_activation(pkg):
    class Dummy(torch.nn.Module):
        activation_scheme = "static"

    with pytest.raises(NotImplementedError, match="static"):
        pkg.mi355x_fp8_experts_forward(Dummy(), None, None, None)


def test_registration_with_transformers(pkg):
    pytest.importorskip("transformers")
    from transformers.integrations.finegrained_fp8 import ALL_FP8_EXPERTS_FUNCTIONS, FP8ExpertsInterface

    assert pkg.register()
    assert pkg.IMPLEMENTATION_KEY in FP8ExpertsInterface._global_mapping
    fn = ALL_FP8_EXPERTS_FUNCTIONS.get_interface(pkg.IMPLEMENTATION_KEY, None)
    assert fn is pkg.mi355x_fp8_experts_forward


def test_parameter_layout_matches_transformers_fp8_experts(pkg):
    pytest.importorskip("transformers")
    from transformers.integrations.finegrained_fp8 import FP8Experts
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig

    cfg = Qwen3MoeConfig(hidden_size=256, num_experts=8, num_experts_per_tok=2, moe_intermediate_size=128)
    with torch.device("meta"):
        ref = FP8Experts(cfg, block_size=(128, 128))
        ours = pkg.MI355XFp8Experts(8, 256, 128)
    ref_p = {n: (tuple(p.shape), p.dtype) for n, p in ref.named_parameters()}
    our_p = {n: (tuple(p.shape), p.dtype) for n, p in ours.named_parameters()}
    assert ref_p == our_p


def test_swap_finds_qwen3_moe_blocks(pkg, monkeypatch):
    pytest.importorskip("transformers")
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeForCausalLM

    cfg = Qwen3MoeConfig(vocab_size=64, hidden_size=256, intermediate_size=256, num_hidden_layers=2,
                         num_attention_heads=2, num_key_value_heads=1, head_dim=128, num_experts=8,
                         num_experts_per_tok=2, moe_intermediate_size=128, norm_topk_prob=True)
    with torch.device("meta"):
        model = Qwen3MoeForCausalLM(cfg)
    seen = []
    monkeypatch.setattr(pkg.MI355XSparseMoeBlock, "from_hf_block",
                        classmethod(lambda cls, block, **kw: seen.append(block) or torch.nn.Identity()))
    assert pkg.swap_moe_blocks(model) == 2
    assert len(seen) == 2
    assert all(isinstance(layer.mlp, torch.nn.Identity) for layer in model.model.layers)


def test_torch_ops_are_registered(pkg):
    ops = torch.ops.moe_mi355x
    for name in ("route", "align", "moe_fp8", "moe_block_fp8"):
        assert hasattr(ops, name), name
    pkg.torch_ops.register()  # a second registration in the same process is a no-op


def test_torch_ops_fake_shapes(pkg):
    """The operators' fake implementations (meta tensors: no device, no library call) give
    the shapes and dtypes of the real outputs."""
    T, H, I, E, k = 5, 256, 128, 16, 4
    m = dict(device="meta")
    x = torch.empty((T, H), dtype=torch.bfloat16, **m)
    wr = torch.empty((E, H), dtype=torch.bfloat16, **m)
    ids, w, logits = torch.ops.moe_mi355x.route(x, wr, k, True)
    assert (ids.shape, ids.dtype, w.shape, w.dtype, logits.shape) == ((T, k), torch.int32, (T, k), torch.bfloat16,
                                                                       (T, E))
    perm, tiles, counts, offsets, n_tiles = torch.ops.moe_mi355x.align(ids, E, 16)
    assert perm.shape == (T * k,) and counts.shape == (E,) and offsets.shape == (E + 1,) and n_tiles.shape == (1,)
    assert tiles.shape == (pkg.torch_ops.align_max_tiles(T * k, E, 16), 4)
    fp8 = torch.float8_e4m3fn
    w13 = torch.empty((E, 2 * I, H), dtype=fp8, **m)
    s13 = torch.empty((E, 2 * I // 128, H // 128), dtype=torch.float32, **m)
    w2 = torch.empty((E, H, I), dtype=fp8, **m)
    s2 = torch.empty((E, H // 128, I // 128), dtype=torch.float32, **m)
    assert torch.ops.moe_mi355x.moe_fp8(x, ids, w, w13, s13, w2, s2).shape == (T, H)
    x3 = torch.empty((2, 3, H), dtype=torch.bfloat16, **m)
    out = torch.ops.moe_mi355x.moe_block_fp8(x3, wr, k, True, w13, s13, w2, s2)
    assert out.shape == (2, 3, H) and out.dtype == torch.bfloat16


def test_align_max_tiles_matches_library(pkg):
    lib = pkg._lib.load()
    for S in (0, 1, 7, 8, 64, 512, 1000, 32768):
        for E in (1, 8, 128):
            for bm in (16, 32, 128):
                assert pkg.torch_ops.align_max_tiles(S, E, bm) == max(lib.moe_mi355x_align_max_tiles(S, E, bm), 1)


def test_bf16_experts_stay_bf16_unless_fp8_is_requested(pkg):
    """The reference runs bf16 experts (torch_backend.py:38-40): the swap keeps them bf16 (the
    bf16 path) unless quantize_fp8=True asks for the FP8 requantisation."""
    pytest.importorskip("transformers")
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeForCausalLM

    cfg = Qwen3MoeConfig(vocab_size=64, hidden_size=256, intermediate_size=256, num_hidden_layers=2,
                         num_attention_heads=2, num_key_value_heads=1, head_dim=128, num_experts=8,
                         num_experts_per_tok=2, moe_intermediate_size=128, norm_topk_prob=True)
    with torch.device("meta"):
        model = Qwen3MoeForCausalLM(cfg).to(torch.bfloat16)
    assert pkg.swap_moe_blocks(model) == 2
    for layer in model.model.layers:
        assert isinstance(layer.mlp, pkg.MI355XSparseMoeBlock) and not layer.mlp.is_fp8
        assert isinstance(layer.mlp.experts, pkg.experts.MI355XBf16Experts)
        assert layer.mlp.experts.gate_up_proj.dtype == torch.bfloat16
        assert tuple(layer.mlp.experts.gate_up_proj.shape) == (8, 256, 256)


@pytest.mark.parametrize("H,I,E,k", [(2048, 768, 128, 8), (2048, 768, 100, 6), (4096, 1536, 128, 8),
                                     (512, 256, 64, 8)])
def test_numerics_buckets_split_at_key_changes(pkg, H, I, E, k):
    """Every batch size inside a bucket has the bucket's numerics key, so a padded replay of the
    bucket's graph computes each real row as the unpadded eager call does."""
    lib = pkg._lib.load()
    buckets = pkg.experts.numerics_buckets(pkg.experts.DEFAULT_BUCKETS, H, I, E, k)
    assert set(pkg.experts.DEFAULT_BUCKETS) <= set(buckets)
    prev = 0
    for b in buckets:
        kb = lib.moe_mi355x_block_numerics_key(b, H, I, E, k, 1)
        assert kb != 0
        for t in range(prev + 1, b + 1):
            assert lib.moe_mi355x_block_numerics_key(t, H, I, E, k, 1) == kb, (t, b)
        prev = b
    # the tile height changes at S = 8 E and S = 16 E: both are bucket edges
    for edge in (8 * E // k, 16 * E // k):
        if edge < buckets[-1]:
            assert edge in buckets
