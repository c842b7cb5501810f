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
                        classmethod(lambda cls, block: seen.append(block) or torch.nn.Identity()))
    assert pkg.swap_moe_blocks(model) == 2
    assert len(seen) == 2
    assert all(isinstance(layer.mlp, torch.nn.Identity) for layer in model.model.layers)
