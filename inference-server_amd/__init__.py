"""MI355X (gfx950) Qwen3-MoE FP8 expert hot path.

Importable as ``inference_server_amd`` (the on-disk folder name carries a hyphen;
``__graft_entry__.load_package()`` registers it under that module name).

Layers:
  ``_lib``     ctypes binding of ``libmoe_mi355x.so`` (C ABI: ``include/moe_mi355x.h``)
  ``kernels``  torch-tensor wrappers of every entry point
  ``torch_ops`` the route / align / moe_fp8 / moe_block_fp8 entry points as ``torch.ops.moe_mi355x``
  ``experts``  drop-in modules, the transformers experts-interface registration, and the
               HIP-graph replay of a block per decode batch bucket
  ``checkpoint`` FP8 expert layers from a local safetensors checkpoint
  ``build``    hipcc build of the library
"""

from __future__ import annotations

from . import _lib, decode, kernels, torch_ops  # noqa: F401
from .checkpoint import CheckpointIndex, load_moe_block, load_moe_layer  # noqa: F401
from .experts import (  # noqa: F401
    IMPLEMENTATION_KEY,
    MI355XFp8Experts,
    MI355XGraphedMoeBlock,
    MI355XSparseMoeBlock,
    MI355XTopKRouter,
    mi355x_fp8_experts_forward,
    register,
    swap_moe_blocks,
)
from .kernels import (  # noqa: F401
    align,
    experts_bf16,
    experts_fp8,
    kv_append,
    moe_block_bf16,
    moe_block_fp8,
    moe_sublayer_fp8,
    paged_attention_decode,
    qk_norm_rope_append,
    linear_bf16,
    rms_norm,
    quantize_act_fp8,
    quantize_weight_fp8,
    route,
    topk_softmax,
)

__version__ = "0.1.0"
