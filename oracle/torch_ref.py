"""The reference's PyTorch CPU path for the MoE block, restated in torch.

TEST AND BASELINE INFRASTRUCTURE ONLY: ``tests/`` pin it, ``bench.py``'s ``cpu_baseline`` leg
times it on the GPU box's host cores.  The product package never imports it.

The reference server runs its model on ``DEVICE=cpu`` when no accelerator is configured
(src/inference_server/config.py:13-23); a Qwen3-MoE layer then executes transformers'
``Qwen3MoeTopKRouter.forward`` (TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267) and the
default ``grouped_mm_experts_forward`` (TF/integrations/moe.py:377-478), TF = transformers 5.15.0.
This module follows those lines op for op with torch's CPU kernels:

  logits = F.linear(x, W_r)  ->  softmax fp32  ->  topk  ->  renormalise  ->  bf16
  sort(expert ids)  ->  gather rows  ->  histc  ->  cumsum  ->  grouped_mm(gate_up)
  ->  silu(gate) * up  ->  grouped_mm(down)  ->  * routing weight  ->  inverse permutation
  ->  view(T, k, H).sum(1)  ->  bf16

``experts_bf16`` is that path on bf16 weights (its output is pinned against
the golden vectors transformers wrote).  ``experts_fp8_dequant`` is the FP8 configurations' CPU
path: weights dequantised once to fp32 (``Fp8Dequantize``, TF/integrations/finegrained_fp8.py:
1005-1048), the dynamic per-token, per-128-column activation quantisation applied to both GEMM
inputs (the rule the FP8 kernels define, finegrained_fp8.py:191-196), fp32 grouped GEMMs whose
outputs are rounded to bf16 as the reference's bf16 GEMMs are.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

FP8_MAX = 448.0
GROUP = 128


def route(x: torch.Tensor, w_router: torch.Tensor, k: int, renorm: bool = True):
    """``Qwen3MoeTopKRouter.forward`` (modeling_qwen3_moe.py:258-267): (logits, weights, ids)."""
    logits = F.linear(x, w_router)
    probs = torch.softmax(logits, dim=-1, dtype=torch.float32)
    vals, ids = torch.topk(probs, k, dim=-1)
    if renorm:
        vals = vals / vals.sum(dim=-1, keepdim=True)
    return logits, vals.to(x.dtype), ids


def dequantize_weight(q: torch.Tensor, scale_inv: torch.Tensor) -> torch.Tensor:
    """``Fp8Dequantize._dequantize_one`` (finegrained_fp8.py:1005-1048): e4m3 codes times the
    fp32 scale of their 128x128 block, fp32 [..., N, K]."""
    w = q.to(torch.float32)
    *lead, N, K = w.shape
    w = w.view(*lead, N // GROUP, GROUP, K // GROUP, GROUP) * scale_inv.view(*lead, N // GROUP, 1, K // GROUP, 1)
    return w.view(*lead, N, K)


def quant_dequant_act(x: torch.Tensor) -> torch.Tensor:
    """Dynamic activation quantisation per row and 128-column group, then back to fp32:
    s = amax / 448 (1 for an all-zero group), q = e4m3(clamp(x / s)), x' = q * s."""
    R, C = x.shape
    g = x.to(torch.float32).view(R, C // GROUP, GROUP)
    amax = g.abs().amax(dim=-1, keepdim=True)
    s = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = (g / s).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return (q.to(torch.float32) * s).view(R, C)


def _grouped_experts(x, top_k_index, top_k_weights, w13, w2, num_experts, act_quant: bool):
    """``grouped_mm_experts_forward`` (moe.py:377-478).  ``w13`` [E, 2I, H] and ``w2`` [E, H, I]
    in the GEMM dtype (bf16, or fp32 dequantised weights); the GEMM outputs are bf16."""
    T, H = x.shape
    k = top_k_index.shape[-1]
    sample_weights = top_k_weights.reshape(-1)
    expert_ids = top_k_index.reshape(-1)
    expert_ids_g, perm = torch.sort(expert_ids)
    xg = x[perm // k]
    wg = sample_weights[perm]
    tokens_per_expert = torch.histc(expert_ids_g.float(), bins=num_experts, min=0, max=num_experts - 1)
    offsets = torch.cumsum(tokens_per_expert, dim=0, dtype=torch.int32)
    a = quant_dequant_act(xg) if act_quant else xg
    y = F.grouped_mm(a.to(w13.dtype), w13.transpose(-2, -1), offs=offsets).to(torch.bfloat16)
    gate, up = y.chunk(2, dim=-1)
    h = F.silu(gate) * up  # bf16 ops: silu rounded to bf16, the product rounded again
    a2 = quant_dequant_act(h) if act_quant else h
    z = F.grouped_mm(a2.to(w2.dtype), w2.transpose(-2, -1), offs=offsets).to(torch.bfloat16)
    weighted = z * wg.unsqueeze(-1)
    inv_perm = torch.empty_like(perm)
    inv_perm[perm] = torch.arange(perm.size(0))
    weighted = weighted[inv_perm]
    return weighted.view(T, k, H).sum(dim=1).to(x.dtype)


def experts_bf16(x, top_k_index, top_k_weights, w13, w2):
    """bf16 experts: the reference's default path."""
    return _grouped_experts(x, top_k_index, top_k_weights, w13, w2, w13.shape[0], act_quant=False)


def experts_fp8_dequant(x, top_k_index, top_k_weights, w13_f32, w2_f32):
    """FP8 experts on fp32 weights dequantised once (``dequantize_weight``), with dynamic
    activation quantisation of both GEMM inputs."""
    return _grouped_experts(x, top_k_index, top_k_weights, w13_f32, w2_f32, w13_f32.shape[0], act_quant=True)


def block_fp8_dequant(x, w_router, k, w13_f32, w2_f32, renorm: bool = True):
    """``Qwen3MoeSparseMoeBlock.forward`` (modeling_qwen3_moe.py:276-281) on dequantised FP8 experts."""
    _, w, ids = route(x, w_router, k, renorm)
    return experts_fp8_dequant(x, ids, w, w13_f32, w2_f32)
