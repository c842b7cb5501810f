"""Write golden vectors of the reference's bf16 MoE block, computed by transformers on CPU.

The reference server (AdvayMonga/inference-server) has no MoE code; its Qwen3-MoE path is
transformers' ``Qwen3MoeSparseMoeBlock`` (transformers 5.15.0,
models/qwen3_moe/modeling_qwen3_moe.py:270-281) with the default ``grouped_mm`` experts
implementation (integrations/moe.py:377-478), run by ``TorchBackend`` on ``DEVICE=cpu``.
These vectors pin what the oracle cannot derive from first principles: the CPU router's
bf16 logits, ``torch.topk``'s tie order, and the bf16 rounding sequence of the grouped
experts forward.

Inputs are NOT stored: they are regenerated from a numpy PCG64 seed by ``make_inputs`` (the
tests call the same function) and checked against the stored SHA-256 digests.

Run from the repo root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))

CASES = {
    # Qwen3-30B-A3B-shaped layer, 16 tokens, seed 0
    "c1_30b_t16": dict(T=16, H=2048, E=128, k=8, I=768, seed=0),
    # a small layer with more tokens (more ties, more experts per token batch)
    "small_t256": dict(T=256, H=256, E=16, k=4, I=128, seed=1),
}


def _bf16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    bits = a.view(np.uint32)
    r = (bits + np.uint32(0x7FFF) + ((bits >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    return r.view(np.float32)


def make_inputs(T, H, E, k, I, seed):
    """x ~ N(0,1), router and expert weights ~ N(0, 0.02), all rounded to bf16 (float32 arrays)."""
    rng = np.random.default_rng(seed)
    x = _bf16(rng.standard_normal((T, H), dtype=np.float32))
    wr = _bf16(rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.02))
    w13 = _bf16(rng.standard_normal((E, 2 * I, H), dtype=np.float32) * np.float32(0.02))
    w2 = _bf16(rng.standard_normal((E, H, I), dtype=np.float32) * np.float32(0.02))
    return x, wr, w13, w2


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def run_case(name, T, H, E, k, I, seed):
    import torch
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock

    x, wr, w13, w2 = make_inputs(T, H, E, k, I, seed)
    cfg = Qwen3MoeConfig(hidden_size=H, num_experts=E, num_experts_per_tok=k, moe_intermediate_size=I,
                         norm_topk_prob=True)
    cfg._experts_implementation = "grouped_mm"  # the default chosen at from_pretrained time
    block = Qwen3MoeSparseMoeBlock(cfg).to(torch.bfloat16).eval()
    with torch.no_grad():
        block.gate.weight.copy_(torch.from_numpy(wr).to(torch.bfloat16))
        block.experts.gate_up_proj.copy_(torch.from_numpy(w13).to(torch.bfloat16))
        block.experts.down_proj.copy_(torch.from_numpy(w2).to(torch.bfloat16))
        xt = torch.from_numpy(x).to(torch.bfloat16)
        logits, scores, idx = block.gate(xt)
        out = block(xt.view(1, T, H)).view(T, H)

    def bits(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)

    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(
        path,
        shape=np.array([T, H, E, k, I, seed], dtype=np.int64),
        digests=np.array([digest(x), digest(wr), digest(w13), digest(w2)]),
        logits_bf16=bits(logits),
        scores_bf16=bits(scores),
        indices=idx.numpy().astype(np.int64),
        out_bf16=bits(out),
    )
    print(f"wrote {path}")


def main():
    for name, cfg in CASES.items():
        run_case(name, **cfg)


if __name__ == "__main__":
    sys.exit(main())
