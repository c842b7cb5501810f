"""Write golden vectors of the reference's decode-step attention pieces, computed by transformers on CPU.

The reference server's Qwen3-MoE decoder layer is transformers 5.15.0's
``Qwen3MoeDecoderLayer`` (models/qwen3_moe/modeling_qwen3_moe.py:305-348).  Around the MoE
block it runs ``Qwen3MoeRMSNorm`` (:285-299), the rotary embedding (``Qwen3MoeRotaryEmbedding``
:381-436, ``apply_rotary_pos_emb`` :59-81) and ``eager_attention_forward`` (:96-119).  These
vectors pin the bf16 rounding sequence of those functions, which closed forms leave open.

Inputs are NOT stored: ``make_inputs`` regenerates them from a numpy PCG64 seed (the tests call
the same function) and the stored SHA-256 digests check that it did.

Run from the repo root:  python tests/golden/make_golden_attn.py
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from make_golden import _bf16, digest  # noqa: E402

CASES = {
    # 4 query heads on 2 kv heads, a 37-token context
    "attn_g2_l37": dict(Hq=4, Hkv=2, L=37, H=256, seed=11),
    # the Qwen3-30B-A3B head grouping (8 query heads per kv head), 300 tokens
    "attn_g8_l300": dict(Hq=16, Hkv=2, L=300, H=512, seed=12),
}
HEAD_DIM = 128
THETA = 1e6
EPS = 1e-6


def make_inputs(Hq, Hkv, L, H, seed):
    """Pre-rotary q [Hq, d] of the new token, pre-rotary k [L, Hkv, d] and v [L, Hkv, d] of the
    whole context (the last row is the new token), the hidden rows x [4, H] and an RMSNorm
    weight [H], all bf16-valued float32; the new token sits at position L - 1."""
    rng = np.random.default_rng(seed)
    q = _bf16(rng.standard_normal((Hq, HEAD_DIM), dtype=np.float32))
    k = _bf16(rng.standard_normal((L, Hkv, HEAD_DIM), dtype=np.float32))
    v = _bf16(rng.standard_normal((L, Hkv, HEAD_DIM), dtype=np.float32))
    x = _bf16(rng.standard_normal((4, H), dtype=np.float32) * np.float32(3.0))
    w = _bf16(1.0 + 0.1 * rng.standard_normal(H, dtype=np.float32))
    return q, k, v, x, w


def run_case(name, Hq, Hkv, L, H, seed):
    import torch
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import (
        Qwen3MoeRMSNorm,
        Qwen3MoeRotaryEmbedding,
        apply_rotary_pos_emb,
        eager_attention_forward,
    )

    q, k, v, x, w = make_inputs(Hq, Hkv, L, H, seed)
    cfg = Qwen3MoeConfig(hidden_size=H, num_attention_heads=Hq, num_key_value_heads=Hkv, head_dim=HEAD_DIM,
                         rope_theta=THETA, rms_norm_eps=EPS)
    bf = torch.bfloat16
    with torch.no_grad():
        norm = Qwen3MoeRMSNorm(H, eps=EPS).to(bf)
        norm.weight.copy_(torch.from_numpy(w).to(bf))
        x_norm = norm(torch.from_numpy(x).to(bf))

        rope = Qwen3MoeRotaryEmbedding(cfg)
        pos = torch.arange(L, dtype=torch.int64).view(1, L)
        qt = torch.from_numpy(q).to(bf).view(1, Hq, 1, HEAD_DIM)
        kt = torch.from_numpy(k).to(bf).permute(1, 0, 2).reshape(1, Hkv, L, HEAD_DIM)
        vt = torch.from_numpy(v).to(bf).permute(1, 0, 2).reshape(1, Hkv, L, HEAD_DIM)
        cos, sin = rope(vt, pos)                       # [1, L, d] bf16
        k_rot = apply_rotary_pos_emb(kt, kt, cos, sin)[0]
        q_rot = apply_rotary_pos_emb(qt, qt, cos[:, L - 1:], sin[:, L - 1:])[0]

        class _Module:
            num_key_value_groups = Hq // Hkv
            training = False

        attn, _ = eager_attention_forward(_Module(), q_rot, k_rot, vt, None, scaling=HEAD_DIM ** -0.5)

    def bits(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)

    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(
        path,
        shape=np.array([Hq, Hkv, L, H, seed], dtype=np.int64),
        digests=np.array([digest(a) for a in (q, k, v, x, w)]),
        inv_freq=rope.inv_freq.numpy().astype(np.float32),
        rmsnorm_bf16=bits(x_norm),
        cos_bf16=bits(cos[0]),
        sin_bf16=bits(sin[0]),
        q_rot_bf16=bits(q_rot[0, :, 0, :]),
        k_rot_bf16=bits(k_rot[0].permute(1, 0, 2)),
        attn_bf16=bits(attn[0, 0]),  # [Hq, d]
    )
    print(f"wrote {path}")


def main():
    for name, cfg in CASES.items():
        run_case(name, **cfg)


if __name__ == "__main__":
    sys.exit(main())
