"""Shared input builders and comparison helpers for the tests."""

from __future__ import annotations

import numpy as np
import torch

from oracle import moe_oracle as orc

TOL_MAX_ABS = 2e-2  # bf16 layer output vs the dequantise-then-fp32 oracle
TOL_MEAN_REL = 1e-2


def to_bf16(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).to(dev)


def to_f8(q, dev):
    return torch.from_numpy(np.ascontiguousarray(q, dtype=np.uint8)).view(torch.float8_e4m3fn).to(dev)


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def f8_codes(t):
    return t.view(torch.uint8).cpu().numpy()


def np_f32(t):
    return t.detach().float().cpu().numpy()


def bf16_ulp_diff(a, b):
    """Distance in bf16 units in the last place between bf16-valued float32 arrays."""
    def ordered(x):
        bits = orc.bf16_bits(x).astype(np.int32)
        return np.where(bits & 0x8000, -(bits & 0x7FFF), bits)
    return np.abs(ordered(a) - ordered(b))


def errors(out, ref):
    d = np.abs(np.asarray(out, np.float64) - np.asarray(ref, np.float64))
    return float(d.max()), float(d.mean() / max(np.abs(ref).mean(), 1e-30))


def gpu_weights(E, H, I, dev, seed=0, std=0.02):
    """bf16 N(0, std) expert weights generated on the GPU and block-quantised there."""
    from __graft_entry__ import load_package

    pkg = load_package()
    g = torch.Generator(device=dev).manual_seed(seed)
    w13 = (torch.randn((E, 2 * I, H), generator=g, device=dev) * std).to(torch.bfloat16)
    w2 = (torch.randn((E, H, I), generator=g, device=dev) * std).to(torch.bfloat16)
    q13, s13 = pkg.quantize_weight_fp8(w13)
    q2, s2 = pkg.quantize_weight_fp8(w2)
    del w13, w2
    return q13, s13, q2, s2
