"""Pins the torch restatement of the reference's CPU path (oracle/torch_ref.py), which bench.py
times as the CPU baseline (CPU only).

* bf16 experts: transformers' own block wrote golden vectors on CPU (tests/golden/make_golden.py);
  the restatement, fed the golden routing, reproduces the golden output almost bit for bit, and its
  router reproduces the golden logits bit for bit.
* FP8 experts: against the numpy oracle (same routing, same dequantised weights and activation
  quantisation), within bf16 rounding noise.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc
from oracle import torch_ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_golden  # noqa: E402


def _bf(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)


@pytest.mark.parametrize("case", list(make_golden.CASES))
def test_bf16_path_matches_transformers_golden(case):
    cfg = make_golden.CASES[case]
    g = np.load(os.path.join(GOLDEN, f"{case}.npz"))
    x, wr, w13, w2 = make_golden.make_inputs(**cfg)
    T, E, k, H = cfg["T"], cfg["E"], cfg["k"], cfg["H"]
    logits, _, _ = torch_ref.route(_bf(x), _bf(wr), k)
    np.testing.assert_array_equal(logits.view(torch.int16).numpy().view(np.uint16).reshape(-1),
                                  g["logits_bf16"].reshape(-1))
    gi = torch.from_numpy(g["indices"])
    gw = torch.from_numpy(g["scores_bf16"].astype(np.int16)).view(torch.bfloat16).reshape(T, k)
    out = torch_ref.experts_bf16(_bf(x), gi, gw, _bf(w13), _bf(w2))
    ref = orc.from_bf16_bits(g["out_bf16"]).reshape(T, H)
    d = np.abs(out.float().numpy() - ref)
    assert (d == 0).mean() >= 0.99
    assert d.max() <= 2.0 ** -8 * max(float(np.abs(ref).max()), 1e-3) * 2


def test_fp8_path_matches_numpy_oracle():
    rng = np.random.default_rng(3)
    T, H, I, E, k = 40, 256, 128, 8, 3
    x = orc.gen_normal_bf16(rng, (T, H))
    w13 = orc.gen_normal_bf16(rng, (E, 2 * I, H), 0.02)
    w2 = orc.gen_normal_bf16(rng, (E, H, I), 0.02)
    q13, s13 = orc.quantize_weight_fp8(w13)
    q2, s2 = orc.quantize_weight_fp8(w2)
    ids, w = orc.uniform_routing(rng, T, E, k)
    ref = orc.experts_fp8(x, ids, w, q13, s13, q2, s2)
    f8 = lambda q: torch.from_numpy(q).view(torch.float8_e4m3fn)  # noqa: E731
    w13f = torch_ref.dequantize_weight(f8(q13), torch.from_numpy(s13))
    w2f = torch_ref.dequantize_weight(f8(q2), torch.from_numpy(s2))
    np.testing.assert_array_equal(w13f.numpy(), orc.dequantize_weight_fp8(q13, s13))
    out = torch_ref.experts_fp8_dequant(_bf(x), torch.from_numpy(ids.astype(np.int64)), _bf(w), w13f, w2f)
    d = np.abs(out.float().numpy() - ref)
    assert d.max() <= 2e-2 and d.mean() / np.abs(ref).mean() <= 1e-2
    assert (d == 0).mean() >= 0.9  # same rounding chain: mostly identical bits


def test_quant_dequant_act_matches_oracle():
    rng = np.random.default_rng(4)
    x = orc.gen_normal_bf16(rng, (7, 384))
    x[2, :128] = 0.0
    q, s = orc.quantize_act_fp8(x)
    np.testing.assert_array_equal(torch_ref.quant_dequant_act(_bf(x)).numpy(), orc.dequantize_act_fp8(q, s))
