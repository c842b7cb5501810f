"""The block forward captured in a HIP graph (GPU).

The decode step is launch-bound at small batches, so callers capture it once per batch
bucket and replay it.  The path enqueues kernels only (no memsets, no host syncs, no
allocation inside the library), so capture needs nothing special.  Every replay is
checked against the eager result for the same inputs, with eager work and
synchronisations between replays.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import moe_oracle as orc
from tests.helpers import gpu_weights, to_bf16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T", [1, 8, 64, 200, 300])  # 16-, 16-, 16-, 32- and 128-row tiles
def test_block_graph_replays_match_eager(pkg, dev, T):
    E, H, I, k = 128, 2048, 768, 8
    q13, s13, q2, s2 = gpu_weights(E, H, I, dev, seed=2)
    g = torch.Generator(device=dev).manual_seed(3)
    wr = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    rng = np.random.default_rng(40 + T)
    xs = [to_bf16(orc.gen_normal_bf16(rng, (T, H)), dev) for _ in range(4)]
    eager = [pkg.moe_block_fp8(x, wr, k, q13, s13, q2, s2) for x in xs]
    torch.cuda.synchronize()

    x_static = xs[0].clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):  # warm the allocator on the capture stream
        pkg.moe_block_fp8(x_static, wr, k, q13, s13, q2, s2)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = pkg.moe_block_fp8(x_static, wr, k, q13, s13, q2, s2)

    for rep in range(3):
        for i, x in enumerate(xs):
            x_static.copy_(x)
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out_static, eager[i]), f"replay {rep} input {i} differs from eager"
            # eager work between replays must not disturb the graph's buffers
            again = pkg.moe_block_fp8(xs[(i + 1) % len(xs)], wr, k, q13, s13, q2, s2)
            torch.cuda.synchronize()
            assert torch.equal(again, eager[(i + 1) % len(xs)])


def test_graphed_block_buckets_match_eager(pkg, dev):
    """MI355XGraphedMoeBlock: batches padded up to their bucket and replayed from a captured
    graph give the eager block's output for the real rows."""
    E, H, I, k = 64, 512, 256, 8
    block = pkg.MI355XSparseMoeBlock(E, H, I, k, device=dev)
    g = torch.Generator(device=dev).manual_seed(11)
    with torch.no_grad():
        block.gate.weight.copy_((torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16))
        q13, s13, q2, s2 = gpu_weights(E, H, I, dev, seed=4)
        block.experts.gate_up_proj.copy_(q13)
        block.experts.gate_up_proj_scale_inv.copy_(s13)
        block.experts.down_proj.copy_(q2)
        block.experts.down_proj_scale_inv.copy_(s2)
    graphed = pkg.MI355XGraphedMoeBlock(block, buckets=(1, 4, 16))
    rng = np.random.default_rng(9)
    for rep in range(2):
        for T in (1, 3, 4, 9, 16, 20):  # 20: above the largest bucket, eager
            x = to_bf16(orc.gen_normal_bf16(rng, (T, H)), dev).reshape(1, T, H)
            want = block(x)
            got = graphed(x)
            torch.cuda.synchronize()
            assert got.shape == want.shape
            # padding rows change nothing in the real rows' routing or experts
            assert torch.equal(got, want), f"rep {rep} T={T}"


def _random_block(pkg, dev, E, H, I, k, seed, experts_dtype=torch.float8_e4m3fn):
    block = pkg.MI355XSparseMoeBlock(E, H, I, k, device=dev, experts_dtype=experts_dtype)
    g = torch.Generator(device=dev).manual_seed(seed)
    with torch.no_grad():
        block.gate.weight.copy_((torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16))
        if experts_dtype == torch.bfloat16:
            block.experts.gate_up_proj.copy_((torch.randn((E, 2 * I, H), generator=g, device=dev) * 0.02).to(torch.bfloat16))
            block.experts.down_proj.copy_((torch.randn((E, H, I), generator=g, device=dev) * 0.02).to(torch.bfloat16))
        else:
            q13, s13, q2, s2 = gpu_weights(E, H, I, dev, seed=seed + 1)
            block.experts.gate_up_proj.copy_(q13)
            block.experts.gate_up_proj_scale_inv.copy_(s13)
            block.experts.down_proj.copy_(q2)
            block.experts.down_proj_scale_inv.copy_(s2)
    return block


def test_graphed_buckets_across_the_h_quantisation_switches(pkg, dev):
    """I = 1536 > 1024: the h quantisation moves with the batch (routed one-row slots with the
    gate_up hand-off up to 4 tokens here, expert buckets with the hand-off up to S = 2 E = 32
    pairs, then a quant_h launch), and the buckets requested (2, 6, 12) straddle every switch:
    padded replays equal eager bit for bit."""
    E, H, I, k = 16, 256, 1536, 4
    block = _random_block(pkg, dev, E, H, I, k, seed=21)
    graphed = pkg.MI355XGraphedMoeBlock(block, buckets=(2, 6, 12))
    rng = np.random.default_rng(12)
    for rep in range(2):
        for T in (1, 2, 3, 4, 5, 6, 7, 8, 9, 12):
            x = to_bf16(orc.gen_normal_bf16(rng, (T, H)), dev).reshape(1, T, H)
            want = block(x)
            got = graphed(x)
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"rep {rep} T={T}"


def test_graphed_bf16_block_padded_bucket(pkg, dev):
    """bf16 experts: bucket 2 fed one token (the one-token block combines in a separate launch,
    larger ones inside the down GEMM): the padded replay equals eager bit for bit."""
    E, H, I, k = 32, 512, 256, 8
    block = _random_block(pkg, dev, E, H, I, k, seed=31, experts_dtype=torch.bfloat16)
    graphed = pkg.MI355XGraphedMoeBlock(block, buckets=(2, 8))
    rng = np.random.default_rng(13)
    for rep in range(2):
        for T in (1, 2, 5, 8):
            x = to_bf16(orc.gen_normal_bf16(rng, (T, H)), dev).reshape(1, T, H)
            want = block(x)
            got = graphed(x)
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"rep {rep} T={T}"


def test_wrappers_launch_on_the_current_stream(pkg, dev):
    from importlib import import_module
    kernels = import_module(pkg.__name__ + ".kernels")
    x = torch.zeros(4, device=dev)
    assert kernels._stream(x) == torch.cuda.current_stream(dev).cuda_stream
    side = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(side):
        assert kernels._stream(x) == side.cuda_stream
