"""``torch.ops.moe_mi355x.*`` on the GPU: every operator returns exactly what the direct
wrapper returns (same kernels, same bits), and ``torch.library.opcheck`` validates the schema
and the fake implementations against real runs."""

from __future__ import annotations

import pytest
import torch

from tests.helpers import gpu_weights

pytestmark = pytest.mark.gpu

E, H, I, K = 16, 256, 128, 4


def _inputs(dev, T, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
    wr = (torch.randn((E, H), generator=g, device=dev) * 0.05).to(torch.bfloat16)
    return x, wr


@pytest.mark.parametrize("T", [1, 37, 600])
def test_ops_equal_wrappers(pkg, dev, T):
    x, wr = _inputs(dev, T, seed=T)
    q13, s13, q2, s2 = gpu_weights(E, H, I, dev, seed=T)
    ids, w, logits = torch.ops.moe_mi355x.route(x, wr, K, True)
    r_logits, r_w, r_ids = pkg.route(x, wr, K, True, index_dtype=torch.int32)
    assert torch.equal(ids, r_ids) and torch.equal(w, r_w) and torch.equal(logits, r_logits)
    perm, tiles, counts, offsets, n_tiles = torch.ops.moe_mi355x.align(ids, E, 16)
    ref = pkg.align(ids, E, 16)
    for name, got in (("perm", perm), ("tiles", tiles), ("counts", counts), ("offsets", offsets),
                      ("n_tiles", n_tiles)):
        if name == "tiles":  # only the live rows are defined
            n = int(n_tiles.item())
            assert torch.equal(got[:n], ref[name][:n])
        else:
            assert torch.equal(got, ref[name]), name
    out = torch.ops.moe_mi355x.moe_fp8(x, ids, w, q13, s13, q2, s2)
    assert torch.equal(out, pkg.experts_fp8(x, ids, w, q13, s13, q2, s2))
    blk = torch.ops.moe_mi355x.moe_block_fp8(x.reshape(1, T, H), wr, K, True, q13, s13, q2, s2)
    assert blk.shape == (1, T, H)
    assert torch.equal(blk, pkg.moe_block_fp8(x.reshape(1, T, H), wr, K, q13, s13, q2, s2))
    torch.cuda.synchronize()


def test_opcheck(pkg, dev):
    x, wr = _inputs(dev, 40, seed=1)
    q13, s13, q2, s2 = gpu_weights(E, H, I, dev, seed=1)
    ids, w, _ = torch.ops.moe_mi355x.route(x, wr, K, True)
    checks = ("test_schema", "test_faketensor")
    torch.library.opcheck(torch.ops.moe_mi355x.route.default, (x, wr, K, True), test_utils=checks)
    torch.library.opcheck(torch.ops.moe_mi355x.align.default, (ids, E, 16), test_utils=checks)
    # torch's schema check multiplies the inputs to detect mutation, which float8_e4m3fn
    # tensors do not support: the FP8-weight operators get the fake-tensor check, and their
    # inputs are compared byte for byte before and after a call instead
    fp8_args = {"moe_fp8": (x, ids, w, q13, s13, q2, s2), "moe_block_fp8": (x, wr, K, True, q13, s13, q2, s2)}
    for name, args in fp8_args.items():
        op = getattr(torch.ops.moe_mi355x, name).default
        torch.library.opcheck(op, args, test_utils=("test_faketensor",))
        before = [a.view(torch.uint8).clone() for a in args if isinstance(a, torch.Tensor)]
        op(*args)
        after = [a.view(torch.uint8) for a in args if isinstance(a, torch.Tensor)]
        assert all(torch.equal(u, v) for u, v in zip(before, after)), name
    torch.cuda.synchronize()


def test_ops_trace_under_compile(pkg, dev):
    """A function around the block operator compiles with fullgraph=True (the fake
    implementation drives the trace; aot_eager runs the traced graph without codegen) and
    returns the eager result."""
    x, wr = _inputs(dev, 24, seed=2)
    q13, s13, q2, s2 = gpu_weights(E, H, I, dev, seed=2)

    def layer(h):
        return h + torch.ops.moe_mi355x.moe_block_fp8(h, wr, K, True, q13, s13, q2, s2)

    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    assert torch.equal(compiled(x), layer(x))
    torch.cuda.synchronize()
