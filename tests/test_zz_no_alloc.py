"""``moe_mi355x_block_fp8_noalloc``: the block forward with no workspace argument and no allocation
(its scratch is a fixed device array inside the library), called through the C ABI.

Its outputs (block output, logits, ids, weights) must equal ``moe_mi355x_block_fp8``'s bit for bit
on two calls in a row, the second with a smaller batch, so that whatever the first call left in the
shared scratch cannot leak into the second.  A call that needs more scratch than the array holds is
refused with MOE_ERR_SCRATCH before anything is launched (a host-side check, tested on the CPU).
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from tests.helpers import gpu_weights

MOE_ERR_SCRATCH = -4


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _call_pair(lib, x, wr, k, weights, dev):
    """(out, logits, ids, w) from the workspace entry point and from the no-allocation one."""
    q13, s13, q2, s2 = weights
    T, H = x.shape
    E = wr.shape[0]
    I = q2.shape[2]
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    res = []
    for noalloc in (False, True):
        out = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device=dev)
        logits = torch.full((T, E), float("nan"), dtype=torch.bfloat16, device=dev)
        ids = torch.full((T, k), -7, dtype=torch.int32, device=dev)
        w = torch.full((T, k), float("nan"), dtype=torch.bfloat16, device=dev)
        common = (_ptr(x), _ptr(wr), T, H, I, E, k, 1, _ptr(q13), _ptr(s13), _ptr(q2), _ptr(s2), _ptr(out),
                  _ptr(logits), _ptr(ids), 4, _ptr(w))
        if noalloc:
            rc = lib.moe_mi355x_block_fp8_noalloc(*common, stream)
        else:
            nbytes = lib.moe_mi355x_block_workspace_bytes(T, H, I, E, k)
            ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
            rc = lib.moe_mi355x_block_fp8(*common, _ptr(ws), ctypes.c_size_t(ws.numel()), stream)
        assert rc == 0, (noalloc, rc)
        torch.cuda.synchronize(dev)
        res.append((out, logits, ids, w))
    return res


@pytest.mark.gpu
@pytest.mark.parametrize("H,I,T1,T2", [(2048, 768, 300, 40), (4096, 1536, 64, 1)])
def test_noalloc_block_equals_workspace_block(pkg, dev, H, I, T1, T2):
    """Qwen3-30B-A3B shape (300 tokens: the 128-row LDS-tiled GEMMs, then 40: 16-row tiles) and
    Qwen3-235B-A22B shape (decode 64, then 1 token)."""
    lib = pkg._lib.load()
    E, k = 128, 8
    weights = gpu_weights(E, H, I, dev, seed=31)
    g = torch.Generator(device=dev).manual_seed(32)
    wr = (torch.randn((E, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    for T in (T1, T2):  # the second call is smaller: no stale scratch may reach its results
        x = torch.randn((T, H), generator=g, device=dev).to(torch.bfloat16)
        (o_ref, lg_ref, id_ref, w_ref), (o, lg, ids, w) = _call_pair(lib, x, wr, k, weights, dev)
        assert torch.equal(ids, id_ref), T
        assert torch.equal(lg.view(torch.int16), lg_ref.view(torch.int16)), T
        assert torch.equal(w.view(torch.int16), w_ref.view(torch.int16)), T
        assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16)), T
        assert torch.isfinite(o.float()).all()


def test_noalloc_refuses_calls_beyond_its_scratch(pkg):
    """A batch whose workspace exceeds the fixed array returns MOE_ERR_SCRATCH before any HIP call
    (the pointers are placeholders: nothing is dereferenced)."""
    lib = pkg._lib.load()
    cap = lib.moe_mi355x_block_fp8_noalloc_scratch_bytes()
    assert cap == 64 << 20
    H, I, E, k = 2048, 768, 128, 8
    T = 4096
    assert lib.moe_mi355x_block_workspace_bytes(T, H, I, E, k) > cap
    p = ctypes.c_void_p(1 << 20)  # 16-byte aligned placeholder
    rc = lib.moe_mi355x_block_fp8_noalloc(p, p, T, H, I, E, k, 1, p, p, p, p, p, None, None, 4, None, None)
    assert rc == MOE_ERR_SCRATCH
    assert b"scratch" in lib.moe_mi355x_error_string(MOE_ERR_SCRATCH)
