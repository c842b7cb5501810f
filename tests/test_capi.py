"""The C-ABI library loads and exports every symbol include/moe_mi355x.h declares (CPU only).

Only host-side paths are called here: queries (sizes, version, error text) and argument
validation that returns before any HIP call.
"""

from __future__ import annotations

import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "moe_mi355x.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(moe_mi355x_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib(pkg):
    from inference_server_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        import __graft_entry__

        __graft_entry__._load_build_module().build()
    return _lib.load()


def test_header_declares_entry_points():
    names = _declared()
    for n in ["moe_mi355x_route", "moe_mi355x_topk_softmax", "moe_mi355x_align", "moe_mi355x_quantize_act_fp8",
              "moe_mi355x_quantize_weight_fp8", "moe_mi355x_experts_fp8", "moe_mi355x_block_fp8"]:
        assert n in names


def test_every_declared_symbol_is_exported(lib):
    for name in _declared():
        assert hasattr(lib, name), name
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)


def test_binding_covers_header(pkg):
    from inference_server_amd import _lib

    assert sorted(_lib.SIGNATURES) == _declared()


def test_host_queries(lib):
    assert lib.moe_mi355x_version() == (0 << 16) | 2
    assert lib.moe_mi355x_error_string(0) == b"success"
    assert b"workspace" in lib.moe_mi355x_error_string(-2)
    assert lib.moe_mi355x_align_max_tiles(8, 128, 16) == 8            # T=1, k=8: one tile per expert
    assert lib.moe_mi355x_align_max_tiles(32768, 128, 64) == 512 + 128
    assert lib.moe_mi355x_experts_workspace_bytes(64, 2048, 768, 128, 8) > 64 * 8 * 2048 * 2
    assert lib.moe_mi355x_experts_workspace_bytes(64, 2000, 768, 128, 8) == 0  # H not a multiple of 128
    assert lib.moe_mi355x_block_workspace_bytes(64, 2048, 768, 128, 8) > \
        lib.moe_mi355x_experts_workspace_bytes(64, 2048, 768, 128, 8)


def test_argument_validation_before_launch(lib):
    null = None
    # unsupported shapes -> MOE_ERR_INVALID_ARG (-1), no device work attempted
    assert lib.moe_mi355x_experts_fp8(null, null, 4, null, 4, 2000, 768, 128, 8, null, null, null, null, null,
                                      null, 0, null) == -1
    assert lib.moe_mi355x_experts_fp8(null, null, 3, null, 4, 2048, 768, 128, 8, null, null, null, null, null,
                                      null, 0, null) == -1
    assert lib.moe_mi355x_route(null, null, 4, 2048, 300, 8, 1, null, null, 4, null, null, 0, null) == -1
    assert lib.moe_mi355x_route(null, null, 4, 2048, 128, 0, 1, null, null, 4, null, null, 0, null) == -1
    assert lib.moe_mi355x_quantize_act_fp8(null, 4, 100, null, null, null) == -1
    assert lib.moe_mi355x_quantize_weight_fp8(null, 2, 1, 128, 128, null, null, null) == -1
    # T == 0 is a successful no-op
    assert lib.moe_mi355x_experts_fp8(null, null, 4, null, 0, 2048, 768, 128, 8, null, null, null, null, null,
                                      null, 0, null) == 0
    # null tensors with T > 0 are rejected
    assert lib.moe_mi355x_experts_fp8(null, null, 4, null, 1, 2048, 768, 128, 8, null, null, null, null, null,
                                      null, 0, null) == -1


def test_bf16_noalloc_and_numerics_queries(lib):
    """Host-side queries and argument checks of the bf16, no-allocation and sublayer entry points
    (no device work: every case returns before a launch)."""
    null = None
    fake = 0x10000  # a 16-byte-aligned address that is never dereferenced on these paths
    assert lib.moe_mi355x_experts_bf16_workspace_bytes(64, 2048, 768, 128, 8) > 64 * 8 * 2048 * 2
    assert lib.moe_mi355x_experts_bf16_workspace_bytes(64, 2000, 768, 128, 8) == 0
    assert lib.moe_mi355x_block_bf16_workspace_bytes(64, 2048, 768, 128, 8) > \
        lib.moe_mi355x_experts_bf16_workspace_bytes(64, 2048, 768, 128, 8)
    assert lib.moe_mi355x_moe_sublayer_workspace_bytes(64, 2048, 768, 128, 8) > \
        lib.moe_mi355x_block_workspace_bytes(64, 2048, 768, 128, 8)
    # bf16 experts: unsupported shape, T == 0 no-op, null tensors
    assert lib.moe_mi355x_experts_bf16(null, null, 4, null, 4, 2000, 768, 128, 8, null, null, null, null, 0,
                                       null) == -1
    assert lib.moe_mi355x_experts_bf16(null, null, 4, null, 0, 2048, 768, 128, 8, null, null, null, null, 0,
                                       null) == 0
    assert lib.moe_mi355x_experts_bf16(null, null, 4, null, 1, 2048, 768, 128, 8, null, null, null, null, 0,
                                       null) == -1
    assert lib.moe_mi355x_block_bf16(null, null, 1, 2048, 768, 128, 8, 1, null, null, null, null, null, 4, null,
                                     null, 0, null) == -1
    # no-allocation block: 64 MiB of scratch; a call needing more returns MOE_ERR_SCRATCH (-4)
    assert lib.moe_mi355x_block_fp8_noalloc_scratch_bytes() == 64 << 20
    assert lib.moe_mi355x_block_workspace_bytes(4096, 4096, 1536, 128, 8) > 64 << 20
    assert lib.moe_mi355x_block_fp8_noalloc(fake, fake, 4096, 4096, 1536, 128, 8, 1, fake, fake, fake, fake, fake,
                                            null, null, 4, null, null) == -4
    assert b"scratch" in lib.moe_mi355x_error_string(-4)
    assert lib.moe_mi355x_block_fp8_noalloc(null, null, 1, 2048, 768, 128, 8, 1, null, null, null, null, null,
                                            null, null, 4, null, null) == -1
    # tile height (low 16 bits of the numerics key): 16-row up to 8 pairs per expert, then the
    # 128-row LDS-tiled kernels (FP8 and bf16 alike at the 30B shape)
    for fp8 in (1, 0):
        bm = {t: int(lib.moe_mi355x_block_numerics_key(t, 2048, 768, 128, 8, fp8)) & 0xFFFF
              for t in (1, 128, 129, 256, 257, 4096)}
        assert bm == {1: 16, 128: 16, 129: 128, 256: 128, 257: 128, 4096: 128}, (fp8, bm)
    # bf16 shapes the 128-row kernel cannot take: 32-row tiles up to 16 pairs per expert
    assert int(lib.moe_mi355x_block_numerics_key(37, 384, 256, 20, 5, 0)) & 0xFFFF == 32
    # FP8 shapes the 128-row kernel cannot take: 32-row tiles up to 16 pairs per expert, 64 above
    assert int(lib.moe_mi355x_block_numerics_key(30, 384, 256, 6, 3, 1)) & 0xFFFF == 32
    assert int(lib.moe_mi355x_block_numerics_key(100, 384, 256, 6, 3, 1)) & 0xFFFF == 64
    # bf16 above 16 pairs per expert with H % 256 != 0: 64-row tiles
    assert int(lib.moe_mi355x_block_numerics_key(100, 384, 256, 8, 2, 0)) & 0xFFFF == 64


def test_linear_bf16_queries_and_argument_checks(lib):
    """The decode-step projection entry point: workspace query (the K split's fp32 partials) and
    the checks that return before a launch."""
    null = None
    fake = 0x10000  # 16-byte aligned, never dereferenced on these paths
    # batch 128 q/k/v: four K chunks of fp32 partials; one row: no split below 256-deep chunks
    assert lib.moe_mi355x_linear_bf16_workspace_bytes(128, 5120, 2048) == 4 * 128 * 5120 * 4
    assert lib.moe_mi355x_linear_bf16_workspace_bytes(300, 64, 128) == 0
    assert lib.moe_mi355x_linear_bf16_workspace_bytes(8, 100, 2048) == 0   # N not a multiple of 64
    # unsupported shapes -> MOE_ERR_INVALID_ARG (-1)
    assert lib.moe_mi355x_linear_bf16(fake, fake, 8, 100, 2048, fake, fake, 1 << 20, null) == -1
    assert lib.moe_mi355x_linear_bf16(fake, fake, 8, 128, 200, fake, fake, 1 << 20, null) == -1
    assert lib.moe_mi355x_linear_bf16(fake, fake, -1, 128, 256, fake, fake, 1 << 20, null) == -1
    # M == 0 is a successful no-op; null tensors with M > 0 are rejected
    assert lib.moe_mi355x_linear_bf16(null, null, 0, 128, 256, null, null, 0, null) == 0
    assert lib.moe_mi355x_linear_bf16(null, fake, 8, 128, 256, fake, fake, 1 << 20, null) == -1
    # misaligned operand -> MOE_ERR_ALIGNMENT, missing workspace for a split -> MOE_ERR_WORKSPACE
    assert lib.moe_mi355x_linear_bf16(fake + 2, fake, 8, 5120, 2048, fake, fake, 1 << 24, null) == -3
    assert lib.moe_mi355x_linear_bf16(fake, fake, 128, 5120, 2048, fake, null, 0, null) == -2


def test_paged_attention_queries_and_argument_checks(lib):
    """Paged attention: the workspace query (fp32 partial outputs and (max, sum) pairs per
    (sequence, q head, split)) and the checks that return before a launch, including batches whose
    decode grid would not fit the kernel's 32-bit item indices."""
    null = None
    fake = 0x10000  # 16-byte aligned, never dereferenced on these paths
    # config 5: 128 sequences, 32 q / 4 kv heads, 512 pages -> 64-page splits, 8 per sequence
    parts = 128 * 32 * 8
    align = lambda n: (n + 255) // 256 * 256
    assert lib.moe_mi355x_paged_attn_workspace_bytes(128, 32, 4, 512) == align(parts * 128 * 4) + align(parts * 2 * 4)
    # a small batch shortens the splits (down to 8 pages) so that the grid fills more of the chip:
    # one sequence of 64 pages -> 8 splits per head instead of 1
    assert lib.moe_mi355x_paged_attn_workspace_bytes(1, 32, 4, 64) == align(256 * 128 * 4) + align(256 * 2 * 4)
    # invalid shapes and grids past 2^31 items -> 0 bytes, MOE_ERR_INVALID_ARG (-1)
    assert lib.moe_mi355x_paged_attn_workspace_bytes(128, 30, 4, 512) == 0
    assert lib.moe_mi355x_paged_attn_workspace_bytes(1 << 20, 64, 8, 1 << 16) == 0
    args = lambda B, Hq, Hkv, hd, ps, mp: (fake, fake, fake, fake, fake, B, Hq, Hkv, hd, ps, mp, 1 << 20,
                                             0.088, fake, fake, 1 << 30, null)
    assert lib.moe_mi355x_paged_attn_decode(*args(1 << 20, 64, 8, 128, 16, 1 << 16)) == -1
    assert lib.moe_mi355x_paged_attn_decode(*args(4, 32, 4, 64, 16, 8)) == -1    # head_dim 64
    assert lib.moe_mi355x_paged_attn_decode(*args(4, 32, 4, 128, 32, 8)) == -1   # page size 32
    assert lib.moe_mi355x_paged_attn_decode(*args(4, 64, 2, 128, 16, 8)) == -1   # 32 q heads per kv head
    # misaligned q -> MOE_ERR_ALIGNMENT (-3); a short workspace -> MOE_ERR_WORKSPACE (-2)
    a = list(args(4, 32, 4, 128, 16, 8))
    a[0] = fake + 2
    assert lib.moe_mi355x_paged_attn_decode(*a) == -3
    a = list(args(4, 32, 4, 128, 16, 8))
    a[15] = 16
    assert lib.moe_mi355x_paged_attn_decode(*a) == -2


def test_oversized_grids_are_rejected_before_launch(lib):
    """Shapes whose 1-D launch grid would pass 2^31 workgroups return MOE_ERR_INVALID_ARG (-1)
    instead of launching a truncated grid (no device call is made on these paths)."""
    fake = 0x10000
    big = (1 << 31) - 1
    assert lib.moe_mi355x_quantize_act_fp8(fake, big, 4096, fake, fake, None) == -1
    assert lib.moe_mi355x_quantize_weight_fp8(fake, 0, big, 4096, 4096, fake, fake, None) == -1
    assert lib.moe_mi355x_qk_norm_rope_append(fake, fake, fake, fake, fake, big, 64, 4, 128, 1e-6, fake, fake, fake,
                                              fake, 16, 8, 1 << 20, None) == -1
