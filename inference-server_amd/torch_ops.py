"""The hot path's entry points as torch operators, ``torch.ops.moe_mi355x.*``.

Each operator runs the matching wrapper in ``kernels`` (argument checks, then the HIP kernels
of ``libmoe_mi355x.so`` through the C ABI) and has a fake implementation that derives output
shapes and dtypes from input metadata alone, so the operators trace under FakeTensorMode and
``torch.compile`` without touching the device.

  route(x bf16[T,H], w_router bf16[E,H], k, renorm)
      -> (ids int32[T,k], weights bf16[T,k], logits bf16[T,E])
      Qwen3MoeTopKRouter.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267
  align(ids int32|int64[T,k], num_experts, block_m)
      -> (perm int32[S], tiles int32[max_tiles,4], counts int32[E], offsets int32[E+1],
          n_tiles int32[1])
      the sort / histc / cumsum of TF/integrations/moe.py:389-403, plus the tile list
  moe_fp8(x bf16[T,H], ids int32|int64[T,k], weights bf16[T,k], w13, s13, w2, s2) -> bf16[T,H]
      fp8_grouped_mm_experts_forward, TF/integrations/finegrained_fp8.py:498-589
  moe_block_fp8(x bf16[...,H], w_router, k, renorm, w13, s13, w2, s2) -> bf16[...,H]
      Qwen3MoeSparseMoeBlock.forward, modeling_qwen3_moe.py:276-281
  moe_bf16(x bf16[T,H], ids, weights, w13 bf16[E,2I,H], w2 bf16[E,H,I]) -> bf16[T,H]
      grouped_mm_experts_forward on bf16 weights, TF/integrations/moe.py:377-478
  moe_block_bf16(x bf16[...,H], w_router, k, renorm, w13, w2) -> bf16[...,H]
      the block on a bf16 checkpoint

Weights: w13 e4m3fn [E,2I,H] with s13 fp32 [E,2I/128,H/128]; w2 e4m3fn [E,H,I] with s2 fp32
[E,H/128,I/128].  The operators are registered when the package is imported (once per process).
"""

from __future__ import annotations

import torch

from . import kernels

NAMESPACE = "moe_mi355x"


def align_max_tiles(S, num_experts: int, block_m: int):
    """Rows of the tile table for S pairs (``moe_mi355x_align_max_tiles``, align.hip): every
    expert's last tile may be partial, so S / block_m full tiles plus one per hit expert."""
    if S <= 0:
        return 1
    return max(S // block_m + min(S, num_experts), 1)


def _define() -> None:
    lib = f"{NAMESPACE}::"

    @torch.library.custom_op(lib + "route", mutates_args=())
    def route(x: torch.Tensor, w_router: torch.Tensor, k: int, renorm: bool) -> tuple[torch.Tensor, torch.Tensor,
                                                                                      torch.Tensor]:
        logits, weights, ids = kernels.route(x, w_router, k, renorm, index_dtype=torch.int32)
        return ids, weights, logits

    @route.register_fake
    def _(x, w_router, k, renorm):
        E, H = w_router.shape
        T = x.numel() // H
        return (x.new_empty((T, k), dtype=torch.int32), x.new_empty((T, k), dtype=torch.bfloat16),
                x.new_empty((T, E), dtype=torch.bfloat16))

    @torch.library.custom_op(lib + "align", mutates_args=())
    def align(ids: torch.Tensor, num_experts: int, block_m: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                          torch.Tensor, torch.Tensor]:
        out = kernels.align(ids, num_experts, block_m)
        return out["perm"], out["tiles"], out["counts"], out["offsets"], out["n_tiles"]

    @align.register_fake
    def _(ids, num_experts, block_m):
        S = ids.numel()
        i32 = torch.int32
        return (ids.new_empty((S,), dtype=i32), ids.new_empty((align_max_tiles(S, num_experts, block_m), 4), dtype=i32),
                ids.new_empty((num_experts,), dtype=i32), ids.new_empty((num_experts + 1,), dtype=i32),
                ids.new_empty((1,), dtype=i32))

    @torch.library.custom_op(lib + "moe_fp8", mutates_args=())
    def moe_fp8(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, w13: torch.Tensor, s13: torch.Tensor,
                w2: torch.Tensor, s2: torch.Tensor) -> torch.Tensor:
        return kernels.experts_fp8(x, ids, weights, w13, s13, w2, s2)

    @moe_fp8.register_fake
    def _(x, ids, weights, w13, s13, w2, s2):
        return x.new_empty((x.shape[0], w2.shape[1]), dtype=torch.bfloat16)

    @torch.library.custom_op(lib + "moe_block_fp8", mutates_args=())
    def moe_block_fp8(x: torch.Tensor, w_router: torch.Tensor, k: int, renorm: bool, w13: torch.Tensor,
                      s13: torch.Tensor, w2: torch.Tensor, s2: torch.Tensor) -> torch.Tensor:
        return kernels.moe_block_fp8(x, w_router, k, w13, s13, w2, s2, norm_topk_prob=renorm)

    @moe_block_fp8.register_fake
    def _(x, w_router, k, renorm, w13, s13, w2, s2):
        return x.new_empty(x.shape, dtype=torch.bfloat16)

    @torch.library.custom_op(lib + "moe_bf16", mutates_args=())
    def moe_bf16(x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor, w13: torch.Tensor,
                 w2: torch.Tensor) -> torch.Tensor:
        return kernels.experts_bf16(x, ids, weights, w13, w2)

    @moe_bf16.register_fake
    def _(x, ids, weights, w13, w2):
        return x.new_empty((x.shape[0], w2.shape[1]), dtype=torch.bfloat16)

    @torch.library.custom_op(lib + "moe_block_bf16", mutates_args=())
    def moe_block_bf16(x: torch.Tensor, w_router: torch.Tensor, k: int, renorm: bool, w13: torch.Tensor,
                       w2: torch.Tensor) -> torch.Tensor:
        return kernels.moe_block_bf16(x, w_router, k, w13, w2, norm_topk_prob=renorm)

    @moe_block_bf16.register_fake
    def _(x, w_router, k, renorm, w13, w2):
        return x.new_empty(x.shape, dtype=torch.bfloat16)


def registered() -> bool:
    return hasattr(torch.ops, NAMESPACE) and hasattr(getattr(torch.ops, NAMESPACE), "moe_block_bf16")


def register() -> None:
    """Define the operators unless this process already has them (another copy of the package
    may have been imported under a different module name)."""
    if not registered():
        _define()


register()
