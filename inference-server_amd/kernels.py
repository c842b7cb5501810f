"""torch-facing wrappers of the C-ABI entry points.

torch supplies device memory and the current HIP stream; every computation runs in
the HIP kernels of ``libmoe_mi355x.so``.  Tensors must live on a ROCm device, be
contiguous and carry the dtypes listed per op; violations raise ``ValueError`` /
``TypeError`` before anything is launched.  Workspaces are fresh ``torch.empty``
buffers from the caching allocator, so calls on different streams never share one.
"""

from __future__ import annotations

import torch

from . import _lib

FP8 = torch.float8_e4m3fn
BLOCK = 128


def _stream(t: torch.Tensor) -> int:
    # The raw handle of the current stream on t's device; the same value as
    # torch.cuda.current_stream(t.device).cuda_stream without building a Stream object.
    return torch._C._cuda_getCurrentRawStream(t.device.index)


def _need(t: torch.Tensor, name: str, dtypes, ndim: int | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if not isinstance(dtypes, (tuple, list)):
        dtypes = (dtypes,)
    if t.dtype not in dtypes:
        raise TypeError(f"{name} must have dtype {' or '.join(map(str, dtypes))}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name} must be {ndim}-D, got shape {tuple(t.shape)}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a ROCm GPU device, got {t.device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _ws(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def _id_bytes(ids: torch.Tensor) -> int:
    if ids.dtype == torch.int64:
        return 8
    if ids.dtype == torch.int32:
        return 4
    raise TypeError(f"expert ids must be int32 or int64, got {ids.dtype}")


# ---------------------------------------------------------------------------
# routing
# ---------------------------------------------------------------------------


def route(hidden_states: torch.Tensor, router_weight: torch.Tensor, top_k: int, norm_topk_prob: bool = True,
          index_dtype: torch.dtype = torch.int64):
    """``Qwen3MoeTopKRouter.forward`` (TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267).

    Returns ``(router_logits bf16 [T,E], router_scores bf16 [T,k], router_indices [T,k])``,
    the reference's return order.  Ties are broken towards the lower expert id.
    """
    _need(router_weight, "router_weight", torch.bfloat16, 2)
    E, H = router_weight.shape
    x = hidden_states.reshape(-1, H)
    _need(x, "hidden_states", torch.bfloat16, 2)
    if x.device != router_weight.device:
        raise ValueError("hidden_states and router_weight must be on the same device")
    if not 1 <= top_k <= min(E, 32):
        raise ValueError(f"top_k must be in [1, min(E, 32)], got {top_k}")
    T = x.shape[0]
    lib = _lib.load()
    logits = torch.empty((T, E), dtype=torch.bfloat16, device=x.device)
    ids = torch.empty((T, top_k), dtype=index_dtype, device=x.device)
    w = torch.empty((T, top_k), dtype=torch.bfloat16, device=x.device)
    ws = _ws(lib.moe_mi355x_route_workspace_bytes(T, H, E), x.device)
    _lib.check(lib.moe_mi355x_route(x.data_ptr(), router_weight.data_ptr(), T, H, E, top_k, int(norm_topk_prob),
                                    logits.data_ptr(), ids.data_ptr(), _id_bytes(ids), w.data_ptr(),
                                    ws.data_ptr(), ws.numel(), _stream(x)), "moe_mi355x_route")
    return logits, w, ids


def topk_softmax(router_logits: torch.Tensor, top_k: int, norm_topk_prob: bool = True,
                 index_dtype: torch.dtype = torch.int64):
    """softmax(fp32) -> top-k -> renormalise -> bf16 (modeling_qwen3_moe.py:261-266).

    Returns ``(router_scores bf16 [T,k], router_indices [T,k])``.
    """
    _need(router_logits, "router_logits", torch.bfloat16, 2)
    T, E = router_logits.shape
    if not 1 <= top_k <= min(E, 32):
        raise ValueError(f"top_k must be in [1, min(E, 32)], got {top_k}")
    ids = torch.empty((T, top_k), dtype=index_dtype, device=router_logits.device)
    w = torch.empty((T, top_k), dtype=torch.bfloat16, device=router_logits.device)
    lib = _lib.load()
    _lib.check(lib.moe_mi355x_topk_softmax(router_logits.data_ptr(), T, E, top_k, int(norm_topk_prob),
                                           ids.data_ptr(), _id_bytes(ids), w.data_ptr(), _stream(router_logits)),
               "moe_mi355x_topk_softmax")
    return w, ids


# ---------------------------------------------------------------------------
# sort / align
# ---------------------------------------------------------------------------


def align(top_k_index: torch.Tensor, num_experts: int, block_m: int = 16) -> dict:
    """Stable expert sort, counts, offsets and tile list (TF/integrations/moe.py:389-403).

    Returns a dict with ``perm`` int32 [S], ``counts`` int32 [E], ``offsets`` int32 [E+1]
    (exclusive), ``tiles`` int32 [max_tiles, 4] and ``n_tiles`` int32 [1].
    """
    _need(top_k_index, "top_k_index", (torch.int32, torch.int64))
    if top_k_index.dim() != 2:
        raise ValueError("top_k_index must be [T, k]")
    T, k = top_k_index.shape
    if not 1 <= num_experts <= 256:
        raise ValueError("num_experts must be in [1, 256]")
    S = T * k
    lib = _lib.load()
    dev = top_k_index.device
    max_tiles = max(lib.moe_mi355x_align_max_tiles(S, num_experts, block_m), 1)
    out = {
        "perm": torch.empty(S, dtype=torch.int32, device=dev),
        "counts": torch.empty(num_experts, dtype=torch.int32, device=dev),
        "offsets": torch.empty(num_experts + 1, dtype=torch.int32, device=dev),
        "tiles": torch.empty((max_tiles, 4), dtype=torch.int32, device=dev),
        "n_tiles": torch.empty(1, dtype=torch.int32, device=dev),
    }
    ws = _ws(lib.moe_mi355x_align_workspace_bytes(S, num_experts), dev)
    _lib.check(lib.moe_mi355x_align(top_k_index.data_ptr(), _id_bytes(top_k_index), T, k, num_experts, block_m,
                                    out["perm"].data_ptr(), out["counts"].data_ptr(), out["offsets"].data_ptr(),
                                    out["tiles"].data_ptr(), out["n_tiles"].data_ptr(), ws.data_ptr(), ws.numel(),
                                    _stream(top_k_index)), "moe_mi355x_align")
    return out


# ---------------------------------------------------------------------------
# quantisation
# ---------------------------------------------------------------------------


def quantize_act_fp8(x: torch.Tensor):
    """Per-row, per-128-column dynamic e4m3 quantisation. Returns (q fp8 [R,C], scales fp32 [R,C/128])."""
    _need(x, "x", torch.bfloat16, 2)
    R, C = x.shape
    if C % BLOCK:
        raise ValueError(f"columns must be a multiple of {BLOCK}")
    q = torch.empty((R, C), dtype=FP8, device=x.device)
    s = torch.empty((R, C // BLOCK), dtype=torch.float32, device=x.device)
    _lib.check(_lib.load().moe_mi355x_quantize_act_fp8(x.data_ptr(), R, C, q.data_ptr(), s.data_ptr(),
                                                       _stream(x)), "moe_mi355x_quantize_act_fp8")
    return q, s


def quantize_weight_fp8(w: torch.Tensor):
    """128x128 block weight quantisation, ``Fp8Quantize._quantize_one``
    (TF/integrations/finegrained_fp8.py:903-941).  w: [..., N, K] bf16 or fp32.
    Returns (q fp8 [..., N, K], scale_inv fp32 [..., N/128, K/128])."""
    _need(w, "w", (torch.bfloat16, torch.float32))
    if w.dim() < 2:
        raise ValueError("w must be at least 2-D")
    *lead, N, K = w.shape
    if N % BLOCK or K % BLOCK:
        raise ValueError(f"weight dims must be multiples of {BLOCK}")
    B = 1
    for d in lead:
        B *= d
    q = torch.empty(w.shape, dtype=FP8, device=w.device)
    s = torch.empty((*lead, N // BLOCK, K // BLOCK), dtype=torch.float32, device=w.device)
    _lib.check(_lib.load().moe_mi355x_quantize_weight_fp8(w.data_ptr(), 0 if w.dtype == torch.bfloat16 else 1,
                                                          B, N, K, q.data_ptr(), s.data_ptr(), _stream(w)),
               "moe_mi355x_quantize_weight_fp8")
    return q, s


# ---------------------------------------------------------------------------
# experts / block
# ---------------------------------------------------------------------------


def _check_expert_weights(w13, s13, w2, s2):
    _need(w13, "gate_up_proj", FP8, 3)
    _need(w2, "down_proj", FP8, 3)
    _need(s13, "gate_up_proj_scale_inv", torch.float32, 3)
    _need(s2, "down_proj_scale_inv", torch.float32, 3)
    E, I2, H = w13.shape
    I = I2 // 2
    if I2 % 2 or I % BLOCK or H % BLOCK:
        raise ValueError(f"gate_up_proj must be [E, 2I, H] with I, H multiples of {BLOCK}")
    if tuple(w2.shape) != (E, H, I):
        raise ValueError(f"down_proj must be [E, H, I] = {(E, H, I)}, got {tuple(w2.shape)}")
    if tuple(s13.shape) != (E, I2 // BLOCK, H // BLOCK) or tuple(s2.shape) != (E, H // BLOCK, I // BLOCK):
        raise ValueError("scale_inv tensors must be [E, N/128, K/128] (128x128 blocks)")
    if H > 4096 or I > 4096 or not 1 <= E <= 256:
        raise ValueError("supported shapes: H, I <= 4096 and 1 <= E <= 256")
    return E, H, I


def experts_fp8(hidden_states, top_k_index, top_k_weights, gate_up_proj, gate_up_proj_scale_inv, down_proj,
                down_proj_scale_inv):
    """FP8 block-scaled experts, ``fp8_grouped_mm_experts_forward``
    (TF/integrations/finegrained_fp8.py:498-589).  Returns bf16 [T, H]."""
    E, H, I = _check_expert_weights(gate_up_proj, gate_up_proj_scale_inv, down_proj, down_proj_scale_inv)
    _need(hidden_states, "hidden_states", torch.bfloat16, 2)
    _need(top_k_index, "top_k_index", (torch.int32, torch.int64), 2)
    _need(top_k_weights, "top_k_weights", torch.bfloat16, 2)
    T = hidden_states.shape[0]
    if hidden_states.shape[1] != H:
        raise ValueError(f"hidden_states must be [T, {H}]")
    if top_k_index.shape[0] != T or tuple(top_k_weights.shape) != tuple(top_k_index.shape):
        raise ValueError("top_k_index and top_k_weights must both be [T, k]")
    k = top_k_index.shape[1]
    if not 1 <= k <= min(E, 32):
        raise ValueError("k must be in [1, min(E, 32)]")
    lib = _lib.load()
    out = torch.empty((T, H), dtype=torch.bfloat16, device=hidden_states.device)
    ws = _ws(lib.moe_mi355x_experts_workspace_bytes(T, H, I, E, k), hidden_states.device)
    _lib.check(lib.moe_mi355x_experts_fp8(hidden_states.data_ptr(), top_k_index.data_ptr(), _id_bytes(top_k_index),
                                          top_k_weights.data_ptr(), T, H, I, E, k, gate_up_proj.data_ptr(),
                                          gate_up_proj_scale_inv.data_ptr(), down_proj.data_ptr(),
                                          down_proj_scale_inv.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(),
                                          _stream(hidden_states)), "moe_mi355x_experts_fp8")
    return out


def moe_block_fp8(hidden_states, router_weight, top_k, gate_up_proj, gate_up_proj_scale_inv, down_proj,
                  down_proj_scale_inv, norm_topk_prob=True, return_routing=False, index_dtype=torch.int64):
    """Router + FP8 experts in one call (``Qwen3MoeSparseMoeBlock.forward``,
    TF/models/qwen3_moe/modeling_qwen3_moe.py:276-281).  hidden_states: [..., H] bf16."""
    E, H, I = _check_expert_weights(gate_up_proj, gate_up_proj_scale_inv, down_proj, down_proj_scale_inv)
    _need(router_weight, "router_weight", torch.bfloat16, 2)
    if tuple(router_weight.shape) != (E, H):
        raise ValueError(f"router_weight must be [{E}, {H}]")
    shape = hidden_states.shape
    x = hidden_states.reshape(-1, H)
    _need(x, "hidden_states", torch.bfloat16, 2)
    if not 1 <= top_k <= min(E, 32):
        raise ValueError("top_k must be in [1, min(E, 32)]")
    T = x.shape[0]
    lib = _lib.load()
    dev = x.device
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    logits = ids = w = None
    if return_routing:
        logits = torch.empty((T, E), dtype=torch.bfloat16, device=dev)
        ids = torch.empty((T, top_k), dtype=index_dtype, device=dev)
        w = torch.empty((T, top_k), dtype=torch.bfloat16, device=dev)
    ws = _ws(lib.moe_mi355x_block_workspace_bytes(T, H, I, E, top_k), dev)
    _lib.check(lib.moe_mi355x_block_fp8(
        x.data_ptr(), router_weight.data_ptr(), T, H, I, E, top_k, int(norm_topk_prob), gate_up_proj.data_ptr(),
        gate_up_proj_scale_inv.data_ptr(), down_proj.data_ptr(), down_proj_scale_inv.data_ptr(), out.data_ptr(),
        logits.data_ptr() if logits is not None else None, ids.data_ptr() if ids is not None else None,
        _id_bytes(ids) if ids is not None else 4, w.data_ptr() if w is not None else None,
        ws.data_ptr(), ws.numel(), _stream(x)), "moe_mi355x_block_fp8")
    out = out.reshape(shape)
    if return_routing:
        return out, (logits, w, ids)
    return out


def _check_bf16_expert_weights(w13, w2):
    _need(w13, "gate_up_proj", torch.bfloat16, 3)
    _need(w2, "down_proj", torch.bfloat16, 3)
    E, I2, H = w13.shape
    I = I2 // 2
    if I2 % 2 or I % BLOCK or H % BLOCK:
        raise ValueError(f"gate_up_proj must be [E, 2I, H] with I, H multiples of {BLOCK}")
    if tuple(w2.shape) != (E, H, I):
        raise ValueError(f"down_proj must be [E, H, I] = {(E, H, I)}, got {tuple(w2.shape)}")
    if H > 8192 or I > 8192 or not 1 <= E <= 256:
        raise ValueError("supported shapes: H, I <= 8192 and 1 <= E <= 256")
    return E, H, I


def experts_bf16(hidden_states, top_k_index, top_k_weights, gate_up_proj, down_proj):
    """bf16 experts, ``grouped_mm_experts_forward`` (TF/integrations/moe.py:377-478) on bf16
    weights ``gate_up_proj`` [E,2I,H] and ``down_proj`` [E,H,I].  Returns bf16 [T, H]."""
    E, H, I = _check_bf16_expert_weights(gate_up_proj, down_proj)
    _need(hidden_states, "hidden_states", torch.bfloat16, 2)
    _need(top_k_index, "top_k_index", (torch.int32, torch.int64), 2)
    _need(top_k_weights, "top_k_weights", torch.bfloat16, 2)
    T = hidden_states.shape[0]
    if hidden_states.shape[1] != H:
        raise ValueError(f"hidden_states must be [T, {H}]")
    if top_k_index.shape[0] != T or tuple(top_k_weights.shape) != tuple(top_k_index.shape):
        raise ValueError("top_k_index and top_k_weights must both be [T, k]")
    k = top_k_index.shape[1]
    if not 1 <= k <= min(E, 32):
        raise ValueError("k must be in [1, min(E, 32)]")
    lib = _lib.load()
    out = torch.empty((T, H), dtype=torch.bfloat16, device=hidden_states.device)
    ws = _ws(lib.moe_mi355x_experts_bf16_workspace_bytes(T, H, I, E, k), hidden_states.device)
    _lib.check(lib.moe_mi355x_experts_bf16(hidden_states.data_ptr(), top_k_index.data_ptr(), _id_bytes(top_k_index),
                                           top_k_weights.data_ptr(), T, H, I, E, k, gate_up_proj.data_ptr(),
                                           down_proj.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(),
                                           _stream(hidden_states)), "moe_mi355x_experts_bf16")
    return out


def moe_block_bf16(hidden_states, router_weight, top_k, gate_up_proj, down_proj, norm_topk_prob=True,
                   return_routing=False, index_dtype=torch.int64):
    """Router + bf16 experts (``Qwen3MoeSparseMoeBlock.forward`` on a bf16 checkpoint,
    TF/models/qwen3_moe/modeling_qwen3_moe.py:276-281).  hidden_states: [..., H] bf16."""
    E, H, I = _check_bf16_expert_weights(gate_up_proj, down_proj)
    _need(router_weight, "router_weight", torch.bfloat16, 2)
    if tuple(router_weight.shape) != (E, H):
        raise ValueError(f"router_weight must be [{E}, {H}]")
    shape = hidden_states.shape
    x = hidden_states.reshape(-1, H)
    _need(x, "hidden_states", torch.bfloat16, 2)
    if not 1 <= top_k <= min(E, 32):
        raise ValueError("top_k must be in [1, min(E, 32)]")
    T = x.shape[0]
    lib = _lib.load()
    dev = x.device
    out = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    logits = ids = w = None
    if return_routing:
        logits = torch.empty((T, E), dtype=torch.bfloat16, device=dev)
        ids = torch.empty((T, top_k), dtype=index_dtype, device=dev)
        w = torch.empty((T, top_k), dtype=torch.bfloat16, device=dev)
    ws = _ws(lib.moe_mi355x_block_bf16_workspace_bytes(T, H, I, E, top_k), dev)
    _lib.check(lib.moe_mi355x_block_bf16(
        x.data_ptr(), router_weight.data_ptr(), T, H, I, E, top_k, int(norm_topk_prob), gate_up_proj.data_ptr(),
        down_proj.data_ptr(), out.data_ptr(), logits.data_ptr() if logits is not None else None,
        ids.data_ptr() if ids is not None else None, _id_bytes(ids) if ids is not None else 4,
        w.data_ptr() if w is not None else None, ws.data_ptr(), ws.numel(), _stream(x)), "moe_mi355x_block_bf16")
    out = out.reshape(shape)
    if return_routing:
        return out, (logits, w, ids)
    return out


# ---------------------------------------------------------------------------
# paged decode attention
# ---------------------------------------------------------------------------

PAGE_SIZE = 16
HEAD_DIM = 128


def _check_kv_pools(k_cache: torch.Tensor, v_cache: torch.Tensor, num_kv_heads: int) -> None:
    """K pool [pages, Hkv, 16, 128] and V pool [pages, Hkv, 128, 16] of the same size (the
    kernels index both by the same page id)."""
    P = k_cache.shape[0]
    if tuple(k_cache.shape) != (P, num_kv_heads, PAGE_SIZE, HEAD_DIM):
        raise ValueError(f"k_cache must be [pages, {num_kv_heads}, {PAGE_SIZE}, {HEAD_DIM}], got {tuple(k_cache.shape)}")
    if tuple(v_cache.shape) != (P, num_kv_heads, HEAD_DIM, PAGE_SIZE):
        raise ValueError(f"v_cache must be [{P}, {num_kv_heads}, {HEAD_DIM}, {PAGE_SIZE}], got {tuple(v_cache.shape)}")


def paged_attention_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float) -> torch.Tensor:
    """Decode attention of one new token per sequence over a paged KV cache.

    The attention of ``Qwen3MoeAttention.forward`` for a decode step
    (TF/models/qwen3_moe/modeling_qwen3_moe.py:151-191 with ``eager_attention_forward`` :96-119):
    ``q`` bf16 [B, Hq, 128]; ``k_cache`` bf16 [pages, Hkv, 16, 128] (token rows);
    ``v_cache`` bf16 [pages, Hkv, 128, 16] (dim rows); ``block_tables`` int32 [B, max_pages];
    ``context_lens`` int32 [B].  Returns bf16 [B, Hq, 128].
    """
    _need(q, "q", torch.bfloat16, 3)
    _need(k_cache, "k_cache", torch.bfloat16, 4)
    _need(v_cache, "v_cache", torch.bfloat16, 4)
    _need(block_tables, "block_tables", torch.int32, 2)
    _need(context_lens, "context_lens", torch.int32, 1)
    B, Hq, D = q.shape
    P, Hkv, ps, D2 = k_cache.shape
    if D != HEAD_DIM or D2 != HEAD_DIM or ps != PAGE_SIZE:
        raise ValueError(f"head_dim must be {HEAD_DIM} and page size {PAGE_SIZE}")
    if tuple(v_cache.shape) != (P, Hkv, HEAD_DIM, PAGE_SIZE):
        raise ValueError(f"v_cache must be [pages, Hkv, {HEAD_DIM}, {PAGE_SIZE}], got {tuple(v_cache.shape)}")
    if Hq % Hkv or Hq // Hkv > 16:
        raise ValueError(f"Hq ({Hq}) must be a multiple of Hkv ({Hkv}) with at most 16 query heads per kv head")
    if block_tables.shape[0] != B or context_lens.shape[0] != B:
        raise ValueError("block_tables and context_lens need one row per sequence")
    max_pages = block_tables.shape[1]
    lib = _lib.load()
    out = torch.empty_like(q)
    ws = _ws(lib.moe_mi355x_paged_attn_workspace_bytes(B, Hq, Hkv, max_pages), q.device)
    _lib.check(lib.moe_mi355x_paged_attn_decode(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                                block_tables.data_ptr(), context_lens.data_ptr(), B, Hq, Hkv,
                                                HEAD_DIM, PAGE_SIZE, max_pages, P, float(scale), out.data_ptr(),
                                                ws.data_ptr(), ws.numel(), _stream(q)), "paged_attn_decode")
    return out


def kv_append(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
              block_tables: torch.Tensor, positions: torch.Tensor) -> None:
    """Writes one token's k, v (bf16 [B, Hkv, 128]) per sequence at ``positions`` (int32 [B])
    into the paged cache (the cache update of modeling_qwen3_moe.py:170-171)."""
    _need(k, "k", torch.bfloat16, 3)
    _need(v, "v", torch.bfloat16, 3)
    _need(k_cache, "k_cache", torch.bfloat16, 4)
    _need(v_cache, "v_cache", torch.bfloat16, 4)
    _need(block_tables, "block_tables", torch.int32, 2)
    _need(positions, "positions", torch.int32, 1)
    B, Hkv, D = k.shape
    if tuple(v.shape) != (B, Hkv, D) or D != HEAD_DIM:
        raise ValueError("k, v must be [B, Hkv, 128]")
    _check_kv_pools(k_cache, v_cache, Hkv)
    if block_tables.shape[0] != B or positions.shape[0] != B:
        raise ValueError("block_tables and positions need one row per sequence")
    _lib.check(_lib.load().moe_mi355x_kv_append(k.data_ptr(), v.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
                                                block_tables.data_ptr(), positions.data_ptr(), B, Hkv, HEAD_DIM,
                                                PAGE_SIZE, block_tables.shape[1], k_cache.shape[0], _stream(k)),
               "kv_append")


# ---------------------------------------------------------------------------
# decoder-layer pieces around the attention and the MoE block
# ---------------------------------------------------------------------------


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """``Qwen3MoeRMSNorm.forward`` (TF/models/qwen3_moe/modeling_qwen3_moe.py:294-299) over the
    last axis of a bf16 tensor."""
    _need(x, "x", torch.bfloat16)
    _need(weight, "weight", torch.bfloat16, 1)
    C = x.shape[-1]
    if weight.shape[0] != C:
        raise ValueError(f"weight has {weight.shape[0]} entries for {C} columns")
    out = torch.empty_like(x)
    _lib.check(_lib.load().moe_mi355x_rms_norm(x.data_ptr(), weight.data_ptr(), x.numel() // max(C, 1), C,
                                               float(eps), out.data_ptr(), _stream(x)), "rms_norm")
    return out


def linear_bf16(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """``nn.Linear`` without bias on bf16 tensors: ``x [M, K] @ weight[N, K]^T`` with fp32
    accumulation and one bf16 rounding (the q/k/v and o_proj projections of
    ``Qwen3MoeAttention.forward``, TF/models/qwen3_moe/modeling_qwen3_moe.py:162-164, :189).
    Needs N % 64 == 0 and K % 128 == 0."""
    _need(x, "x", torch.bfloat16, 2)
    _need(weight, "weight", torch.bfloat16, 2)
    M, K = x.shape
    N = weight.shape[0]
    if weight.shape[1] != K:
        raise ValueError(f"weight must be [N, {K}], got {tuple(weight.shape)}")
    if N % 64 or K % 128:
        raise ValueError("linear_bf16 needs N % 64 == 0 and K % 128 == 0")
    lib = _lib.load()
    y = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    nws = lib.moe_mi355x_linear_bf16_workspace_bytes(M, N, K)
    ws = _ws(nws, x.device)
    _lib.check(lib.moe_mi355x_linear_bf16(x.data_ptr(), weight.data_ptr(), M, N, K, y.data_ptr(), ws.data_ptr(), nws,
                                          _stream(x)), "moe_mi355x_linear_bf16")
    return y


def qk_norm_rope_append(qkv: torch.Tensor, q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor,
                        inv_freq: torch.Tensor, positions: torch.Tensor, num_heads: int, num_kv_heads: int,
                        eps: float, k_cache: torch.Tensor, v_cache: torch.Tensor,
                        block_tables: torch.Tensor) -> torch.Tensor:
    """q/k RMSNorm, rotary embedding and the KV-cache append of one new token per sequence
    (modeling_qwen3_moe.py:162-171).  ``qkv`` bf16 [B, (Hq + 2 Hkv) * 128]; returns q bf16
    [B, Hq, 128]; k and v go into the paged cache at ``positions``."""
    _need(qkv, "qkv", torch.bfloat16, 2)
    _need(q_norm_weight, "q_norm_weight", torch.bfloat16, 1)
    _need(k_norm_weight, "k_norm_weight", torch.bfloat16, 1)
    _need(inv_freq, "inv_freq", torch.float32, 1)
    _need(positions, "positions", torch.int32, 1)
    _need(k_cache, "k_cache", torch.bfloat16, 4)
    _need(v_cache, "v_cache", torch.bfloat16, 4)
    _need(block_tables, "block_tables", torch.int32, 2)
    B = qkv.shape[0]
    if qkv.shape[1] != (num_heads + 2 * num_kv_heads) * HEAD_DIM or inv_freq.shape[0] != HEAD_DIM // 2:
        raise ValueError("qkv must be [B, (Hq + 2 Hkv) * 128] and inv_freq [64]")
    _check_kv_pools(k_cache, v_cache, num_kv_heads)
    if positions.shape[0] != B or block_tables.shape[0] != B:
        raise ValueError("positions and block tables must match the batch")
    q = torch.empty((B, num_heads, HEAD_DIM), dtype=torch.bfloat16, device=qkv.device)
    _lib.check(_lib.load().moe_mi355x_qk_norm_rope_append(
        qkv.data_ptr(), q_norm_weight.data_ptr(), k_norm_weight.data_ptr(), inv_freq.data_ptr(), positions.data_ptr(),
        B, num_heads, num_kv_heads, HEAD_DIM, float(eps), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
        block_tables.data_ptr(), PAGE_SIZE, block_tables.shape[1], k_cache.shape[0], _stream(qkv)),
        "qk_norm_rope_append")
    return q


def moe_sublayer_fp8(hidden_states, ln_weight, eps, router_weight, top_k, gate_up_proj, gate_up_proj_scale_inv,
                     down_proj, down_proj_scale_inv, norm_topk_prob: bool = True,
                     add: torch.Tensor | None = None) -> torch.Tensor:
    """``h + moe_block(post_attention_layernorm(h))`` (modeling_qwen3_moe.py:344-347): the RMSNorm,
    the MoE block and the residual add in one entry point.  With ``add`` (the attention's o_proj
    output) the sublayer's input is ``h = bf16(hidden_states + add)``, the residual add of
    :341, formed inside the RMSNorm and the combine instead of in a launch of its own."""
    _need(hidden_states, "hidden_states", torch.bfloat16, 2)
    _need(ln_weight, "ln_weight", torch.bfloat16, 1)
    _need(router_weight, "router_weight", torch.bfloat16, 2)
    if add is not None:
        _need(add, "add", torch.bfloat16, 2)
        if add.shape != hidden_states.shape:
            raise ValueError(f"add must match hidden_states {tuple(hidden_states.shape)}, got {tuple(add.shape)}")
    E, H, I = _check_expert_weights(gate_up_proj, gate_up_proj_scale_inv, down_proj, down_proj_scale_inv)
    if not 1 <= top_k <= min(E, 32):
        raise ValueError("top_k must be in [1, min(E, 32)]")
    T = hidden_states.shape[0]
    if hidden_states.shape[1] != H or tuple(router_weight.shape) != (E, H) or ln_weight.shape[0] != H:
        raise ValueError("hidden_states, ln_weight and router_weight must match the experts' hidden size")
    lib = _lib.load()
    out = torch.empty_like(hidden_states)
    ws = _ws(lib.moe_mi355x_moe_sublayer_workspace_bytes(T, H, I, E, top_k), hidden_states.device)
    _lib.check(lib.moe_mi355x_moe_sublayer_fp8(
        hidden_states.data_ptr(), None if add is None else add.data_ptr(), ln_weight.data_ptr(), float(eps),
        router_weight.data_ptr(), T, H, I, E, top_k, int(norm_topk_prob), gate_up_proj.data_ptr(),
        gate_up_proj_scale_inv.data_ptr(), down_proj.data_ptr(), down_proj_scale_inv.data_ptr(), out.data_ptr(),
        ws.data_ptr(), ws.numel(), _stream(hidden_states)), "moe_sublayer_fp8")
    return out
