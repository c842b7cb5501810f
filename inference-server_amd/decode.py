"""Decode step of a Qwen3-MoE model on the MI355X kernels.

One new token per sequence per step, for a batch of sequences with a paged KV cache.  Each
decoder layer follows ``Qwen3MoeDecoderLayer.forward``
(TF/models/qwen3_moe/modeling_qwen3_moe.py:319-348; TF = transformers 5.15.0, the reference
server's model code, reached through TorchBackend's batched decode, torch_backend.py:305-322):

    residual = h;  x = input_layernorm(h)                              (:329-330)
    q, k, v = q_proj(x), k_proj(x), v_proj(x);  q, k = q_norm(q), k_norm(k)   (:162-164)
    q, k = rotary(q, k)                                               (:166-167)
    cache.update(k, v);  a = attention(q, cache)                      (:169-186)
    h = residual + o_proj(a)                                          (:189, :341)
    residual = h;  h = residual + moe_block(post_attention_layernorm(h))     (:344-347)

Per layer this is four entry points of this library plus the two projections:
``moe_mi355x_rms_norm`` (input_layernorm), the fused q/k/v projection,
``moe_mi355x_qk_norm_rope_append`` (q_norm, k_norm, rotary, KV-cache update),
``moe_mi355x_paged_attn_decode``, o_proj, and ``moe_mi355x_moe_sublayer_fp8`` (the residual add
after the attention, post_attention_layernorm, the MoE block, the residual add).  The projections
run on ``moe_mi355x_linear_bf16`` up to ``LINEAR_MAX_ROWS`` sequences, where the pair measures
faster than hipBLASLt in a graph replay (q/k/v + o_proj 1 / 16 / 24 rows: 19.7 / 21.2 / 23.8 us
against 26.1 / 26.4 / 26.6 us), and on hipBLASLt through ``torch.nn.functional.linear`` above
(32 rows: 24.5 against 23.6 us).
``DecodeModel.capture`` records a whole step as one HIP graph, so a step costs one launch.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import kernels

# Batch size up to which the decode step's projections use the library's bf16 linear kernel.
LINEAR_MAX_ROWS = 24


def _linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    if x.shape[0] <= LINEAR_MAX_ROWS:
        return kernels.linear_bf16(x, w)
    return torch.nn.functional.linear(x, w)

PAGE_SIZE = kernels.PAGE_SIZE
HEAD_DIM = kernels.HEAD_DIM


@dataclass(frozen=True)
class DecoderConfig:
    """Shape of a Qwen3-MoE decoder layer (configuration_qwen3_moe.py:85-109 defaults are the
    Qwen3-30B-A3B values)."""

    hidden: int = 2048
    heads: int = 32
    kv_heads: int = 4
    head_dim: int = HEAD_DIM
    experts: int = 128
    top_k: int = 8
    moe_intermediate: int = 768
    rms_eps: float = 1e-6
    rope_theta: float = 1e6
    norm_topk_prob: bool = True


def default_inv_freq(cfg: DecoderConfig, device) -> torch.Tensor:
    """``inv_freq`` of the default rope, computed as ``Qwen3MoeRotaryEmbedding`` does
    (``compute_default_rope_parameters``, modeling_qwen3_moe.py:400-418): fp32 on the CPU, then
    moved to the device.  (The GPU's fp32 pow differs from the CPU's in the last place for a
    third of the entries, which shifts the rotary phase at long positions.)"""
    exps = torch.arange(0, cfg.head_dim, 2, dtype=torch.float) / cfg.head_dim
    return (1.0 / (cfg.rope_theta ** exps)).to(device).contiguous()


class PagedKVCache:
    """Per-layer paged K / V pools in the layout of ``moe_mi355x_paged_attn_decode``:
    K [pages, kv_heads, 16, 128] (token rows), V [pages, kv_heads, 128, 16] (dim rows)."""

    def __init__(self, n_layers: int, n_pages: int, kv_heads: int, device, dtype=torch.bfloat16):
        self.k = [torch.zeros((n_pages, kv_heads, PAGE_SIZE, HEAD_DIM), dtype=dtype, device=device)
                  for _ in range(n_layers)]
        self.v = [torch.zeros((n_pages, kv_heads, HEAD_DIM, PAGE_SIZE), dtype=dtype, device=device)
                  for _ in range(n_layers)]
        self.n_pages = n_pages


class DecoderLayerWeights:
    """Weights of one decoder layer.  The q/k/v projections are stored as one fused
    [(Hq + 2 Hkv) * d, H] matrix (rows: q, then k, then v), so one GEMM serves all three."""

    def __init__(self, cfg: DecoderConfig, ln1, wqkv, q_norm, k_norm, wo, ln2, router, q13, s13, q2, s2):
        self.cfg = cfg
        self.ln1, self.wqkv, self.q_norm, self.k_norm, self.wo, self.ln2 = ln1, wqkv, q_norm, k_norm, wo, ln2
        self.router, self.q13, self.s13, self.q2, self.s2 = router, q13, s13, q2, s2

    @classmethod
    def random(cls, cfg: DecoderConfig, device, generator: torch.Generator, std: float = 0.02):
        """Random-init weights of the architecture: bf16 N(0, std) matrices, unit norm weights,
        FP8 experts block-quantised on the GPU."""
        H, d = cfg.hidden, cfg.head_dim
        bf = torch.bfloat16

        def randn(*shape):
            return (torch.randn(shape, generator=generator, device=device) * std).to(bf)

        ones = lambda n: torch.ones(n, dtype=bf, device=device)  # noqa: E731
        wqkv = randn((cfg.heads + 2 * cfg.kv_heads) * d, H)
        wo = randn(H, cfg.heads * d)
        router = randn(cfg.experts, H)
        w13 = randn(cfg.experts, 2 * cfg.moe_intermediate, H)
        q13, s13 = kernels.quantize_weight_fp8(w13)
        del w13
        w2 = randn(cfg.experts, H, cfg.moe_intermediate)
        q2, s2 = kernels.quantize_weight_fp8(w2)
        del w2
        return cls(cfg, ones(H), wqkv, ones(d), ones(d), wo, ones(H), router, q13, s13, q2, s2)

    @classmethod
    def from_hf_layer(cls, layer, cfg: DecoderConfig):
        """From a transformers ``Qwen3MoeDecoderLayer`` whose MoE block is already an
        ``MI355XSparseMoeBlock`` (``swap_moe_blocks``)."""
        at = layer.self_attn
        wqkv = torch.cat([at.q_proj.weight, at.k_proj.weight, at.v_proj.weight], dim=0).contiguous()
        e = layer.mlp.experts
        return cls(cfg, layer.input_layernorm.weight.detach(), wqkv.detach(), at.q_norm.weight.detach(),
                   at.k_norm.weight.detach(), at.o_proj.weight.detach(), layer.post_attention_layernorm.weight.detach(),
                   layer.mlp.gate.weight.detach(), e.gate_up_proj, e.gate_up_proj_scale_inv, e.down_proj,
                   e.down_proj_scale_inv)


def attention_sublayer(w: DecoderLayerWeights, h, positions, context_lens, block_tables, inv_freq, k_cache,
                       v_cache):
    """``o_proj(attention(input_layernorm(h)))`` for one new token per sequence, appending the
    token's k, v to the cache (modeling_qwen3_moe.py:329-340 with :151-191).  The residual add
    of :341 is left to the caller (the MoE sublayer forms it)."""
    cfg = w.cfg
    B = h.shape[0]
    x = kernels.rms_norm(h, w.ln1, cfg.rms_eps)
    qkv = _linear(x, w.wqkv)
    q = kernels.qk_norm_rope_append(qkv, w.q_norm, w.k_norm, inv_freq, positions, cfg.heads, cfg.kv_heads,
                                    cfg.rms_eps, k_cache, v_cache, block_tables)
    a = kernels.paged_attention_decode(q, k_cache, v_cache, block_tables, context_lens, cfg.head_dim ** -0.5)
    return _linear(a.view(B, cfg.heads * cfg.head_dim), w.wo)


def moe_sublayer(w: DecoderLayerWeights, h, attn_out=None):
    """``h' + moe_block(post_attention_layernorm(h'))`` with ``h' = h + attn_out``
    (modeling_qwen3_moe.py:341-347; ``attn_out`` None: ``h' = h``)."""
    cfg = w.cfg
    return kernels.moe_sublayer_fp8(h, w.ln2, cfg.rms_eps, w.router, cfg.top_k, w.q13, w.s13, w.q2, w.s2,
                                    norm_topk_prob=cfg.norm_topk_prob, add=attn_out)


def decoder_layer(w: DecoderLayerWeights, h, positions, context_lens, block_tables, inv_freq, k_cache, v_cache):
    """One full decoder layer for one decode step (modeling_qwen3_moe.py:319-348)."""
    o = attention_sublayer(w, h, positions, context_lens, block_tables, inv_freq, k_cache, v_cache)
    return moe_sublayer(w, h, o)


class DecodeModel:
    """The decoder-layer stack of a Qwen3-MoE model for batched decode over a paged KV cache.

    ``step(h, positions, context_lens, block_tables)`` runs every layer on the hidden states of
    the batch's new tokens ([B, hidden] bf16; ``positions`` int32 [B] = index of the new token,
    ``context_lens`` = positions + 1, ``block_tables`` int32 [B, max_pages]).  ``capture`` records
    one step as a HIP graph over static input buffers: copy a step's inputs into those buffers,
    then call the graph's ``replay()``.
    """

    def __init__(self, cfg: DecoderConfig, layers: list[DecoderLayerWeights], cache: PagedKVCache):
        self.cfg = cfg
        self.layers = layers
        self.cache = cache
        dev = layers[0].wqkv.device
        self.inv_freq = default_inv_freq(cfg, dev)
        self._graph = None

    def step(self, h, positions, context_lens, block_tables, moe: bool = True, attention: bool = True):
        for i, w in enumerate(self.layers):
            o = None
            if attention:
                o = attention_sublayer(w, h, positions, context_lens, block_tables, self.inv_freq, self.cache.k[i],
                                       self.cache.v[i])
            if moe:
                h = moe_sublayer(w, h, o)
            elif o is not None:
                h = h + o
        return h

    def capture(self, h, positions, context_lens, block_tables, moe: bool = True, attention: bool = True):
        """Records one step on copies of the given inputs; returns the graph handle
        (graph, static inputs, static output)."""
        dev = h.device
        statics = [t.clone() for t in (h, positions, context_lens, block_tables)]
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):  # warm the allocator and the library outside the capture
            self.step(*statics, moe=moe, attention=attention)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = self.step(*statics, moe=moe, attention=attention)
        return graph, statics, out
