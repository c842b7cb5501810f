"""CPU oracle for the decode-step attention of the Qwen3-MoE decoder layer.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package never does.

It restates in numpy what the reference server runs per decoder layer around the MoE
block, through its dependency ``transformers`` 5.15.0 (``TF/`` = ``transformers/``):

* ``rms_norm``: ``Qwen3MoeRMSNorm.forward``, TF/models/qwen3_moe/modeling_qwen3_moe.py:294-299
  (fp32 variance, ``x * rsqrt(var + eps)`` cast back to bf16, times the bf16 weight).
* ``rotary``: ``rotate_half`` / ``apply_rotary_pos_emb`` (:51-81) with the default rope
  ``inv_freq = theta ** -(2i/d)`` of ``Qwen3MoeRotaryEmbedding`` (:381-436), cos/sin in bf16.
* ``decode_attention``: ``eager_attention_forward`` (:96-119) for one query token:
  ``s = bf16(bf16(q . k) * scaling)``, ``p = bf16(softmax_fp32(s))``, ``o = bf16(p . V)``
  with fp32 accumulation, kv head ``h // (Hq / Hkv)`` (``repeat_kv``, :84-93).
* ``gather_paged``: reads a sequence's keys and values out of this library's paged layout
  (K pages [page][kv head][16][128], V pages transposed [page][kv head][128][16]).

Parity status (how each is pinned is in ``tests/test_oracle.py``):

* ``decode_attention``: pinned (pure-Python brute force on tiny shapes, closed forms:
  identical keys give the mean of V, a dominant key selects its V row, kv-head mapping;
  golden vectors written by transformers' ``eager_attention_forward`` on CPU).
* ``rms_norm``, ``rotary``, ``rope_cos_sin``, ``default_inv_freq``: pinned (golden vectors of
  transformers' ``Qwen3MoeRMSNorm``, ``Qwen3MoeRotaryEmbedding`` (its inv_freq and cos / sin)
  and ``apply_rotary_pos_emb`` on CPU; closed forms: rotation preserves pair norms, position 0
  is the identity).
* ``gather_paged``: pinned (round trip against ``scatter_paged`` on a shuffled page table).
"""

from __future__ import annotations

import numpy as np

from .moe_oracle import round_bf16

PAGE = 16


def rms_norm(x, weight, eps: float = 1e-6) -> np.ndarray:
    """``Qwen3MoeRMSNorm.forward`` (modeling_qwen3_moe.py:294-299) over the last axis; x, weight
    bf16-valued float32 arrays, result bf16-valued."""
    x = np.asarray(x, np.float32)
    var = np.mean(np.square(x, dtype=np.float32), axis=-1, keepdims=True, dtype=np.float32)
    y = round_bf16(x * (np.float32(1.0) / np.sqrt(var + np.float32(eps), dtype=np.float32)))
    return round_bf16(np.asarray(weight, np.float32) * y)


def default_inv_freq(head_dim: int = 128, theta: float = 1e6) -> np.ndarray:
    """``1 / theta ** (2i / d)`` in fp32 (``compute_default_rope_parameters``,
    modeling_qwen3_moe.py:400-418).  The reference evaluates the pow with torch's CPU fp32 pow;
    numpy's fp32 pow differs from it in the last place for some entries, so tests that need the
    reference's exact phases pass its own inv_freq (stored with the golden vectors)."""
    return (1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.int64).astype(np.float32) / head_dim))).astype(
        np.float32)


def rope_cos_sin(positions, head_dim: int = 128, theta: float = 1e6, inv_freq=None):
    """cos, sin [len(positions), head_dim] of the default rope (modeling_qwen3_moe.py:381-436):
    ``freqs = pos * inv_freq`` in fp32, ``emb = cat(freqs, freqs)``, cast to bf16; cos / sin
    evaluated in float64 and rounded (within one fp32 ulp of any accurate fp32 cos / sin)."""
    if inv_freq is None:
        inv_freq = default_inv_freq(head_dim, theta)
    inv_freq = np.asarray(inv_freq, np.float32)
    freqs = np.asarray(positions, np.float32)[:, None] * inv_freq[None, :]
    emb = np.concatenate([freqs, freqs], axis=-1).astype(np.float64)
    return round_bf16(np.cos(emb).astype(np.float32)), round_bf16(np.sin(emb).astype(np.float32))


def rotary(x, cos, sin) -> np.ndarray:
    """``q * cos + rotate_half(q) * sin`` (modeling_qwen3_moe.py:51-81) in bf16 arithmetic:
    each product and the sum rounded to bf16.  x [..., n_heads, d]; cos/sin [..., d]."""
    x = np.asarray(x, np.float32)
    d = x.shape[-1]
    rot = np.concatenate([-x[..., d // 2:], x[..., : d // 2]], axis=-1)
    c = np.asarray(cos, np.float32)[..., None, :]
    s = np.asarray(sin, np.float32)[..., None, :]
    return round_bf16(round_bf16(x * c) + round_bf16(rot * s))


def decode_attention(q, keys, values, scale: float) -> np.ndarray:
    """One query token per sequence.  q [Hq, d]; keys, values [L, Hkv, d] (bf16-valued);
    returns bf16-valued [Hq, d]."""
    q = np.asarray(q, np.float32)
    keys = np.asarray(keys, np.float32)
    values = np.asarray(values, np.float32)
    Hq, d = q.shape
    L, Hkv, _ = keys.shape
    G = Hq // Hkv
    out = np.empty((Hq, d), np.float32)
    for h in range(Hq):
        g = h // G
        s = round_bf16(keys[:, g, :].astype(np.float64) @ q[h].astype(np.float64))
        s = round_bf16(s.astype(np.float32) * np.float32(scale))
        m = s.max()
        e = np.exp((s - m).astype(np.float32), dtype=np.float32)
        p = round_bf16(e / e.sum(dtype=np.float32))
        out[h] = round_bf16(p.astype(np.float64) @ values[:, g, :].astype(np.float64))
    return out


def scatter_paged(keys, values, pages):
    """Places one sequence's keys / values [L, Hkv, d] into fresh paged K / V^T caches with the
    given page list (page j holds tokens 16 j .. 16 j + 15).  Returns (k_cache, v_cache)."""
    keys = np.asarray(keys, np.float32)
    values = np.asarray(values, np.float32)
    L, Hkv, d = keys.shape
    n_pages = max(pages) + 1
    kc = np.zeros((n_pages, Hkv, PAGE, d), np.float32)
    vc = np.zeros((n_pages, Hkv, d, PAGE), np.float32)
    for t in range(L):
        pg, slot = pages[t // PAGE], t % PAGE
        kc[pg, :, slot, :] = keys[t]
        vc[pg, :, :, slot] = values[t]
    return kc, vc


def gather_paged(k_cache, v_cache, block_table, length: int):
    """Keys and values [length, Hkv, d] of one sequence from the paged caches."""
    k_cache = np.asarray(k_cache)
    v_cache = np.asarray(v_cache)
    n = (length + PAGE - 1) // PAGE
    pages = np.asarray(block_table[:n], np.int64)
    k = k_cache[pages]                              # [n, Hkv, 16, d]
    v = np.transpose(v_cache[pages], (0, 1, 3, 2))  # [n, Hkv, 16, d]
    k = np.transpose(k, (0, 2, 1, 3)).reshape(n * PAGE, k.shape[1], -1)[:length]
    v = np.transpose(v, (0, 2, 1, 3)).reshape(n * PAGE, v.shape[1], -1)[:length]
    return k, v
