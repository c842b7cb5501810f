/*
 * moe_mi355x.h -- C ABI of the MI355X (gfx950) Qwen3-MoE FP8 expert hot path.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t (passed as
 * void*), enqueues its kernels on that stream and returns 0 on success or a
 * MOE_ERR_* code (or a hipError_t, which is positive) on failure.  No entry point
 * synchronises the stream or allocates device memory; scratch comes in through a
 * caller-owned workspace whose size the matching *_workspace_bytes() call returns.
 *
 * Layouts (row-major, C-contiguous, 16-byte aligned):
 *   bf16  = uint16 bit patterns of bfloat16
 *   fp8   = uint8 OCP e4m3fn codes (torch.float8_e4m3fn)
 *   ids   = int32 or int64 (id_bytes = 4 or 8), [T, k]
 *
 * The reference path these replace lives in the reference server's dependency
 * `transformers` 5.15.0 (reference pyproject.toml:14; TF = transformers/):
 *   TF/models/qwen3_moe/modeling_qwen3_moe.py, TF/integrations/moe.py,
 *   TF/integrations/finegrained_fp8.py.  It is reached from the reference at
 *   src/inference_server/backends/torch_backend.py:38-40 (model load) and
 *   :288-290, :313-320 (every model forward).
 */
#ifndef MOE_MI355X_H
#define MOE_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MOE_OK = 0,
  MOE_ERR_INVALID_ARG = -1,    /* null pointer, bad size or unsupported shape */
  MOE_ERR_WORKSPACE = -2,      /* workspace smaller than *_workspace_bytes() */
  MOE_ERR_ALIGNMENT = -3,      /* a pointer is not 16-byte aligned */
  MOE_ERR_SCRATCH = -4,        /* larger than the no-allocation entry point's fixed scratch */
};

/* Human-readable text for a return code (MOE_ERR_* or hipError_t). */
const char* moe_mi355x_error_string(int code);

/* Library version, (major << 16) | minor. */
int moe_mi355x_version(void);

/*
 * Router: logits = x @ w_router^T (bf16 out, fp32 accumulation), softmax in fp32,
 * top-k by (descending logit, ascending expert id), optional renormalisation,
 * weights cast to bf16.
 * Replaces Qwen3MoeTopKRouter.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267.
 *   x        bf16 [T, H]        w_router bf16 [E, H]
 *   logits   bf16 [T, E] (out)  ids [T, k] (out, id_bytes)  weights bf16 [T, k] (out)
 * Constraints: H % 32 == 0, 1 <= E <= 256, 1 <= k <= min(E, 32).
 */
size_t moe_mi355x_route_workspace_bytes(int T, int H, int E);
int moe_mi355x_route(const void* x, const void* w_router, int T, int H, int E, int k, int renorm,
                     void* logits, void* ids, int id_bytes, void* weights,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * Softmax + top-k + renorm from given bf16 logits (the second half of moe_mi355x_route).
 * Replaces modeling_qwen3_moe.py:261-266.
 */
int moe_mi355x_topk_softmax(const void* logits, int T, int E, int k, int renorm,
                            void* ids, int id_bytes, void* weights, void* stream);

/*
 * Stable expert sort of the T*k (token, slot) pairs plus per-expert counts, offsets
 * and the M-tile list the grouped GEMMs walk.
 * Replaces torch.sort + histc + cumsum, TF/integrations/moe.py:389-403.
 *   ids     [T*k] (id_bytes), values in [0, E)
 *   perm    int32 [T*k]   (out) flat pair index t*k+j in sorted order (stable)
 *   counts  int32 [E]     (out) pairs per expert (the reference's tokens_per_expert)
 *   offsets int32 [E+1]   (out) exclusive prefix; offsets[1:] is the reference's cumsum
 *   tiles   int32 [max_tiles, 4] (out) {expert, first sorted row, rows, 0} per block_m rows
 *   n_tiles int32 [1]     (out)
 * max_tiles = moe_mi355x_align_max_tiles(T*k, E, block_m).
 */
int moe_mi355x_align_max_tiles(int S, int E, int block_m);
size_t moe_mi355x_align_workspace_bytes(int S, int E);
int moe_mi355x_align(const void* ids, int id_bytes, int T, int k, int E, int block_m,
                     int32_t* perm, int32_t* counts, int32_t* offsets, int32_t* tiles,
                     int32_t* n_tiles, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Dynamic activation quantisation, per row and per 128-column group:
 * s = amax/448 (1 if amax == 0), q = e4m3(clamp(x/s, -448, 448)).
 * Replaces the inline activation quantiser of the FP8 grouped GEMM,
 * TF/integrations/finegrained_fp8.py:191-196 (Triton source not shipped).
 *   x bf16 [R, C] -> q fp8 [R, C], scales fp32 [R, C/128].  C % 128 == 0.
 */
int moe_mi355x_quantize_act_fp8(const void* x, int R, int C, void* q, float* scales, void* stream);

/*
 * Weight quantisation per 128x128 tile: scale = 448/amax (1 if amax == 0),
 * q = e4m3(clamp(w*scale, -448, 448)), scale_inv = 1/scale.
 * Replaces Fp8Quantize._quantize_one, TF/integrations/finegrained_fp8.py:903-941.
 *   w [B, N, K] (w_dtype 0 = bf16, 1 = fp32) -> q fp8 [B, N, K], scale_inv fp32 [B, N/128, K/128]
 */
int moe_mi355x_quantize_weight_fp8(const void* w, int w_dtype, int B, int N, int K,
                                   void* q, float* scale_inv, void* stream);

/*
 * FP8 block-scaled experts forward.
 * Replaces fp8_grouped_mm_experts_forward, TF/integrations/finegrained_fp8.py:498-589
 * (signature forward(self, hidden_states, top_k_index, top_k_weights)).
 *   x        bf16 [T, H]          ids [T, k] (id_bytes)      weights bf16 [T, k]
 *   w13      fp8 [E, 2I, H]       s13 fp32 [E, 2I/128, H/128]   (gate rows [0,I), up rows [I,2I))
 *   w2       fp8 [E, H, I]        s2  fp32 [E, H/128, I/128]
 *   out      bf16 [T, H]
 * Constraints: H % 128 == 0, I % 128 == 0, 1 <= E <= 256, 1 <= k <= 32.
 */
size_t moe_mi355x_experts_workspace_bytes(int T, int H, int I, int E, int k);
int moe_mi355x_experts_fp8(const void* x, const void* ids, int id_bytes, const void* weights,
                           int T, int H, int I, int E, int k,
                           const void* w13, const float* s13, const void* w2, const float* s2,
                           void* out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Whole MoE block: router + FP8 experts.
 * Replaces Qwen3MoeSparseMoeBlock.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:276-281.
 * logits / ids / weights may be NULL when the caller does not need them.
 */
size_t moe_mi355x_block_workspace_bytes(int T, int H, int I, int E, int k);
int moe_mi355x_block_fp8(const void* x, const void* w_router, int T, int H, int I, int E, int k,
                         int renorm, const void* w13, const float* s13, const void* w2,
                         const float* s2, void* out, void* logits, void* ids, int id_bytes,
                         void* weights, void* workspace, size_t workspace_bytes, void* stream);

/*
 * bf16 experts forward (no FP8 requantisation): the reference's default path for bf16
 * checkpoints, grouped_mm_experts_forward, TF/integrations/moe.py:377-478.  Same arguments as
 * moe_mi355x_experts_fp8 with bf16 weights and no scales:
 *   w13 bf16 [E, 2I, H] (gate rows [0,I), up rows [I,2I)),  w2 bf16 [E, H, I].
 * Each grouped GEMM returns bf16 (fp32 accumulation), silu(gate) * up in bf16, bf16 routing-weight
 * product, fp32 slot-order sum, bf16 out.  Constraints: H % 128 == 0, I % 128 == 0, H, I <= 8192.
 */
size_t moe_mi355x_experts_bf16_workspace_bytes(int T, int H, int I, int E, int k);
int moe_mi355x_experts_bf16(const void* x, const void* ids, int id_bytes, const void* weights,
                            int T, int H, int I, int E, int k, const void* w13, const void* w2,
                            void* out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Whole MoE block with bf16 experts: router + moe_mi355x_experts_bf16.
 * Replaces Qwen3MoeSparseMoeBlock.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:276-281, as
 * the reference runs it on a bf16 checkpoint (torch_backend.py:38-40).
 * logits / ids / weights may be NULL when the caller does not need them.
 */
size_t moe_mi355x_block_bf16_workspace_bytes(int T, int H, int I, int E, int k);
int moe_mi355x_block_bf16(const void* x, const void* w_router, int T, int H, int I, int E, int k,
                          int renorm, const void* w13, const void* w2, void* out, void* logits, void* ids,
                          int id_bytes, void* weights, void* workspace, size_t workspace_bytes, void* stream);

/*
 * moe_mi355x_block_fp8 without a workspace argument and without any allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Its scratch is a fixed device array inside the library,
 * moe_mi355x_block_fp8_noalloc_scratch_bytes() = 64 MiB, one per GPU, held until the process ends
 * (enough for moe_mi355x_block_workspace_bytes of decode batches up to 256 tokens at the
 * Qwen3-235B-A22B shape, or 1024 at Qwen3-30B-A3B); a call needing more returns MOE_ERR_SCRATCH
 * and launches nothing.  Every call on a GPU shares that GPU's array: calls that overlap on one GPU
 * (two streams or two threads at once) race.  Results are identical to moe_mi355x_block_fp8's.
 */
size_t moe_mi355x_block_fp8_noalloc_scratch_bytes(void);
int moe_mi355x_block_fp8_noalloc(const void* x, const void* w_router, int T, int H, int I, int E, int k,
                                 int renorm, const void* w13, const float* s13, const void* w2,
                                 const float* s2, void* out, void* logits, void* ids, int id_bytes,
                                 void* weights, void* stream);

/*
 * Which of the block path's batch-size-dependent launch choices can change its output bits
 * (the router GEMM's K chunks and kernel, the expert GEMMs' tile height), for the FP8 block
 * (fp8 != 0) or the bf16 block: two batch sizes with the same key compute every token's row the
 * same way.  0 for unsupported shapes.  A query
 * (host only): a caller that pads batches up to a captured size (a HIP graph per batch bucket)
 * splits its buckets where the key changes, so that a padded batch reproduces the unpadded one
 * bit for bit.  No counterpart in the reference (its eager forward has no buckets).
 */
long long moe_mi355x_block_numerics_key(int T, int H, int I, int E, int k, int fp8);

/*
 * Paged GQA decode attention, one new token per sequence (the attention of a decode step of
 * Qwen3MoeAttention.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:151-191, with
 * eager_attention_forward :96-119): for query head h of sequence b, over the keys
 * 0 .. context_lens[b]-1 of kv head h / (Hq / Hkv):
 *   s = bf16(bf16(q . k) * scale),  out = bf16( softmax_fp32(s) . V )
 * (the softmax is applied unnormalised and divided once, in fp32).
 *   q            bf16 [B, Hq, 128]          out bf16 [B, Hq, 128]
 *   k_cache      bf16 [pages, Hkv, 16, 128] (token rows)
 *   v_cache      bf16 [pages, Hkv, 128, 16] (transposed: dim rows)
 *   block_tables int32 [B, max_pages]       page of each 16-token block of a sequence (device
 *                                           data); an entry outside [0, num_pages) (a -1 pad, a
 *                                           stale id) is an empty page: it is never read and its
 *                                           keys are left out of the softmax
 *   context_lens int32 [B]                  >= 1, <= 16 * max_pages (device data: a larger value
 *                                           is clamped to the table; 0, or a context whose pages
 *                                           are all empty, gives a zero output)
 *   num_pages                               pages in each of k_cache and v_cache
 * The KV layout is this library's; the reference keeps a contiguous per-layer cache.
 * Constraints: head_dim == 128, page_size == 16, Hq % Hkv == 0, Hq / Hkv <= 16; q, k_cache,
 * v_cache and out 16-byte aligned; B * Hkv * (splits of max_pages) < 2^31 (splits of up to 64
 * pages; the workspace query returns 0 past it).
 */
size_t moe_mi355x_paged_attn_workspace_bytes(int B, int Hq, int Hkv, int max_pages);
int moe_mi355x_paged_attn_decode(const void* q, const void* k_cache, const void* v_cache,
                                 const int32_t* block_tables, const int32_t* context_lens, int B, int Hq,
                                 int Hkv, int head_dim, int page_size, int max_pages, int num_pages, float scale,
                                 void* out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * KV-cache append of one token per sequence at position positions[b] (the cache update of
 * Qwen3MoeAttention.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:170-171, in the paged
 * layout above).  k, v: bf16 [B, Hkv, 128] (k after k_norm and rotary embedding).
 * positions[b] in [0, 16 * max_pages), its page allocated in block_tables; a position outside
 * the table, or a table entry outside [0, num_pages), writes nothing.
 */
int moe_mi355x_kv_append(const void* k, const void* v, void* k_cache, void* v_cache,
                         const int32_t* block_tables, const int32_t* positions, int B, int Hkv,
                         int head_dim, int page_size, int max_pages, int num_pages, void* stream);

/*
 * RMSNorm over the last axis: out = bf16(w * bf16(x * (1 / sqrt(mean(x^2) + eps)))), fp32
 * statistics.  Replaces Qwen3MoeRMSNorm.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:294-299.
 *   x, out bf16 [rows, cols]   weight bf16 [cols]       cols % 8 == 0, cols <= 8192
 */
int moe_mi355x_rms_norm(const void* x, const void* weight, int rows, int cols, float eps, void* out,
                        void* stream);

/*
 * bf16 linear layer without bias: y = bf16(x @ w^T), fp32 accumulation, one rounding.  Replaces
 * the nn.Linear projections of Qwen3MoeAttention.forward (q_proj / k_proj / v_proj fused into
 * one weight, and o_proj), TF/models/qwen3_moe/modeling_qwen3_moe.py:162-164 and :189.
 *   x bf16 [M, K]   w bf16 [N, K]   y bf16 [M, N]     N % 64 == 0, K % 128 == 0, 16-byte aligned
 * The K dimension is split over workgroups when the output alone would not fill the GPU; the fp32
 * partials then go to `workspace` (linear_bf16_workspace_bytes(M, N, K) bytes, 0 when no split)
 * and are summed in a fixed order, so results do not depend on timing.
 */
size_t moe_mi355x_linear_bf16_workspace_bytes(int M, int N, int K);
int moe_mi355x_linear_bf16(const void* x, const void* w, int M, int N, int K, void* y, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * The per-token tail of the q/k/v projections of a decode step: per-head RMSNorm of q and k
 * (q_norm / k_norm), the rotary embedding at positions[b] (cos / sin of positions[b] * inv_freq
 * in fp32, cast to bf16), q written out, k and v appended to the paged cache (layout of
 * moe_mi355x_paged_attn_decode).  Replaces Qwen3MoeAttention.forward's
 * TF/models/qwen3_moe/modeling_qwen3_moe.py:162-171 (with apply_rotary_pos_emb :59-81 and
 * Qwen3MoeRotaryEmbedding.forward :421-436) for one token per sequence.
 *   qkv      bf16 [B, (Hq + 2 Hkv) * 128]  (q heads, then k heads, then v heads)
 *   q_norm_w, k_norm_w bf16 [128]          inv_freq fp32 [64]      positions int32 [B]
 *   q_out    bf16 [B, Hq, 128]
 * positions[b] in [0, 16 * max_pages), its page allocated in block_tables; for a position
 * outside the table, or a table entry outside [0, num_pages), q is written and the cache is not.
 */
int moe_mi355x_qk_norm_rope_append(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                   const float* inv_freq, const int32_t* positions, int B, int Hq, int Hkv,
                                   int head_dim, float eps, void* q_out, void* k_cache, void* v_cache,
                                   const int32_t* block_tables, int page_size, int max_pages, int num_pages,
                                   void* stream);

/*
 * MoE sublayer of a decoder layer: out = h' + moe_block(rms_norm(h', ln_weight)) with
 * h' = bf16(h + h_add) (h_add NULL: h' = h), the residual add done in the top-k combine.
 * Replaces Qwen3MoeDecoderLayer.forward's TF/models/qwen3_moe/modeling_qwen3_moe.py:341-347
 * (the residual add after the attention, post_attention_layernorm, the sparse block :276-281,
 * the residual add).  h_add is the attention's o_proj output; other arguments as
 * moe_mi355x_block_fp8.  The residual add and the RMSNorm run in one launch (which also writes
 * h'), the router GEMM and the x quantisation in the next; the residual add after the block rides
 * in the combine.
 */
size_t moe_mi355x_moe_sublayer_workspace_bytes(int T, int H, int I, int E, int k);
int moe_mi355x_moe_sublayer_fp8(const void* h, const void* h_add, const void* ln_weight, float eps,
                                const void* w_router, int T, int H, int I, int E, int k, int renorm,
                                const void* w13, const float* s13, const void* w2, const float* s2, void* out,
                                void* workspace, size_t workspace_bytes, void* stream);

/*
 * Kernel timing (instrumentation; no counterpart in the reference).  While enabled, each
 * kernel launch of this library is bracketed by hipEvents on its stream; profile_read
 * waits for them and returns the launch count and summed duration (ms) of one slot:
 *   0 router_gemm  1 topk_softmax  2 quant_act  3 align  4 gemm_gate_up  5 quant_h
 *   6 gemm_down    7 combine   8 linear
 * Enabling (or disabling) clears what was recorded.
 */
int moe_mi355x_profile_enable(int on);
int moe_mi355x_profile_read(int slot, int* count, double* total_ms);
const char* moe_mi355x_profile_slot_name(int slot);

#ifdef __cplusplus
}
#endif

#endif /* MOE_MI355X_H */
