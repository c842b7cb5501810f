// Fused element-wise pieces of the Qwen3-MoE decoder layer around the MoE block and the
// attention, in the reference's bf16 rounding order (TF = transformers 5.15.0):
//
//   rms_norm_kernel:  Qwen3MoeRMSNorm.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:294-299:
//                     y = bf16(w * bf16(x * (1 / sqrt(mean(x^2) + eps)))), fp32 statistics.
//   qk_norm_rope_append_kernel: the per-head q_norm / k_norm (:162-163), the rotary embedding
//                     (:166-167 with rotate_half / apply_rotary_pos_emb :51-81 and the default
//                     rope of Qwen3MoeRotaryEmbedding :421-436: cos / sin of pos * inv_freq in
//                     fp32, cast to bf16) and the KV-cache update (:169-171) of one new token per
//                     sequence, one launch for all heads of the batch.
#include "common.h"

namespace {

constexpr int kHD = 128;
constexpr int kPage = 16;

// y = bf16(w * bf16(x * r)), r = 1 / sqrt(sum(x^2) / C + eps): one wave per row, C <= 8192,
// C % 8 == 0.  The row, its residual addend (ADD) and the norm weight are all loaded at the start
// (16-byte loads), unconditionally: a lane past the row's end reloads the last chunk and zeroes
// it (a branch around loads makes the compiler wait for them where it joins, and the weight,
// loaded after the row's sum, cost a second round trip).  With ADD the normalised row is
// x = bf16(x + add) (the decoder layer's residual add before the post-attention norm,
// modeling_qwen3_moe.py:341), also written to `sum_out` when non-null.
template <int MAXV, bool ADD>  // uint4 chunks (8 values) per lane
__global__ __launch_bounds__(256) void rms_norm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ add,
                                                       const uint16_t* __restrict__ w, int R, int C, float eps,
                                                       uint16_t* __restrict__ out, uint16_t* __restrict__ sum_out) {
  // every product and sum below is rounded like the reference's separate torch ops: no
  // multiply-add contraction across the bf16 roundings
#pragma clang fp contract(off)
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= R) return;
  const int lane = threadIdx.x & 63;
  const uint16_t* xr = x + (long)row * C;
  uint4 v[MAXV], av[MAXV], wv[MAXV];
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = min((i * 64 + lane) * 8, C - 8);
    v[i] = *(const uint4*)(xr + c);
    if constexpr (ADD) av[i] = *(const uint4*)(add + (long)row * C + c);
    wv[i] = *(const uint4*)(w + c);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = (i * 64 + lane) * 8;
    if constexpr (ADD) {
      const uint32_t xu[4] = {v[i].x, v[i].y, v[i].z, v[i].w}, au[4] = {av[i].x, av[i].y, av[i].z, av[i].w};
      uint32_t su[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = __uint_as_float(xu[j] << 16) + __uint_as_float(au[j] << 16);
        const float hi = __uint_as_float(xu[j] & 0xffff0000u) + __uint_as_float(au[j] & 0xffff0000u);
        su[j] = (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
      }
      v[i] = make_uint4(su[0], su[1], su[2], su[3]);
      if (sum_out != nullptr && c < C) *(uint4*)(sum_out + (long)row * C + c) = v[i];
    }
    if (c >= C) v[i] = make_uint4(0, 0, 0, 0);  // past the row: contributes nothing, never stored
    const uint32_t u[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = __uint_as_float(u[j] << 16), b = __uint_as_float(u[j] & 0xffff0000u);
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)C + eps);
#pragma unroll
  for (int i = 0; i < MAXV; ++i) {
    const int c = (i * 64 + lane) * 8;
    if (c >= C) continue;
    const uint32_t u[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
    const uint32_t wu[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = round_bf16(__uint_as_float(u[j] << 16) * r);
      const float b = round_bf16(__uint_as_float(u[j] & 0xffff0000u) * r);
      const float ya = __uint_as_float(wu[j] << 16) * a;
      const float yb = __uint_as_float(wu[j] & 0xffff0000u) * b;
      o[j] = (uint32_t)f32_to_bf16(ya) | ((uint32_t)f32_to_bf16(yb) << 16);
    }
    *(uint4*)(out + (long)row * C + c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// One wave per (token, head) of the fused qkv row [q heads | k heads | v heads], head_dim 128:
// lane l holds elements l and l + 64, exactly the pair rotate_half mixes.
//   q heads: rmsnorm(q_w) -> rotary -> q_out [B, Hq, 128]
//   k heads: rmsnorm(k_w) -> rotary -> k_cache (token rows) at positions[b]
//   v heads: v_cache (dim rows) at positions[b]
__global__ __launch_bounds__(256) void qk_norm_rope_append_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ qw, const uint16_t* __restrict__ kw,
    const float* __restrict__ inv_freq, const int32_t* __restrict__ positions, int B, int Hq, int Hkv, float eps,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const int32_t* __restrict__ block_tables, int max_pages, int num_pages) {
  // x * cos + rotate_half(x) * sin: both products are rounded to bf16 before the sum (the
  // reference's separate bf16 ops), so no multiply-add contraction here
#pragma clang fp contract(off)
  const int nh = Hq + 2 * Hkv;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= B * nh) return;
  const int b = item / nh, h = item % nh;
  const int lane = threadIdx.x & 63;
  const uint16_t* src = qkv + ((long)b * nh + h) * kHD;
  // every load that depends only on the item goes out first (the norm weight and the rotary
  // frequency too, used after the head's sum), so a q head costs one round trip
  const uint16_t* nw = h < Hq ? qw : kw;
  const uint16_t s0 = src[lane], s1 = src[lane + 64];
  const uint16_t w0 = nw[lane], w1 = nw[lane + 64];
  const float ifreq = inv_freq[lane];
  float x0 = bf16_to_f32(s0), x1 = bf16_to_f32(s1);
  const int pos = positions[b];
  // a position outside the block table, or a table entry outside the pools (a -1 pad, a stale
  // id), has no page: q is still written, the cache is not
  const bool in_table = pos >= 0 && pos < kPage * max_pages;
  const long page = in_table ? block_tables[(long)b * max_pages + pos / kPage] : -1;
  if ((page < 0 || page >= num_pages) && h >= Hq) return;
  const int slot = pos % kPage;
  if (h >= Hq + Hkv) {  // v head: transposed page rows
    const int g = h - Hq - Hkv;
    uint16_t* dst = v_cache + (page * Hkv + g) * (long)(kHD * kPage);
    dst[lane * kPage + slot] = s0;
    dst[(lane + 64) * kPage + slot] = s1;
    return;
  }
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float r = 1.0f / sqrtf(ss / (float)kHD + eps);
  x0 = round_bf16(bf16_to_f32(w0) * round_bf16(x0 * r));
  x1 = round_bf16(bf16_to_f32(w1) * round_bf16(x1 * r));
  // cos / sin of pos * inv_freq[lane] (both halves of emb = cat(freqs, freqs) share it)
  const float f = (float)pos * ifreq;
  const float c = round_bf16(cosf(f)), s = round_bf16(sinf(f));
  // element lane: x0 * cos - x1 * sin; element lane + 64: x1 * cos + x0 * sin (bf16 steps)
  const float y0 = round_bf16(round_bf16(x0 * c) + round_bf16(-x1 * s));
  const float y1 = round_bf16(round_bf16(x1 * c) + round_bf16(x0 * s));
  uint16_t* dst;
  if (h < Hq) {
    dst = q_out + ((long)b * Hq + h) * kHD;
  } else {
    dst = k_cache + (page * Hkv + (h - Hq)) * (long)(kHD * kPage) + slot * kHD;
  }
  dst[lane] = f32_to_bf16(y0);
  dst[lane + 64] = f32_to_bf16(y1);
}

}  // namespace

int moe_launch_rms_norm(const void* x, const void* add, const void* w, int R, int C, float eps, void* out,
                        void* sum_out, hipStream_t s) {
  if (R <= 0) return MOE_OK;
  const dim3 grid((R + 3) / 4), block(256);
  const int chunks = (C / 8 + 63) / 64;
#define MOE_RMS(V_)                                                                                        \
  do {                                                                                                     \
    if (add != nullptr)                                                                                    \
      hipLaunchKernelGGL((rms_norm_kernel<V_, true>), grid, block, 0, s, (const uint16_t*)x,               \
                         (const uint16_t*)add, (const uint16_t*)w, R, C, eps, (uint16_t*)out, (uint16_t*)sum_out); \
    else                                                                                                   \
      hipLaunchKernelGGL((rms_norm_kernel<V_, false>), grid, block, 0, s, (const uint16_t*)x,              \
                         (const uint16_t*)add, (const uint16_t*)w, R, C, eps, (uint16_t*)out, (uint16_t*)sum_out); \
  } while (0)
  if (chunks <= 1)
    MOE_RMS(1);
  else if (chunks <= 4)
    MOE_RMS(4);
  else
    MOE_RMS(16);
#undef MOE_RMS
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}

extern "C" int moe_mi355x_rms_norm(const void* x, const void* weight, int rows, int cols, float eps, void* out,
                                   void* stream) {
  MOE_RETURN_IF(rows < 0 || cols <= 0 || cols % 8 || cols > 8192, MOE_ERR_INVALID_ARG);
  if (rows == 0) return MOE_OK;
  MOE_RETURN_IF(!x || !weight || !out, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!moe_aligned16(x) || !moe_aligned16(weight) || !moe_aligned16(out), MOE_ERR_ALIGNMENT);
  return moe_launch_rms_norm(x, nullptr, weight, rows, cols, eps, out, nullptr, (hipStream_t)stream);
}

extern "C" int moe_mi355x_qk_norm_rope_append(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                              const float* inv_freq, const int32_t* positions, int B, int Hq,
                                              int Hkv, int head_dim, float eps, void* q_out, void* k_cache,
                                              void* v_cache, const int32_t* block_tables, int page_size,
                                              int max_pages, int num_pages, void* stream) {
  MOE_RETURN_IF(B < 0 || Hq <= 0 || Hkv <= 0 || head_dim != kHD || page_size != kPage || max_pages <= 0 ||
                    num_pages < 0,
                MOE_ERR_INVALID_ARG);
  if (B == 0) return MOE_OK;
  MOE_RETURN_IF(!qkv || !q_norm_w || !k_norm_w || !inv_freq || !positions || !q_out || !k_cache || !v_cache ||
                    !block_tables,
                MOE_ERR_INVALID_ARG);
  const long items = (long)B * (Hq + 2 * Hkv);
  MOE_RETURN_IF(!moe_grid_fits((items + 3) / 4), MOE_ERR_INVALID_ARG);
  hipLaunchKernelGGL(qk_norm_rope_append_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)qkv, (const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w, inv_freq, positions,
                     B, Hq, Hkv, eps, (uint16_t*)q_out, (uint16_t*)k_cache, (uint16_t*)v_cache, block_tables,
                     max_pages, num_pages);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}
