// FP8 e4m3 quantisers: dynamic per-row/per-128 activation quantisation and the
// per-128x128-tile weight quantiser.  Both are HBM-bound byte streams: 16-byte
// vector loads per lane, the group reduction stays inside 16 adjacent lanes.
#include "common.h"

namespace {

// One 128-column group is handled by 16 lanes x 8 bf16 values.
__global__ __launch_bounds__(256) void quant_act_kernel(const uint16_t* __restrict__ x, long n_groups,
                                                        uint8_t* __restrict__ q, float* __restrict__ scales) {
  const long g = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  if (g >= n_groups) return;  // the 16 lanes of a group leave together
  const long elem = g * MOE_GROUP + sub * 8;  // groups are contiguous: row r, group j -> r*C + j*128
  quant_group16(x + elem, q + elem, scales + g, sub);
}

// One workgroup per 128x128 tile; thread t owns row t/2, 64 contiguous columns.
template <typename TIn>
__global__ __launch_bounds__(256) void quant_weight_kernel(const TIn* __restrict__ w, int N, int K,
                                                           uint8_t* __restrict__ q,
                                                           float* __restrict__ scale_inv) {
  const int kb_n = K / MOE_GROUP, nb_n = N / MOE_GROUP;
  const int tile = blockIdx.x;
  const int b = tile / (nb_n * kb_n);
  const int nb = (tile / kb_n) % nb_n;
  const int kb = tile % kb_n;
  const int row = threadIdx.x >> 1, half = threadIdx.x & 1;
  const long base = ((long)b * N + (long)nb * MOE_GROUP + row) * K + (long)kb * MOE_GROUP + half * 64;
  float v[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) {
    if constexpr (sizeof(TIn) == 2)
      v[i] = bf16_to_f32(((const uint16_t*)w)[base + i]);
    else
      v[i] = ((const float*)w)[base + i];
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 64; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = wave_max(amax);
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // scale = 448 / amax, stored inverse 1 / scale, both in fp32 (finegrained_fp8.py:924-928)
  const float scale = amax > 0.f ? MOE_FP8_MAX / amax : 1.0f;
  if (threadIdx.x == 0) scale_inv[tile] = 1.0f / scale;
  uint32_t packed[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    packed[i] = pack4_e4m3(clamp_fp8(v[4 * i] * scale), clamp_fp8(v[4 * i + 1] * scale),
                           clamp_fp8(v[4 * i + 2] * scale), clamp_fp8(v[4 * i + 3] * scale));
  uint4* dst = (uint4*)(q + base);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    dst[i] = make_uint4(packed[4 * i], packed[4 * i + 1], packed[4 * i + 2], packed[4 * i + 3]);
}

}  // namespace

int moe_launch_quant_act(const void* x, int R, int C, void* q, float* scales, hipStream_t s, int slot) {
  if (R == 0) return MOE_OK;
  const long n_groups = (long)R * (C / MOE_GROUP);
  const long blocks = (n_groups + 15) / 16;
  MOE_RETURN_IF(!moe_grid_fits(blocks), MOE_ERR_INVALID_ARG);
  MOE_LAUNCH(slot, s, quant_act_kernel, dim3((unsigned)blocks), dim3(256), 0, s, (const uint16_t*)x,
             n_groups, (uint8_t*)q, scales);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}

extern "C" int moe_mi355x_quantize_act_fp8(const void* x, int R, int C, void* q, float* scales,
                                           void* stream) {
  MOE_RETURN_IF(R < 0 || C <= 0 || C % MOE_GROUP, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(R > 0 && (!x || !q || !scales), MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(R > 0 && (!moe_aligned16(x) || !moe_aligned16(q)), MOE_ERR_ALIGNMENT);
  return moe_launch_quant_act(x, R, C, q, scales, (hipStream_t)stream);
}

extern "C" int moe_mi355x_quantize_weight_fp8(const void* w, int w_dtype, int B, int N, int K,
                                              void* q, float* scale_inv, void* stream) {
  MOE_RETURN_IF(B < 0 || N <= 0 || K <= 0 || N % MOE_GROUP || K % MOE_GROUP, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(w_dtype != 0 && w_dtype != 1, MOE_ERR_INVALID_ARG);
  if (B == 0) return MOE_OK;
  MOE_RETURN_IF(!w || !q || !scale_inv, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!moe_aligned16(w) || !moe_aligned16(q), MOE_ERR_ALIGNMENT);
  const long tiles = (long)B * (N / MOE_GROUP) * (K / MOE_GROUP);
  MOE_RETURN_IF(!moe_grid_fits(tiles), MOE_ERR_INVALID_ARG);
  hipStream_t s = (hipStream_t)stream;
  if (w_dtype == 0)
    hipLaunchKernelGGL(quant_weight_kernel<uint16_t>, dim3((unsigned)tiles), dim3(256), 0, s,
                       (const uint16_t*)w, N, K, (uint8_t*)q, scale_inv);
  else
    hipLaunchKernelGGL(quant_weight_kernel<float>, dim3((unsigned)tiles), dim3(256), 0, s,
                       (const float*)w, N, K, (uint8_t*)q, scale_inv);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}
