// Per-token routing from the router GEMM's K-split partials (softmax, top-k with the
// canonical tie rule, renormalisation), shared by the top-k kernels and the single-token
// gate_up GEMM that routes its own slot.
//
// Reference: Qwen3MoeTopKRouter.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267.
#pragma once

#include "common.h"

namespace {

constexpr int kMaxKSplit = 16;  // router K-split partials summed into one logit

// bf16 bit pattern -> unsigned key that orders like the value (-0 folded onto +0).
__device__ __forceinline__ uint32_t bf16_order_key(uint16_t b) {
  if (b == 0x8000u) b = 0;
  return (b & 0x8000u) ? (uint32_t)(~b & 0xffffu) : (uint32_t)(b | 0x8000u);
}

// Routing of one token by one wave.  Each lane holds experts lane, lane+64, ... (NC = E / 64
// rounded up of them).  Either sums the router's K-split partials (part != nullptr) and writes
// the bf16 logits, or reads given logits.  Lane j < k returns the j-th expert (descending
// logit, ties to the lower id) and its (renormalised) weight before the bf16 cast.
template <int NC>
__device__ __forceinline__ void route_token_nc(const float* __restrict__ part, int ksplit,
                                               const uint16_t* __restrict__ logits_in, int T, int E, int k,
                                               int renorm, uint16_t* __restrict__ logits_out, int t, int& my_e,
                                               float& my_w) {
  const int lane = threadIdx.x & 63;
  uint16_t lb[NC];
  bool valid[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int e = lane + 64 * c;
    valid[c] = e < E;
    lb[c] = 0;
    if (!valid[c]) continue;
    if (part) {
      // all partial loads issue before the first add: they are independent, and a
      // load-add chain would pay the cross-XCD load latency ksplit times
      // (unconditional loads of a clamped slab index: a guarded load would compile to a
      // branch and a wait per partial)
      float pv[kMaxKSplit];
#pragma unroll
      for (int z = 0; z < kMaxKSplit; ++z) pv[z] = part[((long)min(z, ksplit - 1) * T + t) * E + e];
      float s = 0.f;
#pragma unroll
      for (int z = 0; z < kMaxKSplit; ++z) s += z < ksplit ? pv[z] : 0.f;
      lb[c] = f32_to_bf16(s);
      if (logits_out) logits_out[(long)t * E + e] = lb[c];
    } else {
      lb[c] = logits_in[(long)t * E + e];
    }
  }
  // softmax in fp32 (modeling_qwen3_moe.py:261)
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < NC; ++c)
    if (valid[c]) m = fmaxf(m, bf16_to_f32(lb[c]));
  m = wave_max_uniform(m);
  float ex[NC];
  float zsum = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    ex[c] = valid[c] ? expf(bf16_to_f32(lb[c]) - m) : 0.f;
    zsum += ex[c];
  }
  zsum = wave_sum_uniform(zsum);
  float prob[NC];  // the softmax, one division per expert (before the selection rounds)
#pragma unroll
  for (int c = 0; c < NC; ++c) prob[c] = ex[c] / zsum;
  uint32_t key[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
    key[c] = valid[c] ? ((bf16_order_key(lb[c]) << 16) | (0xffffu - (uint32_t)(lane + 64 * c))) : 0u;
  // top-k: k rounds of wave arg-max on (logit, -id)   (modeling_qwen3_moe.py:262)
  my_e = 0;
  float my_p = 0.f, psum = 0.f;
  for (int j = 0; j < k; ++j) {
    uint32_t best = key[0];
#pragma unroll
    for (int c = 1; c < NC; ++c) best = key[c] > best ? key[c] : best;
    best = wave_max_u32_uniform(best);
    const int ew = (int)(0xffffu - (best & 0xffffu));
    const int owner = ew & 63, slot = ew >> 6;
    float pv = 0.f;
    if (lane == owner) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
        if (c == slot) {
          pv = prob[c];
          key[c] = 0u;
        }
    }
    pv = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(pv), owner));
    psum += pv;  // sequential fp32 sum in top-k order, identical in every lane
    if (lane == j) {
      my_e = ew;
      my_p = pv;
    }
  }
  my_w = renorm ? my_p / psum : my_p;  // modeling_qwen3_moe.py:263-266
}

__device__ __forceinline__ void route_token(const float* __restrict__ part, int ksplit,
                                            const uint16_t* __restrict__ logits_in, int T, int E, int k,
                                            int renorm, uint16_t* __restrict__ logits_out, int t, int& my_e,
                                            float& my_w) {
  if (E <= 64)
    route_token_nc<1>(part, ksplit, logits_in, T, E, k, renorm, logits_out, t, my_e, my_w);
  else if (E <= 128)
    route_token_nc<2>(part, ksplit, logits_in, T, E, k, renorm, logits_out, t, my_e, my_w);
  else if (E <= 192)
    route_token_nc<3>(part, ksplit, logits_in, T, E, k, renorm, logits_out, t, my_e, my_w);
  else
    route_token_nc<4>(part, ksplit, logits_in, T, E, k, renorm, logits_out, t, my_e, my_w);
}

__device__ __forceinline__ void store_route(void* ids, int id_bytes, uint16_t* weights, long idx, int e, float w) {
  weights[idx] = f32_to_bf16(w);
  if (id_bytes == 8)
    ((int64_t*)ids)[idx] = e;
  else
    ((int32_t*)ids)[idx] = e;
}

}  // namespace
