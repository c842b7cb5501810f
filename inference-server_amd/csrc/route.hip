// Router: bf16 logits GEMM on MFMA (v_mfma_f32_16x16x32_bf16, fp32 accumulation),
// then a one-wave-per-token softmax / top-k / renormalise pass.
//
// Reference: Qwen3MoeTopKRouter.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267.
#include "align_dev.h"

namespace {

constexpr int kRouterTileT = 16;    // tokens per MFMA tile
constexpr int kRouterWaveE = 16;    // experts per wave
constexpr int kRouterBlockE = 64;   // experts per workgroup (4 waves)
constexpr int kMaxKSplit = 16;      // router K-split partials summed by the top-k kernel

// partial[z, t, e] = sum over k in chunk z of x[t, k] * w[e, k]   (fp32)
// grid (ceil(T/16), ceil(E/64), ksplit), block 256.  With xq != nullptr the workgroups
// of expert block 0 also quantise their 16 x kchunk slice of x (kchunk % 128 == 0), so
// the experts need no separate activation-quantisation pass.
__global__ __launch_bounds__(256) void router_gemm_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ wr, int T, int H,
                                                          int E, int kchunk, float* __restrict__ part,
                                                          uint8_t* __restrict__ xq, float* __restrict__ sx) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t0 = blockIdx.x * kRouterTileT;
  const int kbeg = blockIdx.z * kchunk;
  const int kend = min(H, kbeg + kchunk);
  if (xq != nullptr && blockIdx.y == 0) {
    const int groups = kRouterTileT * ((kend - kbeg) / MOE_GROUP);
    const int sub = threadIdx.x & 15;
    for (int g = threadIdx.x >> 4; g < groups; g += 16) {
      const int t = t0 + g % kRouterTileT;
      const int k0 = kbeg + (g / kRouterTileT) * MOE_GROUP;
      if (t < T) {  // the 16 lanes of a group share t
        const long elem = (long)t * H + k0 + sub * 8;
        quant_group16(x + elem, xq + elem, sx + (long)t * (H / MOE_GROUP) + k0 / MOE_GROUP, sub);
      }
    }
  }
  const int e0 = blockIdx.y * kRouterBlockE + wave * kRouterWaveE;
  if (e0 >= E) return;  // wave-uniform
  const int rt = min(t0 + (lane & 15), T - 1);  // clamped rows compute garbage that is never stored
  const int re = min(e0 + (lane & 15), E - 1);
  const int kq = (lane >> 4) * 8;
  const uint16_t* xa = x + (long)rt * H + kq;
  const uint16_t* wb = wr + (long)re * H + kq;
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  int k = kbeg;
  for (; k + 128 <= kend; k += 128) {
    v8bf a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      a[u] = *(const v8bf*)(xa + k + 32 * u);
      b[u] = *(const v8bf*)(wb + k + 32 * u);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[u], b[u], acc, 0, 0, 0);
  }
  for (; k < kend; k += 32) {
    v8bf a = *(const v8bf*)(xa + k), b = *(const v8bf*)(wb + k);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  // D[i][j] lives in lane j + 16*(i/4), element i%4; i = token, j = expert.
  const int e = e0 + (lane & 15);
  if (e >= E) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + 4 * (lane >> 4) + r;
    if (t < T) part[((long)blockIdx.z * T + t) * E + e] = acc[r];
  }
}

// bf16 bit pattern -> unsigned key that orders like the value (-0 folded onto +0).
__device__ __forceinline__ uint32_t bf16_order_key(uint16_t b) {
  if (b == 0x8000u) b = 0;
  return (b & 0x8000u) ? (uint32_t)(~b & 0xffffu) : (uint32_t)(b | 0x8000u);
}

// Routing of one token by one wave.  Each lane holds experts lane, lane+64, lane+128,
// lane+192.  Either sums the router's K-split partials (part != nullptr) and writes the
// bf16 logits, or reads given logits.  Lane j < k returns the j-th expert (descending
// logit, ties to the lower id) and its (renormalised) weight before the bf16 cast.
__device__ __forceinline__ void route_token(const float* __restrict__ part, int ksplit,
                                            const uint16_t* __restrict__ logits_in, int T, int E, int k,
                                            int renorm, uint16_t* __restrict__ logits_out, int t, int& my_e,
                                            float& my_w) {
  const int lane = threadIdx.x & 63;
  uint16_t lb[4];
  bool valid[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
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
  for (int c = 0; c < 4; ++c)
    if (valid[c]) m = fmaxf(m, bf16_to_f32(lb[c]));
  m = wave_max_uniform(m);
  float ex[4];
  float zsum = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    ex[c] = valid[c] ? expf(bf16_to_f32(lb[c]) - m) : 0.f;
    zsum += ex[c];
  }
  zsum = wave_sum_uniform(zsum);
  uint32_t key[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    key[c] = valid[c] ? ((bf16_order_key(lb[c]) << 16) | (0xffffu - (uint32_t)(lane + 64 * c))) : 0u;
  // top-k: k rounds of wave arg-max on (logit, -id)   (modeling_qwen3_moe.py:262)
  my_e = 0;
  float my_p = 0.f, psum = 0.f;
  for (int j = 0; j < k; ++j) {
    uint32_t best = key[0];
#pragma unroll
    for (int c = 1; c < 4; ++c) best = key[c] > best ? key[c] : best;
    best = wave_max_u32_uniform(best);
    const int ew = (int)(0xffffu - (best & 0xffffu));
    const int owner = ew & 63, slot = ew >> 6;
    float pv = 0.f;
    if (lane == owner) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        if (c == slot) {
          pv = ex[c] / zsum;
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

__device__ __forceinline__ void store_route(void* ids, int id_bytes, uint16_t* weights, long idx, int e, float w) {
  weights[idx] = f32_to_bf16(w);
  if (id_bytes == 8)
    ((int64_t*)ids)[idx] = e;
  else
    ((int32_t*)ids)[idx] = e;
}

// One wave per token, 4 tokens per workgroup.
__global__ __launch_bounds__(256) void topk_softmax_kernel(const float* __restrict__ part, int ksplit,
                                                           const uint16_t* __restrict__ logits_in, int T,
                                                           int E, int k, int renorm,
                                                           uint16_t* __restrict__ logits_out, void* ids,
                                                           int id_bytes, uint16_t* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  int my_e;
  float my_w;
  route_token(part, ksplit, logits_in, T, E, k, renorm, logits_out, t, my_e, my_w);
  if (lane < k) store_route(ids, id_bytes, weights, (long)t * k + lane, my_e, my_w);
}

// Decode batches (T * E <= kFusedMaxLogits, T * k <= 4096): routing and the stable
// expert sort in one workgroup.  All router partials are first reduced in parallel
// (coalesced, every load in flight at once) into bf16 logits in LDS; the per-token top-k
// then runs from LDS, and the ids never leave LDS before the sort.
constexpr int kFusedMaxLogits = 32768;

__global__ __launch_bounds__(kChunk) void topk_align_kernel(const float* __restrict__ part, int ksplit, int T,
                                                            int E, int k, int renorm,
                                                            uint16_t* __restrict__ logits_out, void* ids,
                                                            int id_bytes, uint16_t* __restrict__ weights,
                                                            int block_m, int32_t* perm, int32_t* counts,
                                                            int32_t* offsets, int32_t* tiles, int32_t* n_tiles) {
  __shared__ uint16_t s_lg[kFusedMaxLogits];
  __shared__ int s_ids[kSingleMaxS];
  __shared__ int s_cnt[kBuckets];
  __shared__ int s_off[kBuckets];
  __shared__ int s_toff[kBuckets];
  __shared__ int s_wcnt[kWaves][kBuckets];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int TE = T * E;
  for (int e = threadIdx.x; e <= E; e += blockDim.x) s_cnt[e] = 0;
  for (int i = threadIdx.x; i < TE; i += blockDim.x) {
    float pv[kMaxKSplit];  // unconditional loads (clamped slab) so that all of them are in flight
#pragma unroll
    for (int z = 0; z < kMaxKSplit; ++z) pv[z] = part[(long)min(z, ksplit - 1) * TE + i];
    float s = 0.f;
#pragma unroll
    for (int z = 0; z < kMaxKSplit; ++z) s += z < ksplit ? pv[z] : 0.f;
    const uint16_t b = f32_to_bf16(s);
    s_lg[i] = b;
    if (logits_out) logits_out[i] = b;
  }
  __syncthreads();
  for (int t = wave; t < T; t += kWaves) {
    int my_e;
    float my_w;
    route_token(nullptr, 0, s_lg, T, E, k, renorm, nullptr, t, my_e, my_w);
    if (lane < k) {
      store_route(ids, id_bytes, weights, (long)t * k + lane, my_e, my_w);
      s_ids[t * k + lane] = my_e;
    }
  }
  __syncthreads();
  const int S = T * k;
  for (int i = threadIdx.x; i < S; i += blockDim.x) atomicAdd(&s_cnt[s_ids[i]], 1);
  __syncthreads();
  scan_counts(s_cnt, E, block_m, s_off, s_toff);
  __syncthreads();
  emit_meta(s_cnt, s_off, s_toff, E, block_m, counts, offsets, tiles, n_tiles);
  for (int c0 = 0; c0 < S; c0 += kChunk) scatter_chunk(s_ids, 4, S, E, c0, s_off, s_wcnt, perm);
}

int route_ksplit(int T, int H, int E) {
  const int tiles = ((T + kRouterTileT - 1) / kRouterTileT) * ((E + kRouterBlockE - 1) / kRouterBlockE);
  int ks = (256 + tiles - 1) / tiles;
  int kmax = H / 256 > 0 ? H / 256 : 1;
  if (kmax > kMaxKSplit) kmax = kMaxKSplit;
  if (ks > kmax) ks = kmax;
  if (ks < 1) ks = 1;
  return ks;
}

// K chunk per router workgroup; a multiple of 128 when the workgroups also quantise x.
int route_kchunk(int H, int ks, bool quant) {
  const int step = quant ? MOE_GROUP : 32;
  int c = (H + ks - 1) / ks;
  return (c + step - 1) / step * step;
}

bool route_args_ok(int T, int H, int E, int k, int id_bytes) {
  return T >= 0 && H > 0 && H % 32 == 0 && E >= 1 && E <= 256 && k >= 1 && k <= 32 && k <= E &&
         (id_bytes == 4 || id_bytes == 8);
}

}  // namespace

extern "C" size_t moe_mi355x_route_workspace_bytes(int T, int H, int E) {
  if (T <= 0 || H <= 0 || E <= 0) return 0;
  const int ks = route_ksplit(T, H, E);
  return moe_align_up((size_t)ks * T * E * sizeof(float), 256);
}

// Whether moe_launch_route can run the top-k and the expert sort as one workgroup.
bool moe_route_can_fuse_align(int T, int E, int k) {
  // one workgroup routes every token, so the whole top-k runs on one CU: a win over the
  // two-kernel path only while the batch is a handful of tokens
  return T <= 16 && (long)T * E <= kFusedMaxLogits && (long)T * k <= kSingleMaxS;
}

// Router GEMM and top-k softmax.  With xq/sx the router workgroups also quantise x
// (needs H % 128 == 0).  With perm != nullptr (moe_route_can_fuse_align) the top-k and the expert
// sort run fused in one workgroup and write the align outputs too.
int moe_launch_route(const void* x, const void* w_router, int T, int H, int E, int k, int renorm,
                     void* logits, void* ids, int id_bytes, void* weights, void* workspace,
                     size_t workspace_bytes, hipStream_t s, uint8_t* xq, float* sx, int block_m,
                     int32_t* perm, int32_t* counts, int32_t* offsets, int32_t* tiles, int32_t* n_tiles) {
  if (T == 0) return MOE_OK;
  const bool quant = xq != nullptr;
  MOE_RETURN_IF(quant && H % MOE_GROUP, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(perm != nullptr && !moe_route_can_fuse_align(T, E, k), MOE_ERR_INVALID_ARG);
  const int ks = route_ksplit(T, H, E);
  const int kchunk = route_kchunk(H, ks, quant);
  const int ks_eff = (H + kchunk - 1) / kchunk;  // <= ks: the workspace holds ks partial slabs
  MOE_RETURN_IF(workspace_bytes < moe_mi355x_route_workspace_bytes(T, H, E) || !workspace, MOE_ERR_WORKSPACE);
  float* part = (float*)workspace;
  dim3 g1((T + kRouterTileT - 1) / kRouterTileT, (E + kRouterBlockE - 1) / kRouterBlockE, ks_eff);
  MOE_LAUNCH(MOE_PROF_ROUTER_GEMM, s, router_gemm_kernel, g1, dim3(256), 0, s, (const uint16_t*)x,
             (const uint16_t*)w_router, T, H, E, kchunk, part, xq, sx);
  MOE_CHECK_LAUNCH();
  if (perm != nullptr) {
    MOE_LAUNCH(MOE_PROF_TOPK, s, topk_align_kernel, dim3(1), dim3(kChunk), 0, s, part, ks_eff, T, E, k, renorm,
               (uint16_t*)logits, ids, id_bytes, (uint16_t*)weights, block_m, perm, counts, offsets, tiles,
               n_tiles);
  } else {
    MOE_LAUNCH(MOE_PROF_TOPK, s, topk_softmax_kernel, dim3((T + 3) / 4), dim3(256), 0, s, part, ks_eff,
               (const uint16_t*)nullptr, T, E, k, renorm, (uint16_t*)logits, ids, id_bytes, (uint16_t*)weights);
  }
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}

extern "C" int moe_mi355x_route(const void* x, const void* w_router, int T, int H, int E, int k, int renorm,
                                void* logits, void* ids, int id_bytes, void* weights, void* workspace,
                                size_t workspace_bytes, void* stream) {
  MOE_RETURN_IF(!route_args_ok(T, H, E, k, id_bytes), MOE_ERR_INVALID_ARG);
  if (T == 0) return MOE_OK;
  MOE_RETURN_IF(!x || !w_router || !ids || !weights, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!moe_aligned16(x) || !moe_aligned16(w_router), MOE_ERR_ALIGNMENT);
  return moe_launch_route(x, w_router, T, H, E, k, renorm, logits, ids, id_bytes, weights, workspace,
                          workspace_bytes, (hipStream_t)stream, nullptr, nullptr, 0, nullptr, nullptr, nullptr,
                          nullptr, nullptr);
}

extern "C" int moe_mi355x_topk_softmax(const void* logits, int T, int E, int k, int renorm, void* ids,
                                       int id_bytes, void* weights, void* stream) {
  MOE_RETURN_IF(!route_args_ok(T, 32, E, k, id_bytes), MOE_ERR_INVALID_ARG);
  if (T == 0) return MOE_OK;
  MOE_RETURN_IF(!logits || !ids || !weights, MOE_ERR_INVALID_ARG);
  MOE_LAUNCH(MOE_PROF_TOPK, (hipStream_t)stream, topk_softmax_kernel, dim3((T + 3) / 4), dim3(256), 0,
             (hipStream_t)stream, (const float*)nullptr, 0, (const uint16_t*)logits, T, E, k, renorm,
             (uint16_t*)nullptr, ids, id_bytes, (uint16_t*)weights);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}
