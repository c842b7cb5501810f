// Router: bf16 logits GEMM on MFMA (v_mfma_f32_16x16x32_bf16, fp32 accumulation),
// then a one-wave-per-token softmax / top-k / renormalise pass.
//
// Reference: Qwen3MoeTopKRouter.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:258-267.
#include "align_dev.h"
#include "route_dev.h"

namespace {

constexpr int kRouterTileT = 16;    // tokens per MFMA tile
constexpr int kRouterWaveE = 16;    // experts per wave
constexpr int kRouterBlockE = 64;   // experts per workgroup (4 waves)

// partial[z, t, e] = sum over k in chunk z of x[t, k] * w[e, k]   (fp32)
// grid (ceil(T/16), ceil(E/64), ksplit), block 256: wave w computes tokens t0..t0+15 x
// experts e0 + 16 w ..  Each 128-wide K chunk is loaded one chunk ahead of its MFMAs (two
// register sets), so a wave keeps a chunk of loads in flight instead of paying one load
// round trip per chunk.  With xq != nullptr the workgroups of expert block 0 also quantise
// the x rows they load (kchunk % 128 == 0): lane (r, g) holds 8 bf16 at columns
// k + 32 u + 8 g of row r for u = 0..3, i.e. the four lanes r, r+16, r+32, r+48 hold one
// complete 128-column group; every wave forms the group amax and wave w quantises and
// stores the values of u = w.
__global__ __launch_bounds__(256) void router_gemm_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ wr, int T, int H,
                                                          int E, int kchunk, float* __restrict__ part,
                                                          uint8_t* __restrict__ xq, float* __restrict__ sx,
                                                          int32_t* __restrict__ zero, int nzero) {
  // the quantisation's fp32 steps stay separate operations (no multiply-add contraction)
#pragma clang fp contract(off)
  // workgroup 0 clears the expert sort's chunk histograms that the top-k kernel fills next
  if (zero != nullptr && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0)
    for (int i = threadIdx.x; i < nzero; i += blockDim.x) zero[i] = 0;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t0 = blockIdx.x * kRouterTileT;
  const int kbeg = blockIdx.z * kchunk;
  const int kend = min(H, kbeg + kchunk);
  const bool quant = xq != nullptr && blockIdx.y == 0;  // workgroup-uniform
  const int e0 = min(blockIdx.y * kRouterBlockE + wave * kRouterWaveE, E - 1);
  const int rt = min(t0 + (lane & 15), T - 1);  // clamped rows compute garbage that is never stored
  const int re = min(e0 + (lane & 15), E - 1);
  const int kq = (lane >> 4) * 8;
  const uint16_t* xa = x + (long)rt * H + kq;
  const uint16_t* wb = wr + (long)re * H + kq;
  const bool row_ok = t0 + (lane & 15) < T;
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  const int n128 = (kend - kbeg) >> 7;  // whole 128-wide chunks
  v8bf a0[4], b0[4], a1[4], b1[4];
  // MFMAs of chunk c_ on (A_, B_) after issuing the loads of chunk c_ + 1 (clamped: the
  // last chunk reloads itself) into (AN_, BN_), then the x quantisation of chunk c_
#define ROUTER_STEP(A_, B_, AN_, BN_, c_)                                                         \
  do {                                                                                            \
    const int kk_ = kbeg + 128 * (c_);                                                            \
    const int nx_ = kbeg + 128 * min((c_) + 1, n128 - 1);                                         \
    _Pragma("unroll") for (int u = 0; u < 4; ++u) {                                               \
      AN_[u] = *(const v8bf*)(xa + nx_ + 32 * u);                                                 \
      BN_[u] = *(const v8bf*)(wb + nx_ + 32 * u);                                                 \
    }                                                                                             \
    _Pragma("unroll") for (int u = 0; u < 4; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A_[u], B_[u], acc, 0, 0, 0); \
    if (quant) {                                                                                  \
      /* the e4m3 rule of quant_group16: s = amax / 448 (1 if 0), q = e4m3(clamp(x / s)) */      \
      float amax = 0.f;                                                                           \
      _Pragma("unroll") for (int u = 0; u < 4; ++u)                                               \
        _Pragma("unroll") for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf((float)A_[u][i])); \
      amax = fmaxf(amax, __shfl_xor(amax, 16));                                                   \
      amax = fmaxf(amax, __shfl_xor(amax, 32));                                                   \
      const float sc = amax > 0.f ? amax / MOE_FP8_MAX : 1.0f;                                    \
      const v8bf av = wave == 0 ? A_[0] : wave == 1 ? A_[1] : wave == 2 ? A_[2] : A_[3];         \
      float v[8];                                                                                 \
      _Pragma("unroll") for (int i = 0; i < 8; ++i) v[i] = (float)av[i];                          \
      uint2 o;                                                                                    \
      o.x = pack4_e4m3(clamp_fp8(v[0] / sc), clamp_fp8(v[1] / sc), clamp_fp8(v[2] / sc), clamp_fp8(v[3] / sc)); \
      o.y = pack4_e4m3(clamp_fp8(v[4] / sc), clamp_fp8(v[5] / sc), clamp_fp8(v[6] / sc), clamp_fp8(v[7] / sc)); \
      if (row_ok) {                                                                               \
        const long row = t0 + (lane & 15);                                                        \
        *(uint2*)(xq + row * H + kk_ + 32 * wave + kq) = o;                                       \
        if (wave == 0 && kq == 0) sx[row * (H / MOE_GROUP) + kk_ / MOE_GROUP] = sc;               \
      }                                                                                           \
    }                                                                                             \
  } while (0)
  if (n128 > 0) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      a0[u] = *(const v8bf*)(xa + kbeg + 32 * u);
      b0[u] = *(const v8bf*)(wb + kbeg + 32 * u);
    }
  }
  for (int c = 0; c < n128; c += 2) {
    ROUTER_STEP(a0, b0, a1, b1, c);
    if (c + 1 < n128) ROUTER_STEP(a1, b1, a0, b0, c + 1);
  }
#undef ROUTER_STEP
  int k = kbeg + 128 * n128;
  for (; k < kend; k += 32) {
    v8bf a = *(const v8bf*)(xa + k), b = *(const v8bf*)(wb + k);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  }
  // D[i][j] lives in lane j + 16*(i/4), element i%4; i = token, j = expert.
  const int e = blockIdx.y * kRouterBlockE + wave * kRouterWaveE + (lane & 15);
  if (e >= E) return;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + 4 * (lane >> 4) + r;
    if (t < T) part[((long)blockIdx.z * T + t) * E + e] = acc[r];
  }
}

// Router GEMM for large batches: workgroup tile 64 tokens x 128 experts, K in 128-wide
// chunks staged through LDS (x 16 KB, W 32 KB per chunk), so each x row and each router row
// is read once per workgroup instead of once per wave.  Wave w computes tokens 16w..16w+15
// against all 128 experts (8 MFMA tiles).  The next chunk is loaded into registers while the
// current one is computed.  LDS rows are 256 bytes (16 chunks of 8 bf16); chunk c of row r
// is stored at c ^ (r & 15), so the 16 rows of an MFMA fragment read hit 16 distinct bank
// groups.  With xq != nullptr the workgroups of expert block 0 quantise the staged x chunk:
// the four lanes r, r+16, r+32, r+48 of wave w hold row 16w + r's 128-column group.
constexpr int kRtT = 64, kRtE = 128;
__global__ __launch_bounds__(256) void router_gemm_tiled_kernel(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ wr, int T, int H,
                                                                int E, int kchunk, float* __restrict__ part,
                                                                uint8_t* __restrict__ xq, float* __restrict__ sx,
                                                                int32_t* __restrict__ zero, int nzero) {
  if (zero != nullptr && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0)
    for (int i = threadIdx.x; i < nzero; i += blockDim.x) zero[i] = 0;
  __shared__ uint4 s_x[kRtT * 16];
  __shared__ uint4 s_w[kRtE * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int t0 = blockIdx.x * kRtT, eb = blockIdx.y * kRtE;
  const int kbeg = blockIdx.z * kchunk;
  const int nch = (min(H, kbeg + kchunk) - kbeg) >> 7;  // kchunk is a multiple of 128 here
  const bool quant = xq != nullptr && blockIdx.y == 0;
  // loader: x tile 64 rows x 16 chunks (4 per thread), W tile 128 x 16 (8 per thread)
  uint4 xr0, xr1, xr2, xr3, wv0, wv1, wv2, wv3, wv4, wv5, wv6, wv7;
#define RT_LD(dst_, base_, rowbase_, rowmax_, i_)                                                 \
  do {                                                                                            \
    const int idx_ = tid + 256 * (i_);                                                            \
    dst_ = *(const uint4*)((base_) + (long)min((rowbase_) + (idx_ >> 4), (rowmax_)) * H + k0_ + 8 * (idx_ & 15)); \
  } while (0)
#define RT_LOAD(c_)                                                                               \
  do {                                                                                            \
    const int k0_ = kbeg + 128 * (c_);                                                            \
    RT_LD(xr0, x, t0, T - 1, 0); RT_LD(xr1, x, t0, T - 1, 1); RT_LD(xr2, x, t0, T - 1, 2); RT_LD(xr3, x, t0, T - 1, 3); \
    RT_LD(wv0, wr, eb, E - 1, 0); RT_LD(wv1, wr, eb, E - 1, 1); RT_LD(wv2, wr, eb, E - 1, 2); RT_LD(wv3, wr, eb, E - 1, 3); \
    RT_LD(wv4, wr, eb, E - 1, 4); RT_LD(wv5, wr, eb, E - 1, 5); RT_LD(wv6, wr, eb, E - 1, 6); RT_LD(wv7, wr, eb, E - 1, 7); \
  } while (0)
#define RT_ST(arr_, v_, i_)                                                                       \
  do {                                                                                            \
    const int idx_ = tid + 256 * (i_), row_ = idx_ >> 4;                                          \
    arr_[row_ * 16 + ((idx_ & 15) ^ (row_ & 15))] = v_;                                           \
  } while (0)
  RT_LOAD(0);
  v4f acc[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) acc[n] = (v4f){0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < nch; ++c) {
    __syncthreads();  // the previous chunk's readers are done
    RT_ST(s_x, xr0, 0); RT_ST(s_x, xr1, 1); RT_ST(s_x, xr2, 2); RT_ST(s_x, xr3, 3);
    RT_ST(s_w, wv0, 0); RT_ST(s_w, wv1, 1); RT_ST(s_w, wv2, 2); RT_ST(s_w, wv3, 3);
    RT_ST(s_w, wv4, 4); RT_ST(s_w, wv5, 5); RT_ST(s_w, wv6, 6); RT_ST(s_w, wv7, 7);
    __syncthreads();
    RT_LOAD(min(c + 1, nch - 1));  // the last chunk reloads itself (no branch around the loads)
    const int arow = 16 * wave + lr;
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      const int ch = 4 * k4 + lg;
      const v8bf a = __builtin_bit_cast(v8bf, s_x[arow * 16 + (ch ^ lr)]);
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        const v8bf b = __builtin_bit_cast(v8bf, s_w[(16 * n + lr) * 16 + (ch ^ lr)]);
        acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[n], 0, 0, 0);
      }
    }
    if (quant) {
      // the e4m3 rule of quant_group16: s = amax / 448 (1 if 0), q = e4m3(clamp(x / s));
      // lane (r, g) holds chunks 4g..4g+3 of row 16w + r
      float v[32];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ch = 4 * lg + i;
        const uint4 q = s_x[arow * 16 + (ch ^ lr)];
        const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          v[8 * i + 2 * h] = __uint_as_float(w4[h] << 16);
          v[8 * i + 2 * h + 1] = __uint_as_float(w4[h] & 0xffff0000u);
        }
      }
      float amax = 0.f;
#pragma unroll
      for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
      amax = fmaxf(amax, __shfl_xor(amax, 16));
      amax = fmaxf(amax, __shfl_xor(amax, 32));
      const float sc = amax > 0.f ? amax / MOE_FP8_MAX : 1.0f;
      uint32_t o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        o[i] = pack4_e4m3(clamp_fp8(v[4 * i] / sc), clamp_fp8(v[4 * i + 1] / sc), clamp_fp8(v[4 * i + 2] / sc),
                          clamp_fp8(v[4 * i + 3] / sc));
      const int t = t0 + arow;
      if (t < T) {
        uint8_t* dst = xq + (long)t * H + kbeg + 128 * c + 32 * lg;
        *(uint4*)dst = make_uint4(o[0], o[1], o[2], o[3]);
        *(uint4*)(dst + 16) = make_uint4(o[4], o[5], o[6], o[7]);
        if (lg == 0) sx[(long)t * (H / MOE_GROUP) + (kbeg >> 7) + c] = sc;
      }
    }
  }
#undef RT_LOAD
#undef RT_LD
#undef RT_ST
  // D[i][j] lives in lane j + 16*(i/4), element i%4; i = token, j = expert.
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int e = eb + 16 * n + lr;
    if (e >= E) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 16 * wave + 4 * lg + r;
      if (t < T) part[((long)blockIdx.z * T + t) * E + e] = acc[n][r];
    }
  }
}

// One wave per token, 4 tokens per workgroup.  With `bc` (zeroed beforehand) each routed pair
// also counts into its 1024-pair chunk's expert histogram bc[chunk][e], the first pass of the
// expert sort (integer atomics: the counts do not depend on their order).
//
// With `ecnt` (the bucket counts [E] and, after them, one more int: a workgroup count, all zeroed
// beforehand) each pair takes the next place of its expert's bucket instead, bucket[e * T + rank]
// = pair, rank from an atomic count ecnt[e], and the last workgroup to count in writes the 16-row
// decode tile list from the final counts: {expert, first dense row, rows, bucket offset}, experts
// in order (the sorted path's tiles), and the tile count.  The order of the pairs inside a bucket
// (the order of the atomics) changes no result: every tile row is computed on its own.
__global__ __launch_bounds__(256) void topk_softmax_kernel(const float* __restrict__ part, int ksplit,
                                                           const uint16_t* __restrict__ logits_in, int T,
                                                           int E, int k, int renorm,
                                                           uint16_t* __restrict__ logits_out, void* ids,
                                                           int id_bytes, uint16_t* __restrict__ weights,
                                                           int32_t* __restrict__ bc, int32_t* __restrict__ ecnt,
                                                           int32_t* __restrict__ bucket, int32_t* __restrict__ tiles,
                                                           int32_t* __restrict__ n_tiles) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t < T) {
    int my_e;
    float my_w;
    route_token(part, ksplit, logits_in, T, E, k, renorm, logits_out, t, my_e, my_w);
    if (bc != nullptr && lane < k) {
      const int pair = t * k + lane;
      atomicAdd(&bc[(long)(pair / kChunk) * (E + 1) + my_e], 1);
    }
    if (ecnt != nullptr && lane < k) bucket[(long)my_e * T + atomicAdd(&ecnt[my_e], 1)] = t * k + lane;
    if (lane < k) store_route(ids, id_bytes, weights, (long)t * k + lane, my_e, my_w);
  }
  if (ecnt == nullptr) return;  // kernel-uniform
  __shared__ int s_last;
  __shared__ int s_cnt[kBuckets], s_off[kBuckets], s_toff[kBuckets];
  // every wave's count atomics have returned (their ranks addressed the bucket stores): the
  // workgroup's counts are performed; its other stores (bucket entries, ids, weights) carry no
  // release, so they are read only by later launches (the decode GEMMs), which stream order
  // orders after this one; a consumer inside this launch would need xwg_wait_stores() before the
  // count-in below
  __syncthreads();
  if (threadIdx.x == 0) s_last = xwg_count_in(ecnt + E) == (int)gridDim.x - 1;
  __syncthreads();
  if (!s_last) return;
  for (int e = threadIdx.x; e < E; e += blockDim.x) s_cnt[e] = __hip_atomic_load(ecnt + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  scan_counts(s_cnt, E, 16, s_off, s_toff);
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += blockDim.x) {
    if (e == E) {
      n_tiles[0] = s_toff[E];
      continue;
    }
    const int c = s_cnt[e];
    int tix = s_toff[e];
    for (int r = 0; r < c; r += 16, ++tix)
      *(int4*)(tiles + 4 * tix) = make_int4(e, s_off[e] + r, min(16, c - r), e * T + r);
  }
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
                                                            int32_t* offsets, int32_t* tiles, int32_t* n_tiles,
                                                            int32_t* gemm_cnt, int n_gemm_cnt) {
  zero_counters(gemm_cnt, n_gemm_cnt);  // the grouped GEMMs' hand-off counters
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

// Large batches use the LDS-tiled router GEMM (one tile per 64 tokens x 128 experts).
bool route_tiled(int T, int H) { return T >= 512 && H % 128 == 0; }

int route_ksplit(int T, int H, int E) {
  if (route_tiled(T, H)) {
    // about two workgroups per CU; K chunks of at least 256
    const int tiles = ((T + kRtT - 1) / kRtT) * ((E + kRtE - 1) / kRtE);
    int ks = (512 + tiles - 1) / tiles;
    const int kmax = H / 256 > 0 ? (H / 256 < kMaxKSplit ? H / 256 : kMaxKSplit) : 1;
    return ks < 1 ? 1 : (ks > kmax ? kmax : ks);
  }
  const int tiles = ((T + kRouterTileT - 1) / kRouterTileT) * ((E + kRouterBlockE - 1) / kRouterBlockE);
  int ks = (256 + tiles - 1) / tiles;
  // K chunks of at least 256, of 128 up to 16 tokens: there the router is latency-bound and the
  // shorter chunks help (30B layer: T=1 32.8 -> 31.6 us, T=8 72.8 -> 70.7 us; level from 64, where
  // the RMSNorm prologue would also repeat its row sums in twice the workgroups)
  const int kmin = T <= 16 ? 128 : 256;
  int kmax = H / kmin > 0 ? H / kmin : 1;
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

bool route_tiled_host(int T, int H) { return route_tiled(T, H); }

extern "C" size_t moe_mi355x_route_workspace_bytes(int T, int H, int E) {
  if (T <= 0 || H <= 0 || E <= 0) return 0;
  const int ks = route_ksplit(T, H, E);
  return moe_align_up((size_t)ks * T * E * sizeof(float), 256);
}

// What of the block path's routing depends on the batch size and can change the bits of the
// logits: the GEMM kernel (tiled or not) and the K chunks whose fp32 partials are summed.
int moe_route_numerics_key(int T, int H, int E, bool quant) {
  if (T <= 0 || H <= 0 || E <= 0) return 0;
  const int ks = route_ksplit(T, H, E);
  const bool tiled = route_tiled(T, H);
  const int kchunk = route_kchunk(H, ks, quant || tiled);
  return (tiled ? 1 << 16 : 0) | kchunk;
}

// Whether moe_launch_route can run the top-k and the expert sort as one workgroup.
bool moe_route_can_fuse_align(int T, int E, int k) {
  // one workgroup routes every token, so the whole top-k runs on one CU: a win over the
  // two-kernel path only while the batch is a handful of tokens
  return T <= 16 && (long)T * E <= kFusedMaxLogits && (long)T * k <= kSingleMaxS;
}

// Router GEMM alone: fp32 K-split partials [ks_eff, T, E] in the workspace (ks_eff returned),
// with xq/sx the x quantisation, with `zero` the nzero ints there cleared by workgroup 0.
int moe_launch_router_gemm(const void* x, const void* w_router, int T, int H, int E, void* workspace,
                           size_t workspace_bytes, hipStream_t s, uint8_t* xq, float* sx, int32_t* zero, int nzero,
                           int* ks_eff_out) {
  const bool quant = xq != nullptr;
  const int ks = route_ksplit(T, H, E);
  const bool tiled = route_tiled(T, H);
  const int kchunk = route_kchunk(H, ks, quant || tiled);
  const int ks_eff = (H + kchunk - 1) / kchunk;  // <= ks: the workspace holds ks partial slabs
  MOE_RETURN_IF(workspace_bytes < moe_mi355x_route_workspace_bytes(T, H, E) || !workspace, MOE_ERR_WORKSPACE);
  float* part = (float*)workspace;
  if (tiled) {
    dim3 g1((T + kRtT - 1) / kRtT, (E + kRtE - 1) / kRtE, ks_eff);
    MOE_LAUNCH(MOE_PROF_ROUTER_GEMM, s, router_gemm_tiled_kernel, g1, dim3(256), 0, s, (const uint16_t*)x,
               (const uint16_t*)w_router, T, H, E, kchunk, part, xq, sx, zero, nzero);
  } else {
    dim3 g1((T + kRouterTileT - 1) / kRouterTileT, (E + kRouterBlockE - 1) / kRouterBlockE, ks_eff);
    MOE_LAUNCH(MOE_PROF_ROUTER_GEMM, s, router_gemm_kernel, g1, dim3(256), 0, s, (const uint16_t*)x,
               (const uint16_t*)w_router, T, H, E, kchunk, part, xq, sx, zero, nzero);
  }
  MOE_CHECK_LAUNCH();
  *ks_eff_out = ks_eff;
  return MOE_OK;
}

// Router GEMM and top-k softmax.  With xq/sx the router workgroups also quantise x
// (needs H % 128 == 0).  With perm != nullptr (moe_route_can_fuse_align) the top-k and the expert
// sort run fused in one workgroup and write the align outputs too.
int moe_launch_route(const void* x, const void* w_router, int T, int H, int E, int k, int renorm,
                     void* logits, void* ids, int id_bytes, void* weights, void* workspace,
                     size_t workspace_bytes, hipStream_t s, uint8_t* xq, float* sx, int block_m,
                     int32_t* perm, int32_t* counts, int32_t* offsets, int32_t* tiles, int32_t* n_tiles,
                     int32_t* chunk_counts, int32_t* gemm_cnt, int n_gemm_cnt) {
  if (T == 0) return MOE_OK;
  const bool quant = xq != nullptr;
  MOE_RETURN_IF(chunk_counts != nullptr && perm != nullptr, MOE_ERR_INVALID_ARG);
  const int nzero = chunk_counts ? (int)(((long)T * k + kChunk - 1) / kChunk) * (E + 1) : 0;
  MOE_RETURN_IF(quant && H % MOE_GROUP, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(perm != nullptr && !moe_route_can_fuse_align(T, E, k), MOE_ERR_INVALID_ARG);
  int ks_eff = 0;
  int rc = moe_launch_router_gemm(x, w_router, T, H, E, workspace, workspace_bytes, s, xq, sx, chunk_counts, nzero,
                                  &ks_eff);
  if (rc) return rc;
  float* part = (float*)workspace;
  if (perm != nullptr) {
    MOE_LAUNCH(MOE_PROF_TOPK, s, topk_align_kernel, dim3(1), dim3(kChunk), 0, s, part, ks_eff, T, E, k, renorm,
               (uint16_t*)logits, ids, id_bytes, (uint16_t*)weights, block_m, perm, counts, offsets, tiles,
               n_tiles, gemm_cnt, n_gemm_cnt);
  } else {
    MOE_LAUNCH(MOE_PROF_TOPK, s, topk_softmax_kernel, dim3((T + 3) / 4), dim3(256), 0, s, part, ks_eff,
               (const uint16_t*)nullptr, T, E, k, renorm, (uint16_t*)logits, ids, id_bytes, (uint16_t*)weights,
               chunk_counts, (int32_t*)nullptr, (int32_t*)nullptr, (int32_t*)nullptr, (int32_t*)nullptr);
  }
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}

// Router GEMM (clearing the nzero ints at `zero`, which must cover ecnt [E + 1]), then the top-k
// with the expert buckets (bucket [E, T]) and the 16-row decode tile list (tiles, n_tiles).
int moe_launch_route_buckets(const void* x, const void* w_router, int T, int H, int E, int k, int renorm,
                             void* logits, void* ids, int id_bytes, void* weights, void* workspace,
                             size_t workspace_bytes, hipStream_t s, uint8_t* xq, float* sx, int32_t* zero, int nzero,
                             int32_t* ecnt, int32_t* bucket, int32_t* tiles, int32_t* n_tiles) {
  int ks_eff = 0;
  int rc = moe_launch_router_gemm(x, w_router, T, H, E, workspace, workspace_bytes, s, xq, sx, zero, nzero, &ks_eff);
  if (rc) return rc;
  MOE_LAUNCH(MOE_PROF_TOPK, s, topk_softmax_kernel, dim3((T + 3) / 4), dim3(256), 0, s, (const float*)workspace,
             ks_eff, (const uint16_t*)nullptr, T, E, k, renorm, (uint16_t*)logits, ids, id_bytes, (uint16_t*)weights,
             (int32_t*)nullptr, ecnt, bucket, tiles, n_tiles);
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
                          nullptr, nullptr, nullptr, nullptr, 0);
}

extern "C" int moe_mi355x_topk_softmax(const void* logits, int T, int E, int k, int renorm, void* ids,
                                       int id_bytes, void* weights, void* stream) {
  MOE_RETURN_IF(!route_args_ok(T, 32, E, k, id_bytes), MOE_ERR_INVALID_ARG);
  if (T == 0) return MOE_OK;
  MOE_RETURN_IF(!logits || !ids || !weights, MOE_ERR_INVALID_ARG);
  MOE_LAUNCH(MOE_PROF_TOPK, (hipStream_t)stream, topk_softmax_kernel, dim3((T + 3) / 4), dim3(256), 0,
             (hipStream_t)stream, (const float*)nullptr, 0, (const uint16_t*)logits, T, E, k, renorm,
             (uint16_t*)nullptr, ids, id_bytes, (uint16_t*)weights, (int32_t*)nullptr, (int32_t*)nullptr,
             (int32_t*)nullptr, (int32_t*)nullptr, (int32_t*)nullptr);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}
