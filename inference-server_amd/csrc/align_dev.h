// Building blocks of the expert sort / align (stable counting sort with wave ballots),
// shared by the align kernels and the fused top-k + align kernel.
#pragma once

#include "common.h"

namespace {

constexpr int kChunk = 1024;       // pairs per chunk == threads per workgroup
constexpr int kWaves = kChunk / MOE_WAVE;
constexpr int kMaxE = 256;
constexpr int kBuckets = kMaxE + 1;  // experts plus the sentinel bucket

__device__ __forceinline__ int bucket_of(const void* ids, int id_bytes, int i, int E) {
  const long r = id_bytes == 8 ? (long)((const int64_t*)ids)[i] : (long)((const int32_t*)ids)[i];
  return (r < 0 || r >= E) ? E : (int)r;
}
constexpr int kSingleMaxS = 4096;  // pairs the one-workgroup top-k + sort kernel can hold
// Above this many pairs the standalone sort runs on one workgroup per 1024-pair chunk (chunk
// histograms, then a scan + stable scatter per chunk) instead of one workgroup: 512 tokens x 8
// slots 13.5 -> 7.6 us.
constexpr int kAlignOneWgMaxS = 2048;

// Exclusive scans of counts and of ceil(count / block_m) over experts; wave 0 of the block.
__device__ void scan_counts(const int* s_cnt, int E, int block_m, int* s_off, int* s_toff) {
  const int lane = threadIdx.x & 63;
  if ((threadIdx.x >> 6) != 0) return;
  int c[4], t[4], sc = 0, st = 0;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = lane * 4 + q;
    c[q] = e < E ? s_cnt[e] : 0;
    t[q] = (c[q] + block_m - 1) / block_m;
    sc += c[q];
    st += t[q];
  }
  int ic = sc, it = st;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int oc = __shfl_up(ic, d, MOE_WAVE), ot = __shfl_up(it, d, MOE_WAVE);
    if (lane >= d) {
      ic += oc;
      it += ot;
    }
  }
  int ec = ic - sc, et = it - st;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = lane * 4 + q;
    if (e < E) {
      s_off[e] = ec;
      s_toff[e] = et;
    }
    ec += c[q];
    et += t[q];
  }
  if (lane == 63) {
    s_off[E] = ic;
    s_toff[E] = it;
  }
}

// Zeroes the n counters at `zero` (the grouped GEMMs' hand-off counters, which the align of the
// same call clears so that no earlier call can leave them dirty).
__device__ __forceinline__ void zero_counters(int32_t* zero, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) zero[i] = 0;
}

// Writes counts, offsets and the tile list from the scanned LDS arrays.
__device__ void emit_meta(const int* s_cnt, const int* s_off, const int* s_toff, int E, int block_m,
                          int32_t* counts, int32_t* offsets, int32_t* tiles, int32_t* n_tiles) {
  for (int e = threadIdx.x; e <= E; e += blockDim.x) {
    offsets[e] = s_off[e];
    if (e == E) {
      n_tiles[0] = s_toff[E];
      continue;
    }
    const int c = s_cnt[e];
    counts[e] = c;
    int tix = s_toff[e];
    for (int r = 0; r < c; r += block_m, ++tix) {
      int4 v = make_int4(e, s_off[e] + r, min(block_m, c - r), 0);
      *(int4*)(tiles + 4 * tix) = v;
    }
  }
}

// Stable placement of one chunk of pairs [chunk0, chunk0 + 1024).  s_base holds the
// next free sorted slot of every expert and is advanced by the chunk's counts.
__device__ void scatter_chunk(const void* ids, int id_bytes, int S, int E, int chunk0, int* s_base,
                              int (*s_wcnt)[kBuckets], int32_t* perm) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int i = chunk0 + threadIdx.x;
  const bool valid = i < S;
  const int e = valid ? bucket_of(ids, id_bytes, i, E) : E + 1;  // E + 1 marks a lane with no pair
  for (int x = lane; x <= E; x += MOE_WAVE) s_wcnt[wave][x] = 0;
  __syncthreads();
  uint64_t mask = __ballot(1);
#pragma unroll
  for (int b = 0; b < 9; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t bal = __ballot(bit);
    mask &= bit ? bal : ~bal;
  }
  const int rank = __popcll(mask & lanemask_lt());
  if (valid && rank == 0) s_wcnt[wave][e] = __popcll(mask);
  __syncthreads();
  if (valid) {
    int prefix = 0;
    for (int w = 0; w < wave; ++w) prefix += s_wcnt[w][e];
    perm[s_base[e] + prefix + rank] = i;
  }
  __syncthreads();
  for (int x = threadIdx.x; x <= E; x += blockDim.x) {
    int tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot += s_wcnt[w][x];
    s_base[x] += tot;
  }
  __syncthreads();
}

}  // namespace
