// Expert sort / align: stable counting sort of the T*k (token, slot) pairs by
// expert id, per-expert counts and offsets, and the block_m-row tile list the
// grouped GEMMs iterate over.
//
// Reference: TF/integrations/moe.py:389-403 (torch.sort, histc, cumsum).
//
// Stability comes from wave ballots: lanes holding the same expert id are
// found with one ballot per id bit, a lane's rank among them is the popcount of
// that mask below its own lane, and per-wave totals are scanned in LDS in wave
// order.  Pairs are processed in 1024-pair chunks in index order, so the result
// equals a stable argsort.
//
// Ids outside [0, E) are expert-parallel sentinels (moe.py:405-419): they are left
// out of counts and tiles and placed, stably, after offsets[E] at the tail of perm.
#include "align_dev.h"

namespace {

// Whole align in one workgroup (small S: decode batches).
__global__ __launch_bounds__(kChunk) void align_single_kernel(const void* ids, int id_bytes, int S, int E,
                                                              int block_m, int32_t* perm, int32_t* counts,
                                                              int32_t* offsets, int32_t* tiles,
                                                              int32_t* n_tiles, int32_t* zero, int nzero) {
  zero_counters(zero, nzero);
  __shared__ int s_cnt[kBuckets];
  __shared__ int s_off[kBuckets];
  __shared__ int s_toff[kBuckets];
  __shared__ int s_wcnt[kWaves][kBuckets];
  for (int e = threadIdx.x; e <= E; e += blockDim.x) s_cnt[e] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < S; i += blockDim.x) atomicAdd(&s_cnt[bucket_of(ids, id_bytes, i, E)], 1);
  __syncthreads();
  scan_counts(s_cnt, E, block_m, s_off, s_toff);
  __syncthreads();
  emit_meta(s_cnt, s_off, s_toff, E, block_m, counts, offsets, tiles, n_tiles);
  // s_off doubles as the running base from here on; s_off[E] starts the sentinel tail
  for (int c0 = 0; c0 < S; c0 += kChunk) scatter_chunk(ids, id_bytes, S, E, c0, s_off, s_wcnt, perm);
}

// Large S, pass 1: per-chunk histograms  bc[b, e].
__global__ __launch_bounds__(kChunk) void align_count_kernel(const void* ids, int id_bytes, int S, int E,
                                                             int32_t* bc) {
  __shared__ int s_cnt[kBuckets];
  for (int e = threadIdx.x; e <= E; e += blockDim.x) s_cnt[e] = 0;
  __syncthreads();
  const int i = blockIdx.x * kChunk + threadIdx.x;
  if (i < S) atomicAdd(&s_cnt[bucket_of(ids, id_bytes, i, E)], 1);
  __syncthreads();
  for (int e = threadIdx.x; e <= E; e += blockDim.x) bc[(long)blockIdx.x * (E + 1) + e] = s_cnt[e];
}

// Large S, pass 2 (one launch): every workgroup reduces all chunk histograms (its
// chunk's starting slot per expert = offset of the expert + counts of the earlier chunks),
// workgroup 0 writes counts, offsets and the tile list, and each places its chunk stably.
__global__ __launch_bounds__(kChunk) void align_scan_scatter_kernel(const void* ids, int id_bytes, int S, int E,
                                                                    int block_m, const int32_t* __restrict__ bc,
                                                                    int nb, int32_t* perm, int32_t* counts,
                                                                    int32_t* offsets, int32_t* tiles,
                                                                    int32_t* n_tiles, int32_t* zero, int nzero) {
  if (blockIdx.x == 0) zero_counters(zero, nzero);
  __shared__ int s_cnt[kBuckets];
  __shared__ int s_off[kBuckets];
  __shared__ int s_toff[kBuckets];
  __shared__ int s_base[kBuckets];
  __shared__ int s_wcnt[kWaves][kBuckets];
  const int b = blockIdx.x;
  for (int e = threadIdx.x; e <= E; e += blockDim.x) {
    int tot = 0, pre = 0;
#pragma unroll 8
    for (int c = 0; c < nb; ++c) {
      const int v = bc[(long)c * (E + 1) + e];
      tot += v;
      pre += c < b ? v : 0;
    }
    s_cnt[e] = tot;
    s_base[e] = pre;
  }
  __syncthreads();
  scan_counts(s_cnt, E, block_m, s_off, s_toff);
  __syncthreads();
  if (b == 0) emit_meta(s_cnt, s_off, s_toff, E, block_m, counts, offsets, tiles, n_tiles);
  for (int e = threadIdx.x; e <= E; e += blockDim.x) s_base[e] += s_off[e];
  __syncthreads();
  scatter_chunk(ids, id_bytes, S, E, b * kChunk, s_base, s_wcnt, perm);
}

}  // namespace

extern "C" int moe_mi355x_align_max_tiles(int S, int E, int block_m) {
  if (S <= 0 || E <= 0 || block_m <= 0) return 0;
  return S / block_m + (S < E ? S : E);
}

extern "C" size_t moe_mi355x_align_workspace_bytes(int S, int E) {
  if (S <= kAlignOneWgMaxS) return 0;
  const size_t nb = (S + kChunk - 1) / kChunk;
  return moe_align_up(nb * (E + 1) * sizeof(int32_t), 256);
}

int moe_launch_align_counted(const void* ids, int id_bytes, int S, int E, int block_m, const int32_t* bc,
                             int32_t* perm, int32_t* counts, int32_t* offsets, int32_t* tiles, int32_t* n_tiles,
                             hipStream_t s, int32_t* zero, int nzero);

// `zero` / `nzero`: counters of the grouped GEMMs' hand-offs, cleared by the align kernel.
int moe_launch_align(const void* ids, int id_bytes, int S, int E, int block_m, int32_t* perm,
                     int32_t* counts, int32_t* offsets, int32_t* tiles, int32_t* n_tiles, void* workspace,
                     size_t workspace_bytes, hipStream_t s, int32_t* zero, int nzero) {
  if (S <= kAlignOneWgMaxS) {
    MOE_LAUNCH(MOE_PROF_ALIGN, s, align_single_kernel, dim3(1), dim3(kChunk), 0, s, ids, id_bytes, S, E, block_m, perm,
                       counts, offsets, tiles, n_tiles, zero, nzero);
    MOE_CHECK_LAUNCH();
    return MOE_OK;
  }
  MOE_RETURN_IF(!workspace || workspace_bytes < moe_mi355x_align_workspace_bytes(S, E), MOE_ERR_WORKSPACE);
  const int nb = (S + kChunk - 1) / kChunk;
  int32_t* bc = (int32_t*)workspace;
  MOE_LAUNCH(MOE_PROF_ALIGN, s, align_count_kernel, dim3(nb), dim3(kChunk), 0, s, ids, id_bytes, S, E, bc);
  MOE_CHECK_LAUNCH();
  return moe_launch_align_counted(ids, id_bytes, S, E, block_m, bc, perm, counts, offsets, tiles, n_tiles, s, zero,
                                  nzero);
}

// The rest of the large-S align once the chunk histograms bc [nb, E + 1] are filled (by
// align_count_kernel, or by the top-k kernel of the block path).
int moe_launch_align_counted(const void* ids, int id_bytes, int S, int E, int block_m, const int32_t* bc,
                             int32_t* perm, int32_t* counts, int32_t* offsets, int32_t* tiles, int32_t* n_tiles,
                             hipStream_t s, int32_t* zero, int nzero) {
  const int nb = (S + kChunk - 1) / kChunk;
  MOE_LAUNCH(MOE_PROF_ALIGN, s, align_scan_scatter_kernel, dim3(nb), dim3(kChunk), 0, s, ids, id_bytes, S, E,
             block_m, bc, nb, perm, counts, offsets, tiles, n_tiles, zero, nzero);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}

extern "C" int moe_mi355x_align(const void* ids, int id_bytes, int T, int k, int E, int block_m,
                                int32_t* perm, int32_t* counts, int32_t* offsets, int32_t* tiles,
                                int32_t* n_tiles, void* workspace, size_t workspace_bytes, void* stream) {
  MOE_RETURN_IF(T < 0 || k < 1 || E < 1 || E > kMaxE || block_m < 1, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(id_bytes != 4 && id_bytes != 8, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!counts || !offsets || !n_tiles, MOE_ERR_INVALID_ARG);
  const long S = (long)T * k;
  MOE_RETURN_IF(S > (1L << 30), MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(S > 0 && (!ids || !perm || !tiles), MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!moe_aligned16(tiles), MOE_ERR_ALIGNMENT);
  return moe_launch_align(ids, id_bytes, (int)S, E, block_m, perm, counts, offsets, tiles, n_tiles, workspace,
                          workspace_bytes, (hipStream_t)stream, nullptr, 0);
}
