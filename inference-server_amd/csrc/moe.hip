// Experts / block entry points: activation quantisation -> align -> gate_up GEMM
// (fused SiLU*up) -> intermediate quantisation -> down GEMM (fused routing-weight
// product and inverse permutation) -> deterministic top-k combine.
//
// Reference: fp8_grouped_mm_experts_forward, TF/integrations/finegrained_fp8.py:498-589,
// and Qwen3MoeSparseMoeBlock.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:276-281.
#include <mutex>

#include "common.h"

int moe_gemm_block_m(int S, int E, int H, int I);
int moe_down_col_blocks(int S, int H, int block_m);
int moe_launch_grouped_gemms(const uint8_t* xq, const float* sx, const uint8_t* w13, const float* s13,
                             const uint8_t* w2, const float* s2, const int32_t* perm, const int32_t* tiles,
                             const int32_t* n_tiles, int max_tiles, const uint16_t* topk_w, uint16_t* h,
                             uint8_t* hq, float* sh, uint16_t* pairs, int S, int H, int I, int k,
                             int block_m, hipStream_t s, int32_t* tile_cnt, int32_t* tok_cnt, uint16_t* comb,
                             const uint16_t* residual);
bool route_tiled_host(int T, int H);
int moe_launch_router_gemm(const void* x, const void* w_router, int T, int H, int E, void* workspace,
                           size_t workspace_bytes, hipStream_t s, uint8_t* xq, float* sx, int32_t* zero, int nzero,
                           int* ks_eff_out);
int moe_launch_grouped_gemms_routed(const uint8_t* xq, const float* sx, const uint8_t* w13, const float* s13,
                                    const uint8_t* w2, const float* s2, const float* part, int ksplit, int T, int E,
                                    int renorm, uint16_t* logits, void* ids, int id_bytes, uint16_t* wts,
                                    int32_t* perm, int32_t* tiles, int32_t* n_tiles, uint16_t* h, uint8_t* hq,
                                    float* sh, uint16_t* pairs, int H, int I, int k, hipStream_t s, int32_t* tile_cnt,
                                    int32_t* tok_cnt, uint16_t* comb, const uint16_t* residual);
int moe_launch_route_buckets(const void* x, const void* w_router, int T, int H, int E, int k, int renorm,
                             void* logits, void* ids, int id_bytes, void* weights, void* workspace,
                             size_t workspace_bytes, hipStream_t s, uint8_t* xq, float* sx, int32_t* zero, int nzero,
                             int32_t* ecnt, int32_t* bucket, int32_t* tiles, int32_t* n_tiles);
int moe_launch_grouped_gemms_buckets(const uint8_t* xq, const float* sx, const uint8_t* w13, const float* s13,
                                     const uint8_t* w2, const float* s2, const int32_t* bucket, const int32_t* tiles,
                                     const int32_t* n_tiles, int T, int max_tiles, const uint16_t* topk_w,
                                     uint16_t* h, uint8_t* hq, float* sh, uint16_t* pairs, int H, int I, int k,
                                     hipStream_t s, int32_t* tile_cnt, int32_t* tok_cnt, uint16_t* comb,
                                     const uint16_t* residual);
int moe_launch_route(const void* x, const void* w_router, int T, int H, int E, int k, int renorm,
                     void* logits, void* ids, int id_bytes, void* weights, void* workspace,
                     size_t workspace_bytes, hipStream_t s, uint8_t* xq, float* sx, int block_m,
                     int32_t* perm, int32_t* counts, int32_t* offsets, int32_t* tiles, int32_t* n_tiles,
                     int32_t* chunk_counts, int32_t* gemm_cnt, int n_gemm_cnt);
int moe_launch_align_counted(const void* ids, int id_bytes, int S, int E, int block_m, const int32_t* bc,
                             int32_t* perm, int32_t* counts, int32_t* offsets, int32_t* tiles, int32_t* n_tiles,
                             hipStream_t s, int32_t* zero, int nzero);
extern "C" size_t moe_mi355x_route_workspace_bytes(int T, int H, int E);
bool moe_route_can_fuse_align(int T, int E, int k);
extern "C" int moe_mi355x_align_max_tiles(int S, int E, int block_m);
extern "C" size_t moe_mi355x_align_workspace_bytes(int S, int E);

namespace {

// out[t, :] = bf16( sum_j pairs[t*k + j, :] ) with fp32 accumulation in slot order
// (moe.py:476 view(T,k,H).sum(1)); sentinel slots (ids outside [0,E)) add zero.
// `wts` (bf16 [T, k]) non-null: the pair rows hold bf16(z) and the routing weight is applied
// here, bf16(bf16(z) * w), the same rounding as a weighted pair row; null: already weighted.
// `residual` (bf16 [T, H]) non-null: out = bf16(residual + bf16(sum)), the decoder layer's
// residual add after the MoE block (TF/models/qwen3_moe/modeling_qwen3_moe.py:347).
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ pairs, const void* ids,
                                                      int id_bytes, const uint16_t* __restrict__ wts, int T,
                                                      int k, int H, int E, const uint16_t* __restrict__ residual,
                                                      uint16_t* __restrict__ out) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int per_row = H / 8;
  if (idx >= (long)T * per_row) return;
  const int t = (int)(idx / per_row), c8 = (int)(idx % per_row);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  // rows are loaded unconditionally (a sentinel slot's row exists, unwritten) and masked
  // afterwards, so that the k loads are in flight together rather than one per branch
  constexpr int kUnroll = 8;
  // eight weights of a token in one 16-byte load when the rows allow it
  const bool wvec = wts != nullptr && (k & 7) == 0 && ((uintptr_t)wts & 15) == 0;
  for (int j0 = 0; j0 < k; j0 += kUnroll) {
    uint4 v[kUnroll];
    bool ok[kUnroll];
    float wt[kUnroll];
    if (wvec) {
      const uint4 w8 = *(const uint4*)(wts + (long)t * k + j0);
      const uint32_t ww[4] = {w8.x, w8.y, w8.z, w8.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wt[2 * i] = __uint_as_float(ww[i] << 16);
        wt[2 * i + 1] = __uint_as_float(ww[i] & 0xffff0000u);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int pr = t * k + min(j0 + u, k - 1);
      const long id = id_bytes == 8 ? (long)((const int64_t*)ids)[pr] : (long)((const int32_t*)ids)[pr];
      ok[u] = j0 + u < k && id >= 0 && id < E;
      if (!wvec) wt[u] = wts ? bf16_to_f32(wts[pr]) : 1.0f;
      v[u] = *(const uint4*)(pairs + (long)pr * H + c8 * 8);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float lo = __uint_as_float(w[i] << 16), hi = __uint_as_float(w[i] & 0xffff0000u);
        if (wts) {
          lo = round_bf16(lo * wt[u]);
          hi = round_bf16(hi * wt[u]);
        }
        acc[2 * i] += ok[u] ? lo : 0.f;
        acc[2 * i + 1] += ok[u] ? hi : 0.f;
      }
    }
  }
  if (residual != nullptr) {
    const uint4 rv = *(const uint4*)(residual + (long)t * H + c8 * 8);
    const uint32_t ru[4] = {rv.x, rv.y, rv.z, rv.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc[2 * i] = __uint_as_float(ru[i] << 16) + round_bf16(acc[2 * i]);
      acc[2 * i + 1] = __uint_as_float(ru[i] & 0xffff0000u) + round_bf16(acc[2 * i + 1]);
    }
  }
  uint4 o;
  o.x = (uint32_t)f32_to_bf16(acc[0]) | ((uint32_t)f32_to_bf16(acc[1]) << 16);
  o.y = (uint32_t)f32_to_bf16(acc[2]) | ((uint32_t)f32_to_bf16(acc[3]) << 16);
  o.z = (uint32_t)f32_to_bf16(acc[4]) | ((uint32_t)f32_to_bf16(acc[5]) << 16);
  o.w = (uint32_t)f32_to_bf16(acc[6]) | ((uint32_t)f32_to_bf16(acc[7]) << 16);
  *(uint4*)(out + (long)t * H + c8 * 8) = o;
}

}  // namespace

// out = bf16(sum_j pairs[t*k + j]) in slot order (+ residual), see combine_kernel.
int moe_launch_combine(const uint16_t* pairs, const void* ids, int id_bytes, const uint16_t* wts, int T, int k, int H,
                       int E, const uint16_t* residual, uint16_t* out, hipStream_t s) {
  const long threads = (long)T * (H / 8);
  MOE_RETURN_IF(!moe_grid_fits((threads + 255) / 256), MOE_ERR_INVALID_ARG);
  MOE_LAUNCH(MOE_PROF_COMBINE, s, combine_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, pairs, ids,
             id_bytes, wts, T, k, H, E, residual, out);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}

namespace {

struct ExpertsWs {
  uint8_t* xq;
  float* sx;
  int32_t* perm;
  int32_t* counts;
  int32_t* offsets;
  int32_t* tiles;
  int32_t* n_tiles;
  void* align_ws;
  size_t align_ws_bytes;
  uint16_t* h;
  uint8_t* hq;
  float* sh;
  uint16_t* pairs;
  int32_t* cnt;    // 16-row tiles: the GEMMs' hand-off counters, [max_tiles, I/128] then [T, down column blocks]
  int n_cnt;       // 0 on the other paths
  int32_t* ecnt;   // 16-row tiles: expert bucket counts [E] and a workgroup count, after the n_cnt counters
  int n_ecnt;
  int32_t* bucket; // 16-row tiles: expert buckets [E, T] of pair indices
  size_t total;
  int block_m;
  int max_tiles;
};

ExpertsWs carve_experts(void* base, int T, int H, int I, int E, int k) {
  ExpertsWs w{};
  const int S = T * k;
  w.block_m = moe_gemm_block_m(S, E, H, I);
  w.max_tiles = moe_mi355x_align_max_tiles(S, E, w.block_m);
  WsCarver c(base);
  w.xq = c.take<uint8_t>((size_t)T * H);
  w.sx = c.take<float>((size_t)T * (H / MOE_GROUP));
  w.perm = c.take<int32_t>(S);
  w.counts = c.take<int32_t>(E);
  w.offsets = c.take<int32_t>(E + 1);
  w.tiles = c.take<int32_t>((size_t)4 * (w.max_tiles > 0 ? w.max_tiles : 1));
  w.n_tiles = c.take<int32_t>(4);
  w.align_ws_bytes = moe_mi355x_align_workspace_bytes(S, E);
  w.align_ws = c.take<char>(w.align_ws_bytes);
  w.h = c.take<uint16_t>(w.block_m >= 128 ? 0 : (size_t)S * I);  // the prefill GEMM quantises h in place
  w.hq = c.take<uint8_t>((size_t)S * I);
  w.sh = c.take<float>((size_t)S * (I / MOE_GROUP));
  w.pairs = c.take<uint16_t>((size_t)S * H);
  w.n_cnt = w.block_m != 16 ? 0 : w.max_tiles * (I / MOE_GROUP) + T * moe_down_col_blocks(S, H, w.block_m);
  w.n_ecnt = w.block_m != 16 ? 0 : E + 1;  // the bucket counts and the top-k's workgroup count
  w.cnt = c.take<int32_t>(w.n_cnt + w.n_ecnt);  // one range, cleared by one launch
  w.ecnt = w.cnt ? w.cnt + w.n_cnt : nullptr;
  w.bucket = c.take<int32_t>(w.block_m != 16 ? 0 : (size_t)E * T);
  w.total = moe_align_up(c.off, 256);
  return w;
}

bool experts_args_ok(int T, int H, int I, int E, int k, int id_bytes) {
  return T >= 0 && H > 0 && I > 0 && H % MOE_GROUP == 0 && I % MOE_GROUP == 0 && H <= 4096 && I <= 4096 &&
         E >= 1 && E <= 256 && k >= 1 && k <= 32 && k <= E && (id_bytes == 4 || id_bytes == 8) &&
         (long)T * k < (1L << 28);
}

// Experts after routing.  `prepared` = x already quantised into w.xq/w.sx and the align
// outputs already written, hand-off counters cleared (the block path fuses all of it into its
// routing kernels).  `ids_valid`: every id is in [0, E) (the block path's own routing), so on
// decode tiles the down GEMM combines each token itself; caller ids may hold expert-parallel
// sentinels and go through the combine kernel.
int launch_experts(const void* x, const void* ids, int id_bytes, const void* weights, int T, int H, int I,
                   int E, int k, const void* w13, const float* s13, const void* w2, const float* s2, void* out,
                   const ExpertsWs& w, hipStream_t s, bool prepared = false, const void* residual = nullptr,
                   bool ids_valid = false) {
  const int S = T * k;
  int rc;
  if (!prepared) {
    rc = moe_launch_quant_act(x, T, H, w.xq, w.sx, s);
    if (rc) return rc;
    rc = moe_launch_align(ids, id_bytes, S, E, w.block_m, w.perm, w.counts, w.offsets, w.tiles, w.n_tiles,
                          w.align_ws, w.align_ws_bytes, s, w.cnt, w.n_cnt);
    if (rc) return rc;
  }
  // the hand-offs pay on 16-row tiles (batches up to 8 pairs per expert): fewer launches outweigh
  // each workgroup's wait for its stores; on 32-row tiles the separate launches are faster
  // (Qwen3-30B-A3B layer at 256 tokens: 163 against 172 us).  The h quantisation's hand-off pays
  // only up to 2 pairs per expert: above, the separate quant_h launch is faster (64 tokens: 130.5
  // against 133 us, 128 tokens: 141 against 144 us; level at 8-32 tokens)
  const bool decode = w.block_m == 16;
  const bool quant_handoff = decode && S <= 2 * E;
  const bool fused_combine = decode && ids_valid;
  rc = moe_launch_grouped_gemms(w.xq, w.sx, (const uint8_t*)w13, s13, (const uint8_t*)w2, s2, w.perm, w.tiles,
                                w.n_tiles, w.max_tiles, (const uint16_t*)weights, w.h, w.hq, w.sh, w.pairs, S, H,
                                I, k, w.block_m, s, quant_handoff ? w.cnt : nullptr,
                                fused_combine ? w.cnt + (long)w.max_tiles * (I / MOE_GROUP) : nullptr, (uint16_t*)out,
                                (const uint16_t*)residual);
  if (rc) return rc;
  if (fused_combine) return MOE_OK;
  return moe_launch_combine(w.pairs, ids, id_bytes, w.block_m >= 128 ? (const uint16_t*)weights : nullptr, T, k, H,
                            E, (const uint16_t*)residual, (uint16_t*)out, s);
}

bool experts_ptrs_ok(const void* x, const void* ids, const void* weights, const void* w13, const float* s13,
                     const void* w2, const float* s2, const void* out) {
  return x && ids && weights && w13 && s13 && w2 && s2 && out;
}

bool experts_aligned(const void* x, const void* w13, const void* w2, const void* out) {
  return moe_aligned16(x) && moe_aligned16(w13) && moe_aligned16(w2) && moe_aligned16(out);
}

}  // namespace

extern "C" const char* moe_mi355x_error_string(int code) {
  switch (code) {
    case MOE_OK: return "success";
    case MOE_ERR_INVALID_ARG: return "invalid argument (null pointer, size or unsupported shape)";
    case MOE_ERR_WORKSPACE: return "workspace missing or smaller than the *_workspace_bytes() size";
    case MOE_ERR_ALIGNMENT: return "a tensor pointer is not 16-byte aligned";
    case MOE_ERR_SCRATCH:
      return "the call needs more scratch than the no-allocation entry point's fixed device buffer holds "
             "(moe_mi355x_block_fp8_noalloc_scratch_bytes); use moe_mi355x_block_fp8 with a workspace";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}

// 0.2: num_pages added to the paged-attention, KV-append and q/k-norm-rope-append entry points.
extern "C" int moe_mi355x_version(void) { return (0 << 16) | 2; }

extern "C" size_t moe_mi355x_experts_workspace_bytes(int T, int H, int I, int E, int k) {
  if (!experts_args_ok(T, H, I, E, k, 4)) return 0;
  return carve_experts(nullptr, T, H, I, E, k).total;
}

extern "C" int moe_mi355x_experts_fp8(const void* x, const void* ids, int id_bytes, const void* weights, int T,
                                      int H, int I, int E, int k, const void* w13, const float* s13,
                                      const void* w2, const float* s2, void* out, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  MOE_RETURN_IF(!experts_args_ok(T, H, I, E, k, id_bytes), MOE_ERR_INVALID_ARG);
  if (T == 0) return MOE_OK;
  MOE_RETURN_IF(!experts_ptrs_ok(x, ids, weights, w13, s13, w2, s2, out), MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!experts_aligned(x, w13, w2, out), MOE_ERR_ALIGNMENT);
  const ExpertsWs w = carve_experts(workspace, T, H, I, E, k);
  MOE_RETURN_IF(!workspace || workspace_bytes < w.total, MOE_ERR_WORKSPACE);
  return launch_experts(x, ids, id_bytes, weights, T, H, I, E, k, w13, s13, w2, s2, out, w, (hipStream_t)stream);
}

namespace {
struct BlockWs {
  void* route_ws;
  size_t route_bytes;
  uint16_t* logits;
  int32_t* ids;
  uint16_t* weights;
  void* experts_ws;
  size_t experts_bytes;
  size_t total;
};

BlockWs carve_block(void* base, int T, int H, int I, int E, int k) {
  BlockWs b{};
  WsCarver c(base);
  b.route_bytes = moe_mi355x_route_workspace_bytes(T, H, E);
  b.route_ws = c.take<char>(b.route_bytes);
  b.logits = c.take<uint16_t>((size_t)T * E);
  b.ids = c.take<int32_t>((size_t)T * k);
  b.weights = c.take<uint16_t>((size_t)T * k);
  b.experts_bytes = carve_experts(nullptr, T, H, I, E, k).total;
  b.experts_ws = c.take<char>(b.experts_bytes);
  b.total = moe_align_up(c.off, 256);
  return b;
}
}  // namespace

extern "C" size_t moe_mi355x_block_workspace_bytes(int T, int H, int I, int E, int k) {
  if (!experts_args_ok(T, H, I, E, k, 4)) return 0;
  return carve_block(nullptr, T, H, I, E, k).total;
}

namespace {
// Batches of up to 4 tokens skip the top-k + sort launch: every routing slot is its own one-row
// tile and the gate_up GEMM routes it (the bits of the sorted path).  Two slots that name one
// expert then stream its weights twice, which costs more than the launch saves from 5 tokens on
// (Qwen3-30B-A3B layer: 1 / 2 / 4 tokens 31.7 / 38.1 / 50.8 -> 28.9 / 34.8 / 49.4 us; 5 / 8 tokens
// 54.2 / 68.3 -> 56.1 / 75.6 us).
// The slots are the tiles, so S = T k must fit the tile list and counters carved for at most
// min(S, E) + S / 16 tiles: S <= E.
constexpr int kRoutedMaxTokens = 4;
bool routed_path(int T, int H, int E, int k, int block_m) {
  return T <= kRoutedMaxTokens && block_m == 16 && T * k <= E && E <= 256 && !route_tiled_host(T, H);
}

// Router + experts; `residual` non-null adds it in the combine (moe_mi355x_moe_sublayer_fp8).
int block_impl(const void* x, const void* w_router, int T, int H, int I, int E, int k, int renorm, const void* w13,
               const float* s13, const void* w2, const float* s2, void* out, void* logits, void* ids, int id_bytes,
               void* weights, const BlockWs& b, hipStream_t s, const void* residual) {
  void* lg = logits ? logits : (void*)b.logits;
  void* id_out = ids ? ids : (void*)b.ids;
  const int idb = ids ? id_bytes : 4;
  void* wt = weights ? weights : (void*)b.weights;
  const ExpertsWs w = carve_experts(b.experts_ws, T, H, I, E, k);
  if (routed_path(T, H, E, k, w.block_m)) {
    // router GEMM (clearing the GEMMs' hand-off counters), then gate_up routing its own slots
    int ks_eff = 0;
    int rc = moe_launch_router_gemm(x, w_router, T, H, E, b.route_ws, b.route_bytes, s, w.xq, w.sx, w.cnt, w.n_cnt,
                                    &ks_eff);
    if (rc) return rc;
    return moe_launch_grouped_gemms_routed(w.xq, w.sx, (const uint8_t*)w13, s13, (const uint8_t*)w2, s2,
                                           (const float*)b.route_ws, ks_eff, T, E, renorm, (uint16_t*)lg, id_out, idb,
                                           (uint16_t*)wt, w.perm, w.tiles, w.n_tiles, w.h, w.hq, w.sh, w.pairs, H, I,
                                           k, s, w.cnt, w.cnt + (long)w.max_tiles * (I / MOE_GROUP), (uint16_t*)out,
                                           (const uint16_t*)residual);
  }
  if (w.block_m == 16) {
    // decode tiles: router GEMM (clearing the GEMMs' hand-off counters and the bucket counts), top-k
    // into expert buckets, then the GEMMs on bucket tiles; no sort launch
    int rc = moe_launch_route_buckets(x, w_router, T, H, E, k, renorm, lg, id_out, idb, wt, b.route_ws, b.route_bytes,
                                      s, w.xq, w.sx, w.cnt, w.n_cnt + w.n_ecnt, w.ecnt, w.bucket, w.tiles,
                                      w.n_tiles);
    if (rc) return rc;
    const bool quant_handoff = T * k <= 2 * E;
    return moe_launch_grouped_gemms_buckets(w.xq, w.sx, (const uint8_t*)w13, s13, (const uint8_t*)w2, s2, w.bucket,
                                            w.tiles, w.n_tiles, T, w.max_tiles, (const uint16_t*)wt, w.h, w.hq, w.sh,
                                            w.pairs, H, I, k, s, quant_handoff ? w.cnt : nullptr,
                                            w.cnt + (long)w.max_tiles * (I / MOE_GROUP), (uint16_t*)out,
                                            (const uint16_t*)residual);
  }
  // decode batches: x quantisation rides in the router GEMM, align in the top-k kernel; large
  // batches: the top-k kernel fills the expert sort's chunk histograms (cleared by the router
  // GEMM), and one launch finishes the sort
  const bool fused = moe_route_can_fuse_align(T, E, k);
  const bool counted = !fused && w.align_ws_bytes > 0;
  int rc = moe_launch_route(x, w_router, T, H, E, k, renorm, lg, id_out, idb, wt, b.route_ws, b.route_bytes, s,
                            w.xq, w.sx, w.block_m, fused ? w.perm : nullptr, w.counts, w.offsets, w.tiles,
                            w.n_tiles, counted ? (int32_t*)w.align_ws : nullptr, w.cnt, w.n_cnt);
  if (rc) return rc;
  if (counted) {
    rc = moe_launch_align_counted(id_out, idb, T * k, E, w.block_m, (const int32_t*)w.align_ws, w.perm, w.counts,
                                  w.offsets, w.tiles, w.n_tiles, s, w.cnt, w.n_cnt);
    if (rc) return rc;
  } else if (!fused) {
    rc = moe_launch_align(id_out, idb, T * k, E, w.block_m, w.perm, w.counts, w.offsets, w.tiles, w.n_tiles,
                          w.align_ws, w.align_ws_bytes, s, w.cnt, w.n_cnt);
    if (rc) return rc;
  }
  return launch_experts(x, id_out, idb, wt, T, H, I, E, k, w13, s13, w2, s2, out, w, s, /*prepared=*/true, residual,
                        /*ids_valid=*/true);
}
}  // namespace

int moe_route_numerics_key(int T, int H, int E, bool quant);
int moe_bf16_block_m(int S, int E, int H, int I);

extern "C" long long moe_mi355x_block_numerics_key(int T, int H, int I, int E, int k, int fp8) {
  if (!experts_args_ok(T, H, I, E, k, 4) || T == 0) return 0;
  const int bm = fp8 ? moe_gemm_block_m(T * k, E, H, I) : moe_bf16_block_m(T * k, E, H, I);
  return ((long long)moe_route_numerics_key(T, H, E, fp8 != 0) << 16) | bm;
}

extern "C" int moe_mi355x_block_fp8(const void* x, const void* w_router, int T, int H, int I, int E, int k,
                                    int renorm, const void* w13, const float* s13, const void* w2,
                                    const float* s2, void* out, void* logits, void* ids, int id_bytes,
                                    void* weights, void* workspace, size_t workspace_bytes, void* stream) {
  MOE_RETURN_IF(!experts_args_ok(T, H, I, E, k, id_bytes), MOE_ERR_INVALID_ARG);
  if (T == 0) return MOE_OK;
  MOE_RETURN_IF(!x || !w_router || !w13 || !s13 || !w2 || !s2 || !out, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!experts_aligned(x, w13, w2, out) || !moe_aligned16(w_router), MOE_ERR_ALIGNMENT);
  const BlockWs b = carve_block(workspace, T, H, I, E, k);
  MOE_RETURN_IF(!workspace || workspace_bytes < b.total, MOE_ERR_WORKSPACE);
  return block_impl(x, w_router, T, H, I, E, k, renorm, w13, s13, w2, s2, out, logits, ids, id_bytes, weights, b,
                    (hipStream_t)stream, nullptr);
}

int moe_launch_rms_norm(const void* x, const void* add, const void* w, int R, int C, float eps, void* out,
                        void* sum_out, hipStream_t s);

extern "C" size_t moe_mi355x_moe_sublayer_workspace_bytes(int T, int H, int I, int E, int k) {
  if (!experts_args_ok(T, H, I, E, k, 4)) return 0;
  return 2 * moe_align_up((size_t)T * H * 2, 256) + carve_block(nullptr, T, H, I, E, k).total;
}

extern "C" int moe_mi355x_moe_sublayer_fp8(const void* h, const void* h_add, const void* ln_weight, float eps,
                                           const void* w_router, int T, int H, int I, int E, int k, int renorm,
                                           const void* w13, const float* s13, const void* w2, const float* s2,
                                           void* out, void* workspace, size_t workspace_bytes, void* stream) {
  MOE_RETURN_IF(!experts_args_ok(T, H, I, E, k, 4), MOE_ERR_INVALID_ARG);
  if (T == 0) return MOE_OK;
  MOE_RETURN_IF(!h || !ln_weight || !w_router || !w13 || !s13 || !w2 || !s2 || !out, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!experts_aligned(h, w13, w2, out) || !moe_aligned16(w_router) || !moe_aligned16(ln_weight) ||
                    (h_add && !moe_aligned16(h_add)),
                MOE_ERR_ALIGNMENT);
  MOE_RETURN_IF(H > 8192, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!workspace || workspace_bytes < moe_mi355x_moe_sublayer_workspace_bytes(T, H, I, E, k),
                MOE_ERR_WORKSPACE);
  hipStream_t s = (hipStream_t)stream;
  const size_t row_bytes = moe_align_up((size_t)T * H * 2, 256);
  void* xn = workspace;                                 // the normalised rows
  void* hs = (char*)workspace + row_bytes;              // bf16(h + h_add), the residual
  const BlockWs b = carve_block((char*)workspace + 2 * row_bytes, T, H, I, E, k);
  // residual add + RMSNorm in one launch, then the block (router GEMM + x quantisation in one
  // launch).  Folding the RMSNorm into the router GEMM instead (each router workgroup summing its
  // rows' squares over the whole hidden width) was measured slower at every batch: 30B sublayer
  // at 1 / 8 / 64 / 128 / 256 tokens 36.9 / 75.2 / 138.3 / 147.5 / 172.8 us this way against
  // 39.8 / 77.9 / 145.0 / 154.9 / 182.4 us fused.
  int rc = moe_launch_rms_norm(h, h_add, ln_weight, T, H, eps, xn, h_add ? hs : nullptr, s);
  if (rc) return rc;
  return block_impl(xn, w_router, T, H, I, E, k, renorm, w13, s13, w2, s2, out, nullptr, nullptr, 4, nullptr, b, s,
                    h_add ? hs : h);
}

// ---------------------------------------------------------------------------
// No-allocation variant of moe_mi355x_block_fp8 for callers that cannot allocate (code under HIP
// graph capture, tight serving loops).  Its scratch is this file-scope device array: one copy per
// GPU the library runs on, held until the process ends.  Host code never passes the array's name
// to a kernel (on the host it is a stand-in, not a device address): the device address comes from
// hipGetSymbolAddress, once per device on that device's first call, and is kept per device.
// Every call on a GPU shares that GPU's array, so calls that overlap on one GPU (two streams, two
// threads) race; nothing in it has to start at zero (every kernel writes what it later reads, and
// the router clears the sort's histogram slots itself).
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's scratch array (looked up on the device's first call).
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return MOE_ERR_INVALID_ARG;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr) return MOE_ERR_INVALID_ARG;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOE_OK;
}
}  // namespace

extern "C" size_t moe_mi355x_block_fp8_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int moe_mi355x_block_fp8_noalloc(const void* x, const void* w_router, int T, int H, int I, int E, int k,
                                            int renorm, const void* w13, const float* s13, const void* w2,
                                            const float* s2, void* out, void* logits, void* ids, int id_bytes,
                                            void* weights, void* stream) {
  MOE_RETURN_IF(!experts_args_ok(T, H, I, E, k, id_bytes), MOE_ERR_INVALID_ARG);
  if (T == 0) return MOE_OK;
  MOE_RETURN_IF(!x || !w_router || !w13 || !s13 || !w2 || !s2 || !out, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!experts_aligned(x, w13, w2, out) || !moe_aligned16(w_router), MOE_ERR_ALIGNMENT);
  const size_t need = carve_block(nullptr, T, H, I, E, k).total;
  MOE_RETURN_IF(need > kNoAllocScratchBytes, MOE_ERR_SCRATCH);
  void* base = nullptr;
  const int rc = scratch_for_current_device(&base);
  if (rc) return rc;
  const BlockWs b = carve_block(base, T, H, I, E, k);
  return block_impl(x, w_router, T, H, I, E, k, renorm, w13, s13, w2, s2, out, logits, ids, id_bytes, weights, b,
                    (hipStream_t)stream, nullptr);
}
