// Entry points of the bf16-expert path: the reference's default checkpoint dtype (its backend
// loads every model with dtype=torch.bfloat16, src/inference_server/backends/torch_backend.py:
// 38-40) run without FP8 requantisation.  align -> gate_up (bf16 MFMA, fused SiLU*up, bf16 h)
// -> down (bf16 MFMA, routing-weight product, inverse permutation) -> slot-order combine.
//
// Reference: grouped_mm_experts_forward, TF/integrations/moe.py:377-478 (with the gate of
// :509-520), and Qwen3MoeSparseMoeBlock.forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:276-281.
#include "common.h"

int moe_bf16_block_m(int S, int E, int H, int I);
int moe_launch_grouped_gemms_bf16(const uint16_t* x, const uint16_t* w13, const uint16_t* w2, const int32_t* perm,
                                  const int32_t* tiles, const int32_t* n_tiles, int max_tiles, const uint16_t* topk_w,
                                  uint16_t* h, uint16_t* pairs, int S, int H, int I, int k, int block_m,
                                  hipStream_t s, int32_t* tok_cnt, uint16_t* comb, const int32_t* bucket);
int moe_launch_route_buckets(const void* x, const void* w_router, int T, int H, int E, int k, int renorm,
                             void* logits, void* ids, int id_bytes, void* weights, void* workspace,
                             size_t workspace_bytes, hipStream_t s, uint8_t* xq, float* sx, int32_t* zero, int nzero,
                             int32_t* ecnt, int32_t* bucket, int32_t* tiles, int32_t* n_tiles);
int moe_launch_combine(const uint16_t* pairs, const void* ids, int id_bytes, const uint16_t* wts, int T, int k, int H,
                       int E, const uint16_t* residual, uint16_t* out, hipStream_t s);
int moe_launch_route(const void* x, const void* w_router, int T, int H, int E, int k, int renorm, void* logits,
                     void* ids, int id_bytes, void* weights, void* workspace, size_t workspace_bytes, hipStream_t s,
                     uint8_t* xq, float* sx, int block_m, int32_t* perm, int32_t* counts, int32_t* offsets,
                     int32_t* tiles, int32_t* n_tiles, int32_t* chunk_counts, int32_t* gemm_cnt, int n_gemm_cnt);
int moe_launch_align_counted(const void* ids, int id_bytes, int S, int E, int block_m, const int32_t* bc,
                             int32_t* perm, int32_t* counts, int32_t* offsets, int32_t* tiles, int32_t* n_tiles,
                             hipStream_t s, int32_t* zero, int nzero);
bool moe_route_can_fuse_align(int T, int E, int k);
extern "C" size_t moe_mi355x_route_workspace_bytes(int T, int H, int E);
extern "C" int moe_mi355x_align_max_tiles(int S, int E, int block_m);
extern "C" size_t moe_mi355x_align_workspace_bytes(int S, int E);

namespace {

struct Bf16Ws {
  int32_t* perm;
  int32_t* counts;
  int32_t* offsets;
  int32_t* tiles;
  int32_t* n_tiles;
  void* align_ws;
  size_t align_ws_bytes;
  uint16_t* h;
  uint16_t* pairs;
  int32_t* cnt;  // 16-row tiles: the down GEMM's per-token hand-off counters [T, H / 64]
  int n_cnt;     // 0 on the other tiles
  int32_t* ecnt;    // 16-row tiles: expert bucket counts [E] and a workgroup count, after cnt
  int32_t* bucket;  // 16-row tiles: expert buckets [E, T] of pair indices
  size_t total;
  int block_m;
  int max_tiles;
};

Bf16Ws carve_bf16(void* base, int T, int H, int I, int E, int k) {
  Bf16Ws w{};
  const int S = T * k;
  w.block_m = moe_bf16_block_m(S, E, H, I);
  w.max_tiles = moe_mi355x_align_max_tiles(S, E, w.block_m);
  WsCarver c(base);
  w.perm = c.take<int32_t>(S);
  w.counts = c.take<int32_t>(E);
  w.offsets = c.take<int32_t>(E + 1);
  w.tiles = c.take<int32_t>((size_t)4 * (w.max_tiles > 0 ? w.max_tiles : 1));
  w.n_tiles = c.take<int32_t>(4);
  w.align_ws_bytes = moe_mi355x_align_workspace_bytes(S, E);
  w.align_ws = c.take<char>(w.align_ws_bytes);
  w.h = c.take<uint16_t>((size_t)S * I);
  w.pairs = c.take<uint16_t>((size_t)S * H);
  w.n_cnt = w.block_m == 16 ? T * (H / 64) : 0;
  w.cnt = c.take<int32_t>(w.block_m == 16 ? w.n_cnt + E + 1 : 0);  // one range, cleared by the router
  w.ecnt = w.cnt ? w.cnt + w.n_cnt : nullptr;
  w.bucket = c.take<int32_t>(w.block_m == 16 ? (size_t)E * T : 0);
  w.total = moe_align_up(c.off, 256);
  return w;
}

bool bf16_args_ok(int T, int H, int I, int E, int k, int id_bytes) {
  return T >= 0 && H > 0 && I > 0 && H % MOE_GROUP == 0 && I % MOE_GROUP == 0 && H <= 8192 && I <= 8192 &&
         E >= 1 && E <= 256 && k >= 1 && k <= 32 && k <= E && (id_bytes == 4 || id_bytes == 8) &&
         (long)T * k < (1L << 28);
}

// GEMMs and combine once the align outputs are in w.  `ids_valid`: every id is in [0, E) (the
// block path's own routing), so on 16-row tiles the down GEMM combines each token itself (its
// counters cleared by the align of the same call); caller ids may hold expert-parallel sentinels
// and go through the combine kernel.  At one token the separate combine is cheaper (measured
// layer time 36.0 us with it against 37.6 us fused; from 2 tokens on the fused form wins, e.g.
// 8 tokens 116.7 -> 114.3 us, 64 tokens 239.0 -> 235.8 us, Qwen3-30B-A3B shape).
int bf16_experts_after_align(const void* x, const void* ids, int id_bytes, const void* weights, int T, int H, int I,
                             int E, int k, const void* w13, const void* w2, void* out, const Bf16Ws& w, hipStream_t s,
                             bool ids_valid = false, const int32_t* bucket = nullptr) {
  const bool fused_combine = ids_valid && w.n_cnt > 0 && T > 1;
  int rc = moe_launch_grouped_gemms_bf16((const uint16_t*)x, (const uint16_t*)w13, (const uint16_t*)w2, w.perm,
                                         w.tiles, w.n_tiles, w.max_tiles, (const uint16_t*)weights, w.h, w.pairs,
                                         T * k, H, I, k, w.block_m, s, fused_combine ? w.cnt : nullptr,
                                         (uint16_t*)out, bucket);
  if (rc) return rc;
  if (fused_combine) return MOE_OK;
  // the 128-row tiles leave the routing-weight product to the combine
  return moe_launch_combine(w.pairs, ids, id_bytes, w.block_m == 128 ? (const uint16_t*)weights : nullptr, T, k,
                            H, E, nullptr, (uint16_t*)out, s);
}

struct Bf16BlockWs {
  void* route_ws;
  size_t route_bytes;
  uint16_t* logits;
  int32_t* ids;
  uint16_t* weights;
  void* experts_ws;
  size_t total;
};

Bf16BlockWs carve_bf16_block(void* base, int T, int H, int I, int E, int k) {
  Bf16BlockWs b{};
  WsCarver c(base);
  b.route_bytes = moe_mi355x_route_workspace_bytes(T, H, E);
  b.route_ws = c.take<char>(b.route_bytes);
  b.logits = c.take<uint16_t>((size_t)T * E);
  b.ids = c.take<int32_t>((size_t)T * k);
  b.weights = c.take<uint16_t>((size_t)T * k);
  b.experts_ws = c.take<char>(carve_bf16(nullptr, T, H, I, E, k).total);
  b.total = moe_align_up(c.off, 256);
  return b;
}

}  // namespace

extern "C" size_t moe_mi355x_experts_bf16_workspace_bytes(int T, int H, int I, int E, int k) {
  if (!bf16_args_ok(T, H, I, E, k, 4)) return 0;
  return carve_bf16(nullptr, T, H, I, E, k).total;
}

extern "C" int moe_mi355x_experts_bf16(const void* x, const void* ids, int id_bytes, const void* weights, int T,
                                       int H, int I, int E, int k, const void* w13, const void* w2, void* out,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  MOE_RETURN_IF(!bf16_args_ok(T, H, I, E, k, id_bytes), MOE_ERR_INVALID_ARG);
  if (T == 0) return MOE_OK;
  MOE_RETURN_IF(!x || !ids || !weights || !w13 || !w2 || !out, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!moe_aligned16(x) || !moe_aligned16(w13) || !moe_aligned16(w2) || !moe_aligned16(out),
                MOE_ERR_ALIGNMENT);
  const Bf16Ws w = carve_bf16(workspace, T, H, I, E, k);
  MOE_RETURN_IF(!workspace || workspace_bytes < w.total, MOE_ERR_WORKSPACE);
  hipStream_t s = (hipStream_t)stream;
  const int rc = moe_launch_align(ids, id_bytes, T * k, E, w.block_m, w.perm, w.counts, w.offsets, w.tiles,
                                  w.n_tiles, w.align_ws, w.align_ws_bytes, s);
  if (rc) return rc;
  return bf16_experts_after_align(x, ids, id_bytes, weights, T, H, I, E, k, w13, w2, out, w, s);
}

extern "C" size_t moe_mi355x_block_bf16_workspace_bytes(int T, int H, int I, int E, int k) {
  if (!bf16_args_ok(T, H, I, E, k, 4)) return 0;
  return carve_bf16_block(nullptr, T, H, I, E, k).total;
}

extern "C" int moe_mi355x_block_bf16(const void* x, const void* w_router, int T, int H, int I, int E, int k,
                                     int renorm, const void* w13, const void* w2, void* out, void* logits, void* ids,
                                     int id_bytes, void* weights, void* workspace, size_t workspace_bytes,
                                     void* stream) {
  MOE_RETURN_IF(!bf16_args_ok(T, H, I, E, k, id_bytes), MOE_ERR_INVALID_ARG);
  if (T == 0) return MOE_OK;
  MOE_RETURN_IF(!x || !w_router || !w13 || !w2 || !out, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!moe_aligned16(x) || !moe_aligned16(w_router) || !moe_aligned16(w13) || !moe_aligned16(w2) ||
                    !moe_aligned16(out),
                MOE_ERR_ALIGNMENT);
  const Bf16BlockWs b = carve_bf16_block(workspace, T, H, I, E, k);
  MOE_RETURN_IF(!workspace || workspace_bytes < b.total, MOE_ERR_WORKSPACE);
  hipStream_t s = (hipStream_t)stream;
  const Bf16Ws w = carve_bf16(b.experts_ws, T, H, I, E, k);
  void* lg = logits ? logits : (void*)b.logits;
  void* id_out = ids ? ids : (void*)b.ids;
  const int idb = ids ? id_bytes : 4;
  void* wt = weights ? weights : (void*)b.weights;
  if (w.block_m == 16) {
    // decode tiles: router GEMM (clearing the hand-off counters and the bucket counts), top-k into
    // expert buckets with the tile list, then the GEMMs on bucket tiles; no sort launch (the FP8
    // block's path; here, with GEMMs twice as long, level: 30B layer at 1 / 64 tokens 36.0 / 233.2 us
    // either way)
    int rc = moe_launch_route_buckets(x, w_router, T, H, E, k, renorm, lg, id_out, idb, wt, b.route_ws,
                                      b.route_bytes, s, nullptr, nullptr, w.cnt, w.n_cnt + E + 1, w.ecnt, w.bucket,
                                      w.tiles, w.n_tiles);
    if (rc) return rc;
    return bf16_experts_after_align(x, id_out, idb, wt, T, H, I, E, k, w13, w2, out, w, s, /*ids_valid=*/true,
                                    w.bucket);
  }
  // routing as the FP8 block, without the x quantisation; the sort rides in the top-k kernel
  // for decode batches, in its own launch(es) above
  const bool fused = moe_route_can_fuse_align(T, E, k);
  const bool counted = !fused && w.align_ws_bytes > 0;
  int rc = moe_launch_route(x, w_router, T, H, E, k, renorm, lg, id_out, idb, wt, b.route_ws, b.route_bytes, s,
                            nullptr, nullptr, w.block_m, fused ? w.perm : nullptr, w.counts, w.offsets, w.tiles,
                            w.n_tiles, counted ? (int32_t*)w.align_ws : nullptr, w.cnt, w.n_cnt);
  if (rc) return rc;
  if (counted) {
    rc = moe_launch_align_counted(id_out, idb, T * k, E, w.block_m, (const int32_t*)w.align_ws, w.perm, w.counts,
                                  w.offsets, w.tiles, w.n_tiles, s, w.cnt, w.n_cnt);
  } else if (!fused) {
    rc = moe_launch_align(id_out, idb, T * k, E, w.block_m, w.perm, w.counts, w.offsets, w.tiles, w.n_tiles,
                          w.align_ws, w.align_ws_bytes, s, w.cnt, w.n_cnt);
  }
  if (rc) return rc;
  return bf16_experts_after_align(x, id_out, idb, wt, T, H, I, E, k, w13, w2, out, w, s, /*ids_valid=*/true);
}
