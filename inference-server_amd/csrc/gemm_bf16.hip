// Grouped bf16 GEMMs for bf16 expert weights (the reference's default checkpoint dtype) on
// gfx950 MFMA (v_mfma_f32_16x16x32_bf16, fp32 accumulation in the MFMA).
//
//   MODE_GATE_UP: y = x[token(pair)] @ W13[e]^T, epilogue h = silu(gate) * up in the reference's
//                 bf16 rounding order, written per sorted row (bf16, no re-quantisation).
//                 (TF/integrations/moe.py:440-447 and :509-520)
//   MODE_DOWN:    z = h[row] @ W2[e]^T, epilogue bf16(bf16(z) * routing weight) written at the
//                 pair's original position t*k+j (moe.py:453-470); the combine kernel sums them.
//
// Operand layout of one MFMA (K = 32): lane l supplies row l % 16 of its operand and the eight
// bf16 at K offsets 8 (l / 16) .. +8 of the 32-deep chunk, for A and B alike; a 128-deep K
// block is four chunks, so a lane loads four 16-byte pieces per operand row and K block.  The
// 16x16 fp32 result holds D[4 (l / 16) + q][l % 16] in element q of lane l.
//
// Workgroup = 4 waves = (4 / KS) column groups x KS K-splits; a wave owns 16 output columns
// (gate_up: 16 gate rows + the matching 16 up rows of W13; down: DN adjacent 16-column slices)
// and WM 16-row fragments of one expert tile.  Weights stream from memory into VGPRs once per
// tile, one K block ahead of the MFMAs; K-split partials are summed through LDS in a fixed
// order (deterministic).  bf16 MFMAs accumulate exactly in fp32 (measured: unlike the FP8
// MFMA, whose 128 products are summed with truncation), so the GEMM outputs differ from an fp32
// dot product only by the order of fp32 additions.
#include "common.h"

namespace {

enum { MODE_GATE_UP = 0, MODE_DOWN = 1 };

struct Bf16GemmArgs {
  const uint16_t* a;       // gate_up: x [T, K] (token rows); down: h [S, K] (sorted rows)
  const uint16_t* w;       // [E, Nw, K]
  const int32_t* perm;     // [S] sorted row -> flat pair index
  const int32_t* tiles;    // [max_tiles, 4] {expert, first sorted row, rows, 0}
  const int32_t* n_tiles;  // [1]
  const uint16_t* topk_w;  // down: routing weights bf16 [S] by flat pair
  uint16_t* out;           // gate_up: h [S, N]; down: weighted pair outputs [S, N] by flat pair
  int K;                   // reduction length (multiple of 128)
  int N;                   // output columns (gate_up: I, down: H)
  int topk;
  // down, hand-off (null: off): the pair rows are stored device-scope and each token's k rows are
  // summed in slot order into comb by the workgroup that completes the token's column block
  // (tok_cnt [T, column blocks], zero on entry; every id must be valid)
  int32_t* tok_cnt;
  uint16_t* comb;
  // expert buckets (16-row tiles without a sort): the pairs of tile y's rows are
  // bucket[tiles[y].w ...] (moe_launch_route_buckets)
  const int32_t* bucket;
};

typedef uint4 Frag[4];  // the four 16-byte pieces of one lane for a 128-deep K block

template <int MODE, int WM, int KS, int DN>
__global__ __launch_bounds__(256) void grouped_gemm_bf16_kernel(Bf16GemmArgs p) {
  constexpr int CG = 4 / KS;
  constexpr int NOP = MODE == MODE_GATE_UP ? 2 : DN;
  constexpr int BM = 16 * WM;
  constexpr int WCOLS = MODE == MODE_GATE_UP ? 16 : 16 * DN;

  const int tile = blockIdx.y;
  if (tile >= p.n_tiles[0]) return;  // workgroup-uniform
  const int4 ti = *(const int4*)(p.tiles + 4 * tile);
  const int e = ti.x, row0 = ti.y, rows = ti.z;
  const int32_t* rowpair = p.bucket != nullptr ? p.bucket + ti.w : p.perm + row0;  // the tile rows' pairs

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cg = wave % CG, ks = wave / CG;
  const int lr = lane & 15, lg = lane >> 4;
  const int KB = p.K / MOE_GROUP;
  const int n0 = (blockIdx.x * CG + cg) * WCOLS;
  const int Nw = MODE == MODE_GATE_UP ? 2 * p.N : p.N;

  __shared__ int s_arow[BM];
  __shared__ float s_red[KS > 1 ? (KS - 1) * CG * WM * NOP * 4 * 64 : 1];
  __shared__ int s_done;     // down hand-off: result waves past their stores
  __shared__ int s_tok[BM];  // down hand-off: tokens this workgroup combines
  if (threadIdx.x == 0) s_done = 0;  // visible after the row-setup barrier

  // weight rows of this lane (gate_up: the up rows follow the I gate rows)
  const uint16_t* bptr[NOP];
#pragma unroll
  for (int o = 0; o < NOP; ++o) {
    const int wrow = MODE == MODE_GATE_UP ? n0 + o * p.N : n0 + 16 * o;
    bptr[o] = p.w + ((long)e * Nw + wrow + lr) * p.K + 8 * lg;
  }
  auto load_frag = [&](const uint16_t* base, int kb, Frag& f) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 4; ++u) f[u] = *(const uint4*)(base + (long)kb * MOE_GROUP + 32 * u);
  };

  // the first weight K block goes out before the activation-row setup
  Frag bc[NOP];
  if (ks < KB) {
#pragma unroll
    for (int o = 0; o < NOP; ++o) load_frag(bptr[o], ks, bc[o]);
  }
  for (int r = threadIdx.x; r < BM; r += blockDim.x) {
    const int rr = row0 + min(r, rows - 1);  // rows past the tile end repeat the last row
    s_arow[r] = MODE == MODE_GATE_UP ? rowpair[min(r, rows - 1)] / p.topk : rr;
  }
  __syncthreads();
  const uint16_t* aptr[WM];
#pragma unroll
  for (int mi = 0; mi < WM; ++mi) aptr[mi] = p.a + (long)s_arow[mi * 16 + lr] * p.K + 8 * lg;

  v4f acc[WM][NOP];
#pragma unroll
  for (int mi = 0; mi < WM; ++mi)
#pragma unroll
    for (int o = 0; o < NOP; ++o) acc[mi][o] = (v4f){0.f, 0.f, 0.f, 0.f};

  Frag ac[WM];
  int kb = ks;
  if (kb < KB) {
#pragma unroll
    for (int mi = 0; mi < WM; ++mi) load_frag(aptr[mi], kb, ac[mi]);
  }
  for (; kb < KB; kb += KS) {
    Frag bn[NOP], an[WM];
    const int kn = kb + KS;
    if (kn < KB) {
#pragma unroll
      for (int o = 0; o < NOP; ++o) load_frag(bptr[o], kn, bn[o]);
#pragma unroll
      for (int mi = 0; mi < WM; ++mi) load_frag(aptr[mi], kn, an[mi]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int mi = 0; mi < WM; ++mi)
#pragma unroll
        for (int o = 0; o < NOP; ++o)
          acc[mi][o] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, ac[mi][u]),
                                                               __builtin_bit_cast(v8bf, bc[o][u]), acc[mi][o], 0, 0, 0);
    if (kn < KB) {
#pragma unroll
      for (int o = 0; o < NOP; ++o)
#pragma unroll
        for (int u = 0; u < 4; ++u) bc[o][u] = bn[o][u];
#pragma unroll
      for (int mi = 0; mi < WM; ++mi)
#pragma unroll
        for (int u = 0; u < 4; ++u) ac[mi][u] = an[mi][u];
    }
  }

  if constexpr (KS > 1) {
    constexpr int PER = WM * NOP * 4;
    if (ks > 0) {
      float* dst = s_red + (((ks - 1) * CG + cg) * PER) * 64;
#pragma unroll
      for (int mi = 0; mi < WM; ++mi)
#pragma unroll
        for (int o = 0; o < NOP; ++o)
#pragma unroll
          for (int q = 0; q < 4; ++q) dst[((mi * NOP + o) * 4 + q) * 64 + lane] = acc[mi][o][q];
    }
    __syncthreads();
    if (ks > 0) return;
#pragma unroll
    for (int s = 1; s < KS; ++s) {
      const float* src = s_red + (((s - 1) * CG + cg) * PER) * 64;
#pragma unroll
      for (int mi = 0; mi < WM; ++mi)
#pragma unroll
        for (int o = 0; o < NOP; ++o)
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[mi][o][q] += src[((mi * NOP + o) * 4 + q) * 64 + lane];
    }
  }

  const int col = n0 + lr;
  if constexpr (MODE == MODE_DOWN) {
    if (p.tok_cnt != nullptr) {  // workgroup-uniform
      static_assert(BM <= MOE_WAVE, "one tile row per lane");
      // device-coherent stores: lanes lr and lr ^ 1 hold adjacent columns of the same rows, so the
      // even lane stores rows q = 0, 1 and the odd lane rows 2, 3 as 32-bit stores of both columns
      const bool odd = lr & 1;
#pragma unroll
      for (int mi = 0; mi < WM; ++mi) {
        uint32_t v[NOP][4];
        int dst[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int pair = rowpair[min(mi * 16 + 4 * lg + q, rows - 1)];
          const float wt = bf16_to_f32(p.topk_w[pair]);
#pragma unroll
          for (int o = 0; o < NOP; ++o) v[o][q] = f32_to_bf16(round_bf16(acc[mi][o][q]) * wt);
          dst[q] = pair;
        }
#pragma unroll
        for (int o = 0; o < NOP; ++o) {
          uint32_t pv[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) pv[q] = (uint32_t)__shfl_xor((int)v[o][q], 1);
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            const int q = odd ? 2 + h2 : h2;
            if (mi * 16 + 4 * lg + q >= rows) continue;
            const uint32_t both = odd ? (pv[q] | (v[o][q] << 16)) : (v[o][q] | (pv[q] << 16));
            xwg_store32(p.out + (long)dst[q] * p.N + (col & ~1) + 16 * o, both);
          }
        }
      }
      // each result wave waits for its stores; the last of the CG to get there combines
      xwg_wait_stores();
      int order = 0;
      if (lane == 0) order = atomicAdd(&s_done, 1);
      order = __builtin_amdgcn_readfirstlane(order);
      if (order != CG - 1) return;
      handoff_combine<CG * WCOLS>(rowpair, p.topk, rows, p.tok_cnt, gridDim.x, blockIdx.x, p.out, p.N,
                                  nullptr, p.comb, s_tok);
      return;
    }
  }
#pragma unroll
  for (int mi = 0; mi < WM; ++mi) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = mi * 16 + 4 * lg + q;
      if (r >= rows) continue;
      const int srow = row0 + r;
      if constexpr (MODE == MODE_GATE_UP) {
        p.out[(long)srow * p.N + col] = f32_to_bf16(silu_mul_bf16(acc[mi][0][q], acc[mi][1][q]));
      } else {
        const int pair = rowpair[r];
        const float wt = bf16_to_f32(p.topk_w[pair]);
#pragma unroll
        for (int o = 0; o < NOP; ++o)
          p.out[(long)pair * p.N + col + 16 * o] = f32_to_bf16(round_bf16(acc[mi][o][q]) * wt);
      }
    }
  }
}

template <int MODE, int WM, int KS, int DN = 1>
int launch_bf16_gemm(const Bf16GemmArgs& a, int max_tiles, hipStream_t s) {
  constexpr int CG = 4 / KS;
  constexpr int WCOLS = MODE == MODE_GATE_UP ? 16 : 16 * DN;
  dim3 grid(a.N / (WCOLS * CG), max_tiles);
  MOE_LAUNCH(MODE == MODE_GATE_UP ? MOE_PROF_GATE_UP : MOE_PROF_DOWN, s, (grouped_gemm_bf16_kernel<MODE, WM, KS, DN>),
             grid, dim3(256), 0, s, a);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}

}  // namespace

bool moe_prefill_bf16_ok(int H, int I, long max_rows);
int moe_launch_grouped_gemms_prefill_bf16(const uint16_t* x, const uint16_t* w13, const uint16_t* w2,
                                          const int32_t* perm, const int32_t* tiles, const int32_t* n_tiles,
                                          int max_tiles, uint16_t* h, uint16_t* pairs, int H, int I, int k,
                                          hipStream_t s);
extern "C" int moe_mi355x_align_max_tiles(int S, int E, int block_m);

// Tile height for the bf16 path: 16-row streaming tiles up to 8 pairs per expert; above, the
// 128-row LDS-tiled prefill kernel where the shape allows it (30B layer, 256 tokens: 304 -> 283 us
// against 32-row tiles, level at 129), else 32-row tiles up to 16 pairs per expert and 64 beyond.
int moe_bf16_block_m(int S, int E, int H, int I) {
  if (S <= 8 * E) return 16;
  if (moe_prefill_bf16_ok(H, I, 128L * moe_mi355x_align_max_tiles(S, E, 128))) return 128;
  return S <= 16 * E ? 32 : 64;
}

// gate_up (fused SiLU*up, bf16 h) then down (weighted pair rows; on 128-row tiles bf16(z) rows
// that the combine weights), bf16 weights.  With `bucket` (16-row tiles) the tile rows' pairs come
// from the expert buckets instead of the sort's permutation.
int moe_launch_grouped_gemms_bf16(const uint16_t* x, const uint16_t* w13, const uint16_t* w2, const int32_t* perm,
                                  const int32_t* tiles, const int32_t* n_tiles, int max_tiles, const uint16_t* topk_w,
                                  uint16_t* h, uint16_t* pairs, int S, int H, int I, int k, int block_m,
                                  hipStream_t s, int32_t* tok_cnt, uint16_t* comb, const int32_t* bucket) {
  if (block_m == 128)
    return moe_launch_grouped_gemms_prefill_bf16(x, w13, w2, perm, tiles, n_tiles, max_tiles, h, pairs, H, I, k, s);
  Bf16GemmArgs g1{x, w13, perm, tiles, n_tiles, nullptr, h, H, I, k, nullptr, nullptr, bucket};
  int rc;
  if (block_m == 16)
    rc = launch_bf16_gemm<MODE_GATE_UP, 1, 4>(g1, max_tiles, s);
  else if (block_m == 32)
    rc = launch_bf16_gemm<MODE_GATE_UP, 2, 2>(g1, max_tiles, s);
  else
    rc = launch_bf16_gemm<MODE_GATE_UP, 4, 1>(g1, max_tiles, s);
  if (rc) return rc;
  // the token-combine hand-off on 16-row tiles (tok_cnt [T, H / 64]: CG 2 x 32 columns)
  Bf16GemmArgs g2{h, w2, perm, tiles, n_tiles, topk_w, pairs, I, H, k, block_m == 16 ? tok_cnt : nullptr, comb,
                  bucket};
  if (block_m == 16)
    rc = launch_bf16_gemm<MODE_DOWN, 1, 2, 2>(g2, max_tiles, s);
  else if (block_m == 32)
    rc = launch_bf16_gemm<MODE_DOWN, 2, 2, 1>(g2, max_tiles, s);
  else
    rc = launch_bf16_gemm<MODE_DOWN, 4, 1, 1>(g2, max_tiles, s);
  return rc;
}
