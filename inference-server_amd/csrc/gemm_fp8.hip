// Grouped FP8 (e4m3) GEMMs with 128x128 block scales on gfx950 MFMA.
//
//   MODE_GATE_UP: y = xq[token(pair)] @ W13[e]^T, epilogue h = silu(gate) * up in
//                 the reference's bf16 rounding order, written per sorted row.
//                 (TF/integrations/finegrained_fp8.py:547-563 + moe.py:509-520)
//   MODE_DOWN:    z = hq[row] @ W2[e]^T, epilogue bf16(z) * routing weight (bf16),
//                 written at the pair's original position t*k+j, which folds the
//                 reference's inverse permutation (finegrained_fp8.py:565-583).
//
// One v_mfma_f32_16x16x128_f8f6f4 consumes exactly one 128-deep K block, so the
// two fp32 block scales (activation row scale x weight tile scale) are applied
// once per MFMA result: acc += mfma(a, b, 0) * (sa[row, kb] * sw[nblk, kb]).
//
// Operand layout: lane l supplies row (l % 16) of its operand and bytes
// [32 * (l / 16), 32 * (l / 16) + 32) of the 128-byte K block, for A and for B
// alike, so every product pairs matching K indices.  The 16x16 fp32 result holds
// D[4 * (l / 16) + q][l % 16] in element q of lane l.
//
// Workgroup = 4 waves = (4 / KS) column groups x KS K-splits.  A wave owns 16
// output columns (for gate_up: 16 gate rows + the matching 16 up rows of W13)
// and WM 16-row M fragments of one expert tile.  K-split partials are summed
// through LDS in a fixed order (deterministic).  Each weight byte is read once
// per M tile, straight from HBM into VGPRs: the decode case is a weight stream.
#include "route_dev.h"

namespace {

enum { MODE_GATE_UP = 0, MODE_DOWN = 1 };

struct GemmArgs {
  const uint8_t* a;        // gate_up: xq [T, K] (rows are tokens); down: hq [S, K] (sorted rows)
  const float* sa;         // activation scales, [rows, K/128]
  const uint8_t* w;        // [E, Nw, K]
  const float* sw;         // [E, Nw/128, K/128]
  const int32_t* perm;     // [S] sorted row -> flat pair index
  const int32_t* tiles;    // [max_tiles, 4] {expert, first sorted row, rows, 0}
  const int32_t* n_tiles;  // [1]
  const uint16_t* topk_w;  // down: routing weights bf16 [S] by flat pair
  uint16_t* out;           // gate_up: h [S, N]; down: pair outputs [S, N]
  int K;                   // reduction length
  int N;                   // output columns (gate_up: I, down: H)
  int topk;                // k, for pair -> token
  // Hand-offs inside the launch (null: off).  gate_up: the last workgroup of a (tile, 128-column
  // group) to finish quantises that group of the tile's h rows into hq / sh (tile_cnt
  // [max_tiles, N / 128], zero on entry).  down: the
  // last of a token's k pair rows to finish a column block sums the token's k rows of that block
  // in slot order into comb (tok_cnt [T, column blocks], zero on entry; every id must be valid).
  int32_t* tile_cnt;
  uint8_t* hq;
  float* sh;
  int32_t* tok_cnt;
  uint16_t* comb;
  const uint16_t* residual;  // down: comb = bf16(residual + bf16(sum)) when non-null
  // ROUTED gate_up (single-token decode): tile y is routing slot y = t * topk + j, one row, and
  // the workgroup routes token t itself from the router GEMM's K-split partials; the workgroups
  // of column block 0 write the routing outputs and the one-row tile list the down GEMM reads.
  const float* part;  // [ksplit, T, E] fp32
  int ksplit, T, E, renorm;
  uint16_t* logits;   // bf16 [T, E] or null
  void* ids;          // [T, topk], int32 or int64 (id_bytes)
  int id_bytes;
  uint16_t* wts;      // bf16 [T, topk]
  int32_t* perm_out;  // [S]: identity (slot y holds pair y)
  int32_t* tiles_out; // [S, 4]: {expert, y, 1, 0}
  int32_t* n_tiles_out;
  // expert buckets (decode tiles without a sort, moe_launch_route_buckets): the pairs of tile y's
  // rows are bucket[tiles[y].w ...]
  const int32_t* bucket;
  // exact accumulation (moe_exact_accum): e4m3 operands widened to bf16, bf16 MFMAs
  int exact;
};

constexpr int kMaxKB = 32;  // K <= 4096

// DN: 16-column slices per wave in the down GEMM (adjacent), so that a wave streams as
// many weight bytes per setup as a gate_up wave (which pairs a gate and an up slice).
// SHA (32-row tiles, no K split): the tile's activation K block is staged once per workgroup in
// LDS and every column wave reads its fragments there, instead of each wave loading the same
// rows from memory (the four column waves would put 4x the activation bytes through L1).
// The 16-row down GEMM is held to 80 VGPRs (6 waves per SIMD instead of 5, no spills): more
// weight streams in flight (down at 8 / 32 / 64 tokens 25.7 / 42.4 / 47.2 -> 24.7 / 41.2 / 46.4
// us).  The same bound on gate_up spills and runs slower (64 tokens 70 -> 119 us); with its loads
// rewritten as a uniform base + 32-bit lane offsets it fits 80 VGPRs (2 spilled) but still runs
// slower at 6 waves (64 tokens 69.5 -> 86.3 us), and capped at 4 or 3 workgroups per CU (LDS
// padding) slower as well (72.7 / 80.1 us): 5 is gate_up's best occupancy.
// NKW > 0: every wave has exactly NKW K blocks (K = NKW * KS * 128), and the K loop is unrolled
// with each block's loads issued one block ahead of its MFMAs and the wave's weight scales loaded
// before the loop: in the rolled loop a scale load issued behind the next block's loads, and the
// copy of the next block's registers into the current ones, wait for those loads inside the same
// iteration, so a wave has only one block in flight.
// QH (16-row down GEMM): a holds bf16 h; the workgroup quantises its tile's rows into LDS (the
// h quantisation's arithmetic: same codes and scales) and reads the activation fragments there.
constexpr int kQhMaxK = 1024;  // 16 rows of LDS codes within the 6 workgroups per CU of the down GEMM
template <int MODE, int WM, int KS, int DN = 1, bool SHA = false, bool ROUTED = false, int NKW = 0, bool QH = false,
          bool EX = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MODE == MODE_DOWN && WM == 1 ? (EX ? 5 : 6) : 1)))
void grouped_gemm_fp8_kernel(GemmArgs p) {
  constexpr int CG = 4 / KS;                  // column groups per workgroup
  constexpr int NOP = MODE == MODE_GATE_UP ? 2 : DN;  // B operands per wave (gate, up | column slices)
  constexpr int BM = 16 * WM;

  static_assert(!ROUTED || (MODE == MODE_GATE_UP && WM == 1 && !SHA), "routed slots are one-row gate_up tiles");
  static_assert(!QH || (MODE == MODE_DOWN && WM == 1 && !SHA), "h quantised in the 16-row down GEMM");
  const int tile = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // ROUTED: the slot's token is known before its routing, and so are its activation scales and,
  // with NKW, the wave's activation fragments: they are loaded here, so that their round trip
  // overlaps the routing's (which reads what the router GEMM just wrote)
  constexpr int kPreSa = ROUTED ? (16 * kMaxKB + 255) / 256 : 1;
  float sa_pre[kPreSa];
  v8i av_pre[ROUTED && NKW > 0 ? NKW : 1];
  if constexpr (ROUTED) {
    const int t = tile / p.topk;
    const int KBr = p.K / MOE_GROUP;
#pragma unroll
    for (int u = 0; u < kPreSa; ++u) {
      const int i = threadIdx.x + 256 * u;
      sa_pre[u] = i < BM * KBr ? p.sa[(long)t * KBr + i % KBr] : 0.f;
    }
    if constexpr (NKW > 0) {
      const int ks_ = wave / (4 / KS);
#pragma unroll
      for (int i = 0; i < NKW; ++i)
        av_pre[i] = *(const v8i*)(p.a + (long)t * p.K + (lane >> 4) * 32 + (ks_ + i * KS) * MOE_GROUP);
    }
  }
  int e, row0, rows;
  const int32_t* rowpair;  // the pairs of the tile's rows (gate_up's token rows, down's output rows)
  if constexpr (ROUTED) {
    // wave 0 routes the slot's token and hands slot j's expert to the other waves (one routing
    // per workgroup instead of one per wave: 4 waves x 1.5 workgroups per CU routing at once made
    // the routing take ~4 us; single-token layer 27.2 -> 26.3 us with the unrolled K loop)
    const int t = tile / p.topk, j = tile - t * p.topk;
    __shared__ int s_route_e;
    const bool writer = blockIdx.x == 0 && j == 0 && wave == 0;  // one wave per token
    if (wave == 0) {
      int my_e;
      float my_w;
      route_token(p.part, p.ksplit, nullptr, p.T, p.E, p.topk, p.renorm, writer ? p.logits : nullptr, t, my_e,
                  my_w);
      if (lane == j) s_route_e = my_e;
      if (writer && lane < p.topk) store_route(p.ids, p.id_bytes, p.wts, (long)t * p.topk + lane, my_e, my_w);
    }
    __syncthreads();
    e = s_route_e;
    row0 = tile;
    rows = 1;
    rowpair = p.perm_out + tile;
    if (blockIdx.x == 0 && wave == 0 && lane == 0) {
      *(int4*)(p.tiles_out + 4 * tile) = make_int4(e, tile, 1, 0);
      p.perm_out[tile] = tile;
      if (tile == 0) p.n_tiles_out[0] = gridDim.y;
    }
  } else {
    if (tile >= p.n_tiles[0]) return;  // workgroup-uniform
    const int4 ti = *(const int4*)(p.tiles + 4 * tile);
    e = ti.x;
    row0 = ti.y;
    rows = ti.z;
    // Invariant: the tile list and the expert buckets come from an earlier launch (the top-k
    // kernel's last workgroup writes them with plain stores and no release); only stream order
    // makes them visible here, so they must never be read inside the launch that writes them.
    rowpair = p.bucket != nullptr ? p.bucket + ti.w : p.perm + row0;
  }

  const int cg = wave % CG, ks = wave / CG;
  const int lr = lane & 15, lg = lane >> 4;
  const int KB = p.K / MOE_GROUP;
  constexpr int WCOLS = MODE == MODE_GATE_UP ? 16 : 16 * DN;  // output columns per wave
  const int n0 = (blockIdx.x * CG + cg) * WCOLS;
  const int Nw = MODE == MODE_GATE_UP ? 2 * p.N : p.N;

  __shared__ int s_arow[BM];                 // activation row of each tile row
  __shared__ float s_sa[BM][kMaxKB];         // activation scales of the tile
  __shared__ float s_red[KS > 1 ? (KS - 1) * CG * WM * NOP * 4 * 64 : 1];
  // SHA: two K blocks of the tile's activations, 8 16-byte chunks per row; chunk c of row r at
  // c ^ (r & 7), so that the 16-row fragment reads (one chunk column per 16 lanes) are
  // conflict-free
  __shared__ __attribute__((aligned(16))) uint4 s_at[SHA ? 2 : 1][SHA ? BM * 8 : 1];
  static_assert(!SHA || (KS == 1 && BM * 8 == 256), "SHA stages one 16-byte chunk per thread, no K split");
  // QH: the tile's e4m3 h rows; rows 16 B longer than K so that the 16 rows of a fragment read
  // fall in distinct banks
  __shared__ __attribute__((aligned(16))) uint8_t s_hq[QH ? BM : 1][QH ? kQhMaxK + 16 : 1];
  __shared__ int s_done;     // result waves past their hand-off stores
  __shared__ int s_tok[BM];  // down hand-off: tokens this workgroup combines
  if (threadIdx.x == 0) s_done = 0;  // visible after the barriers of the row setup below

  // The weight stream needs only the expert and the column block: its first loads go
  // out before the activation-row setup (perm -> rows -> scales), whose dependent round
  // trips then overlap the weight fetch.
  const uint8_t* bptr[NOP];
  const float* swp[NOP];
#pragma unroll
  for (int o = 0; o < NOP; ++o) {
    const int wrow = MODE == MODE_GATE_UP ? n0 + o * p.N : n0 + 16 * o;  // up rows follow the I gate rows
    bptr[o] = p.w + ((long)e * Nw + wrow + lr) * p.K + lg * 32;
    swp[o] = p.sw + ((long)e * (Nw / MOE_GROUP) + wrow / MOE_GROUP) * KB;
  }

  v8i bc[NOP];
  // with NKW every wave has K blocks (ks < KB): the loads are unconditional, since a branch
  // around them makes the compiler wait for the first one where the branch joins, exposing its
  // full memory latency before the row setup
  if (NKW > 0 || ks < KB) {
#pragma unroll
    for (int o = 0; o < NOP; ++o) bc[o] = *(const v8i*)(bptr[o] + ks * MOE_GROUP);
  }
  float swk[NKW > 0 ? NKW : 1][NOP];  // NKW: the wave's weight scales, loaded up front
  if constexpr (NKW > 0) {
#pragma unroll
    for (int i = 0; i < NKW; ++i)
#pragma unroll
      for (int o = 0; o < NOP; ++o) swk[i][o] = swp[o][ks + i * KS];
  }

  for (int r = threadIdx.x; r < BM; r += blockDim.x) {
    const int rr = row0 + min(r, rows - 1);  // rows past the tile end repeat the last row
    s_arow[r] = ROUTED ? tile / p.topk : MODE == MODE_GATE_UP ? rowpair[min(r, rows - 1)] / p.topk : rr;
  }
  __syncthreads();
  if constexpr (QH) {
    // 16 lanes per (row, 128-column group), 8 values each; rows past the tile's end are not
    // filled (their results are never stored)
    const uint16_t* h = (const uint16_t*)p.a;
    for (int i = threadIdx.x; i < rows * KB * 16; i += blockDim.x) {
      const int r = i / (KB * 16), g = (i >> 4) - r * KB, sub = i & 15;
      const uint4 raw = *(const uint4*)(h + (long)s_arow[r] * p.K + g * MOE_GROUP + sub * 8);
      quant_group16_raw(raw, &s_hq[r][g * MOE_GROUP + sub * 8], &s_sa[r][g], sub);
    }
  } else if constexpr (ROUTED) {
#pragma unroll
    for (int u = 0; u < kPreSa; ++u) {
      const int i = threadIdx.x + 256 * u;
      if (i < BM * KB) s_sa[i / KB][i % KB] = sa_pre[u];
    }
  } else {
    for (int i = threadIdx.x; i < BM * KB; i += blockDim.x) {
      const int r = i / KB, kb = i % KB;
      s_sa[r][kb] = p.sa[(long)s_arow[r] * KB + kb];
    }
  }
  __syncthreads();
  // the activation fragment of row lr (lane (lr, lg): bytes [32 lg, 32 lg + 32) of K block kb)
  auto afrag = [&](const uint8_t* ptr, int kb) __attribute__((always_inline)) -> v8i {
    if constexpr (QH)
      return *(const v8i*)&s_hq[lr][kb * MOE_GROUP + lg * 32];
    else
      return *(const v8i*)(ptr + kb * MOE_GROUP);
  };

  v4f acc[WM][NOP];
#pragma unroll
  for (int mi = 0; mi < WM; ++mi)
#pragma unroll
    for (int o = 0; o < NOP; ++o) acc[mi][o] = (v4f){0.f, 0.f, 0.f, 0.f};

  // the MFMAs of K block kb on activation fragments a and weight fragments b with weight scales swv
  auto mfma_core = [&](const v8i (&a)[WM], const v8i (&b)[NOP], int kb, const float (&swv)[NOP])
      __attribute__((always_inline)) {
#pragma unroll
    for (int mi = 0; mi < WM; ++mi) {
      float sav[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) sav[q] = s_sa[mi * 16 + 4 * lg + q][kb];
#pragma unroll
      for (int o = 0; o < NOP; ++o) {
        const v4f zero = {0.f, 0.f, 0.f, 0.f};
        v4f t;
        if constexpr (EX)
          t = mfma_e4m3_exact(a[mi], b[o]);
        else
          t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[mi], b[o], zero, 0, 0, 0, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[mi][o][q] = fmaf(t[q], sav[q] * swv[o], acc[mi][o][q]);
      }
    }
  };
  // the same on bc, with the weight scales loaded here
  auto mfma_block = [&](const v8i (&a)[WM], int kb) __attribute__((always_inline)) {
    float swv[NOP];
#pragma unroll
    for (int o = 0; o < NOP; ++o) swv[o] = swp[o][kb];
    mfma_core(a, bc, kb, swv);
  };

  if constexpr (SHA) {
    // thread t stages chunk t & 7 of tile row t >> 3: K block kb + 1 is loaded into a register
    // while kb is computed and stored to the other LDS buffer after the MFMAs; one barrier per
    // K block
    const int sr = threadIdx.x >> 3, sc = threadIdx.x & 7;
    const uint8_t* sptr = p.a + (long)s_arow[sr] * p.K + sc * 16;
    const int sidx = sr * 8 + (sc ^ (sr & 7));
    s_at[0][sidx] = *(const uint4*)sptr;
    uint4 ra = *(const uint4*)(sptr + (long)min(1, KB - 1) * MOE_GROUP);
    __syncthreads();
    for (int kb = 0; kb < KB; ++kb) {
      v8i bn[NOP];
      const int kn = kb + 1;
      if (kn < KB) {
#pragma unroll
        for (int o = 0; o < NOP; ++o) bn[o] = *(const v8i*)(bptr[o] + kn * MOE_GROUP);
      }
      // fragment of row mi * 16 + lr: its chunks 2 lg and 2 lg + 1
      v8i af[WM];
#pragma unroll
      for (int mi = 0; mi < WM; ++mi) {
        const int r = mi * 16 + lr;
        const uint4 lo = s_at[kb & 1][r * 8 + ((2 * lg) ^ (r & 7))];
        const uint4 hi = s_at[kb & 1][r * 8 + ((2 * lg + 1) ^ (r & 7))];
        af[mi] = (v8i){(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
      }
      mfma_block(af, kb);
      if (kn < KB) {
        s_at[kn & 1][sidx] = ra;
        ra = *(const uint4*)(sptr + (long)min(kn + 1, KB - 1) * MOE_GROUP);
#pragma unroll
        for (int o = 0; o < NOP; ++o) bc[o] = bn[o];
      }
      __syncthreads();  // block kn visible, and every wave done with buffer kb & 1
    }
  } else if constexpr (NKW > 0) {
    const uint8_t* aptr[WM];
#pragma unroll
    for (int mi = 0; mi < WM; ++mi) aptr[mi] = p.a + (long)s_arow[mi * 16 + lr] * p.K + lg * 32;
    v8i av[NKW][WM], bv[NKW][NOP];
#pragma unroll
    for (int o = 0; o < NOP; ++o) bv[0][o] = bc[o];
    if constexpr (ROUTED) {
#pragma unroll
      for (int i = 0; i < NKW; ++i) av[i][0] = av_pre[i];
    } else {
#pragma unroll
      for (int mi = 0; mi < WM; ++mi) av[0][mi] = afrag(aptr[mi], ks);
    }
#pragma unroll
    for (int i = 0; i < NKW; ++i) {
      if (i + 1 < NKW) {
        const int kn = ks + (i + 1) * KS;
#pragma unroll
        for (int o = 0; o < NOP; ++o) bv[i + 1][o] = *(const v8i*)(bptr[o] + kn * MOE_GROUP);
        if constexpr (!ROUTED) {
#pragma unroll
          for (int mi = 0; mi < WM; ++mi) av[i + 1][mi] = afrag(aptr[mi], kn);
        }
      }
      mfma_core(av[i], bv[i], ks + i * KS, swk[i]);
    }
  } else {
    const uint8_t* aptr[WM];
#pragma unroll
    for (int mi = 0; mi < WM; ++mi) aptr[mi] = p.a + (long)s_arow[mi * 16 + lr] * p.K + lg * 32;
    v8i ac[WM];
    int kb = ks;
    if (kb < KB) {
#pragma unroll
      for (int mi = 0; mi < WM; ++mi) ac[mi] = afrag(aptr[mi], kb);
    }
    for (; kb < KB; kb += KS) {
      v8i bn[NOP], an[WM];
      const int kn = kb + KS;
      if (kn < KB) {
#pragma unroll
        for (int o = 0; o < NOP; ++o) bn[o] = *(const v8i*)(bptr[o] + kn * MOE_GROUP);
#pragma unroll
        for (int mi = 0; mi < WM; ++mi) an[mi] = afrag(aptr[mi], kn);
      }
      mfma_block(ac, kb);
      if (kn < KB) {
#pragma unroll
        for (int o = 0; o < NOP; ++o) bc[o] = bn[o];
#pragma unroll
        for (int mi = 0; mi < WM; ++mi) ac[mi] = an[mi];
      }
    }
  }

  // after the K-split reduction only the ks == 0 waves hold sums; the others leave, freeing their
  // slots for the next workgroups
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

  const bool handoff = MODE == MODE_GATE_UP ? p.tile_cnt != nullptr : p.tok_cnt != nullptr;  // uniform
  const int col = n0 + lr;
#pragma unroll
  for (int mi = 0; mi < WM; ++mi) {
    // one bf16 per (row 4 lg + q, column lr) and output slice o
    uint32_t v[NOP][4];
    int dst_row[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = mi * 16 + 4 * lg + q;
      const int srow = row0 + min(r, rows - 1);
      if constexpr (MODE == MODE_GATE_UP) {
        v[0][q] = f32_to_bf16(silu_mul_bf16(acc[mi][0][q], acc[mi][1][q]));
        dst_row[q] = srow;
      } else {
        const int pair = rowpair[min(r, rows - 1)];
        const float wt = bf16_to_f32(p.topk_w[pair]);
#pragma unroll
        for (int o = 0; o < NOP; ++o) v[o][q] = f32_to_bf16(round_bf16(acc[mi][o][q]) * wt);
        dst_row[q] = pair;
      }
    }
    constexpr int NV = MODE == MODE_GATE_UP ? 1 : NOP;
    if (!handoff) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (mi * 16 + 4 * lg + q >= rows) continue;
#pragma unroll
        for (int o = 0; o < NV; ++o) p.out[(long)dst_row[q] * p.N + col + 16 * o] = (uint16_t)v[o][q];
      }
    } else {
      // device-coherent stores for the wave that finishes the group / token: lanes lr and lr ^ 1
      // hold adjacent columns of the same rows, so the even lane stores rows q = 0, 1 and the odd
      // lane rows 2, 3, each as one 32-bit store of both columns
      const bool odd = lr & 1;
#pragma unroll
      for (int o = 0; o < NV; ++o) {
        uint32_t pv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) pv[q] = (uint32_t)__shfl_xor((int)v[o][q], 1);
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
          const int q = odd ? 2 + h2 : h2;
          if (mi * 16 + 4 * lg + q >= rows) continue;
          const uint32_t both = odd ? (pv[q] | (v[o][q] << 16)) : (v[o][q] | (pv[q] << 16));
          xwg_store32(p.out + (long)dst_row[q] * p.N + (col & ~1) + 16 * o, both);
        }
      }
    }
  }
  if (!handoff) return;
  // The CG result waves of the workgroup each wait for their stores; the last of them to get
  // there counts the workgroup in (an LDS counter elects it), the others leave.
  xwg_wait_stores();
  int order = 0;
  if (lane == 0) order = atomicAdd(&s_done, 1);
  order = __builtin_amdgcn_readfirstlane(order);
  if (order != CG - 1) return;

  if constexpr (MODE == MODE_GATE_UP) {
    // per (tile, 128-column group of h): the last of the group's 128 / (16 CG) workgroups to count
    // in quantises the group for the tile's rows (16 lanes per row, 8 rows in flight per batch)
    constexpr int WG_COLS = 16 * CG;
    const int G = p.N / MOE_GROUP;
    const int gi = blockIdx.x * WG_COLS / MOE_GROUP;
    int last = 0;
    if (lane == 0) last = xwg_count_in(p.tile_cnt + (long)tile * G + gi) == MOE_GROUP / WG_COLS - 1;
    if (!__builtin_amdgcn_readfirstlane(last)) return;
    const int sub = lane & 15, grp = lane >> 4;  // 4 rows at a time
    for (int r0 = grp; r0 < rows; r0 += 32) {
      uint4 hv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = min(r0 + 4 * i, rows - 1);
        hv[i] = xwg_load128(p.out + (long)(row0 + r) * p.N + gi * MOE_GROUP + sub * 8);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = r0 + 4 * i;
        if (r >= rows) break;  // uniform over the 16 lanes of a row
        const long e0 = (long)(row0 + r) * p.N + gi * MOE_GROUP + sub * 8;
        quant_group16_raw(hv[i], p.hq + e0, p.sh + (long)(row0 + r) * G + gi, sub);
      }
    }
  } else {
    static_assert(BM <= MOE_WAVE, "one tile row per lane");
    handoff_combine<CG * WCOLS>(rowpair, p.topk, rows, p.tok_cnt, gridDim.x, blockIdx.x, p.out, p.N, p.residual,
                                p.comb, s_tok);
  }
}

template <int MODE, int WM, int KS, int DN = 1, bool SHA = false, bool ROUTED = false, int NKW = 0, bool QH = false>
int launch_gemm_nkw(const GemmArgs& a, int max_tiles, hipStream_t s) {
  constexpr int CG = 4 / KS;
  constexpr int WCOLS = MODE == MODE_GATE_UP ? 16 : 16 * DN;
  // column blocks vary fastest: the workgroups past the live tiles (max_tiles is a bound)
  // come after every working one instead of between them, and consecutive workgroups stream
  // adjacent weight rows of one expert (gate_up at 64 tokens 75 -> 70 us)
  dim3 grid(a.N / (WCOLS * CG), max_tiles);
  if (a.exact)
    MOE_LAUNCH(MODE == MODE_GATE_UP ? MOE_PROF_GATE_UP : MOE_PROF_DOWN, s,
               (grouped_gemm_fp8_kernel<MODE, WM, KS, DN, SHA, ROUTED, NKW, QH, true>), grid, dim3(256), 0, s, a);
  else
    MOE_LAUNCH(MODE == MODE_GATE_UP ? MOE_PROF_GATE_UP : MOE_PROF_DOWN, s,
               (grouped_gemm_fp8_kernel<MODE, WM, KS, DN, SHA, ROUTED, NKW, QH, false>), grid, dim3(256), 0, s, a);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}

// The unrolled K loop where it pays: the 16-row down GEMM with 3 or 4 K blocks per wave (the
// Qwen3-30B-A3B shape: 30B layer, down at 8 / 32 / 64 / 128 tokens 24.3 / 40.7 / 46.0 / 50.5 ->
// 23.3 / 39.7 / 45.1 / 48.9 us).  Not for gate_up: its 4 blocks per wave took 94 VGPRs and one
// wave per SIMD fewer (1-2 us slower from 32 tokens), and held to 5 waves per SIMD (90 VGPRs) it
// was slower still (64 tokens 69 -> 79 us); nor for 6 or 8 blocks (spills at the down GEMM's
// 80-VGPR bound: Qwen3-235B-A22B down at 64 tokens 149 -> 169 us).
template <int MODE, int WM, int KS, int DN = 1, bool SHA = false, bool ROUTED = false, bool QH = false>
int launch_gemm(const GemmArgs& a, int max_tiles, hipStream_t s) {
  const int KB = a.K / MOE_GROUP;
  if constexpr (MODE == MODE_DOWN && WM == 1 && !SHA) {
    if (KB == 3 * KS) return launch_gemm_nkw<MODE, WM, KS, DN, SHA, ROUTED, 3, QH>(a, max_tiles, s);
    if (KB == 4 * KS) return launch_gemm_nkw<MODE, WM, KS, DN, SHA, ROUTED, 4, QH>(a, max_tiles, s);
    if constexpr (KS == 1)
      if (KB == 6) return launch_gemm_nkw<MODE, WM, KS, DN, SHA, ROUTED, 6, QH>(a, max_tiles, s);
  }
  return launch_gemm_nkw<MODE, WM, KS, DN, SHA, ROUTED, 0, QH>(a, max_tiles, s);
}

// The 16-row down GEMM quantises h itself (QH) where its tile's codes fit the LDS rows and the
// unrolled loop stays within the 80-VGPR bound (4 K blocks per wave with two column slices
// spills): no quant_h launch and no hand-off quantisation in gate_up, whose tail it lengthened.
// Qwen3-30B-A3B layer at 8 / 16 / 32 / 64 tokens: 65.1 / 88.2 / 112.9 / 124.7 ->
// 62.5 / 85.3 / 109.0 / 123.2 us (gate_up 36.1 / 50.8 / 66.0 -> 33.6 / 47.5 / 61.4 us; down level).
bool down_quantises_h(int S, int I) { return I <= kQhMaxK && !(I / MOE_GROUP == 8 && S > 16); }

// 16-row down GEMM; g2.a / g2.sa are bf16 h / null with qh, else hq / its scales.  Quantising h
// with 3, 4 or 6 K blocks in all: four 16-column waves per workgroup, each over the whole K (no
// K split, so no LDS reduction or its barrier; the same 12 KB per wave at the 30B shape): 30B
// down at 1 / 8 / 64 / 128 tokens 11.3 / 23.2 / 46.5 / 54.4 -> 10.9 / 23.0 / 45.8 / 53.8 us.
// Otherwise a two-way K split, and two column slices per wave beyond 2 tokens' pairs (T=8: down
// 25.7 -> 24.9 us; level at 1, 32 and 64 tokens).
// few_pairs (h quantised in gate_up's hand-off, up to 2 pairs per expert) with 12 K blocks: a
// four-way K split of 3 blocks per wave, two column slices (Qwen3-235B-A22B down at 8 / 32
// tokens 68.0 / 129.7 -> 65.3 / 126.5 us; at 64 tokens it was 2.7 us slower, so not there).
int launch_down16(const GemmArgs& g2, int S, int max_tiles, bool qh, hipStream_t s, bool few_pairs = false) {
  const int KB = g2.K / MOE_GROUP;
  if (qh && (KB == 3 || KB == 4 || KB == 6)) return launch_gemm<MODE_DOWN, 1, 1, 1, false, false, true>(g2, max_tiles, s);
  if (qh)
    return S > 16 ? launch_gemm<MODE_DOWN, 1, 2, 2, false, false, true>(g2, max_tiles, s)
                  : launch_gemm<MODE_DOWN, 1, 2, 1, false, false, true>(g2, max_tiles, s);
  if (few_pairs && KB == 12) return launch_gemm_nkw<MODE_DOWN, 1, 4, 2, false, false, 3>(g2, max_tiles, s);
  return S > 16 ? launch_gemm<MODE_DOWN, 1, 2, 2>(g2, max_tiles, s) : launch_gemm<MODE_DOWN, 1, 2>(g2, max_tiles, s);
}

}  // namespace

int moe_launch_grouped_gemms_prefill(const uint8_t* xq, const float* sx, const uint8_t* w13, const float* s13,
                                     const uint8_t* w2, const float* s2, const int32_t* perm, const int32_t* tiles,
                                     const int32_t* n_tiles, int max_tiles, const uint16_t* topk_w, uint8_t* hq,
                                     float* sh, uint16_t* pairs, int H, int I, int k, hipStream_t s);

// Tile height (rows per M tile) for S pairs over E experts: 16-row tiles stream weights
// (decode); beyond 8 pairs per expert 128-row tiles go to the LDS-tiled MFMA kernel (needs
// 256-column tiles of H and at least 4 K blocks in each GEMM for its cross-item DMA pipeline):
// from 9 to 16 pairs per expert it also beats 32-row streaming tiles (30B layer: 192 tokens
// 158 -> 150 us, 256 tokens 161 -> 151 us, level at 129).  Shapes it cannot take stream 32-row
// tiles up to 16 pairs per expert (one tile per expert for the usual loads instead of two 16-row
// ones) and 64-row tiles above.
int moe_gemm_block_m(int S, int E, int H, int I) {
  if (S <= 8 * E) return 16;
  if (H % 256 == 0 && H >= 512 && I >= 512) return 128;
  return S <= 16 * E ? 32 : 64;
}

// Column blocks of the decode down GEMM for S pairs at tile height block_m: the width of the
// per-token hand-off counters (tok_cnt [T, blocks]).
int moe_down_col_blocks(int S, int H, int block_m) {
  if (block_m == 16) return H / 32;  // 32-column workgroups: CG 2 x 16, or CG 1 x 32 (narrow_k)
  if (block_m == 32) return H / 128;                   // CG 4 x 32 columns
  return H / 64;                                       // CG 4 x 16 columns
}

// Decode-tile GEMMs (block_m 16 / 32 / 64) or the prefill GEMMs (128).  Decode tiles: 16-row down
// GEMMs quantise h themselves where down_quantises_h; otherwise with tile_cnt (max_tiles x I/128
// counters, zero on entry) gate_up quantises h and no quant_h launch follows; with tok_cnt (T x moe_down_col_blocks counters, zero on entry) the down GEMM also sums
// each token's pair rows into comb (+ residual), and no combine launch is needed.
int moe_launch_grouped_gemms(const uint8_t* xq, const float* sx, const uint8_t* w13, const float* s13,
                             const uint8_t* w2, const float* s2, const int32_t* perm, const int32_t* tiles,
                             const int32_t* n_tiles, int max_tiles, const uint16_t* topk_w, uint16_t* h,
                             uint8_t* hq, float* sh, uint16_t* pairs, int S, int H, int I, int k,
                             int block_m, hipStream_t s, int32_t* tile_cnt, int32_t* tok_cnt, uint16_t* comb,
                             const uint16_t* residual) {
  if (block_m == 128)
    return moe_launch_grouped_gemms_prefill(xq, sx, w13, s13, w2, s2, perm, tiles, n_tiles, max_tiles, topk_w, hq,
                                            sh, pairs, H, I, k, s);
  const bool qh = block_m == 16 && down_quantises_h(S, I);
  GemmArgs g1{xq, sx, w13, s13, perm, tiles, n_tiles, nullptr, h, H, I, k, qh ? nullptr : tile_cnt, hq, sh,
              nullptr, nullptr, nullptr};
  g1.exact = moe_exact_accum(H);
  int rc;
  if (block_m == 16)
    rc = launch_gemm<MODE_GATE_UP, 1, 4>(g1, max_tiles, s);
  else if (block_m == 32)  // no K split: 64 h columns per workgroup share one load of the tile's rows
    rc = launch_gemm<MODE_GATE_UP, 2, 1, 1, true>(g1, max_tiles, s);
  else
    rc = launch_gemm<MODE_GATE_UP, 4, 1>(g1, max_tiles, s);
  if (rc) return rc;
  if (tile_cnt == nullptr && !qh) {
    // one pass quantises h for the larger tiles, whose down GEMMs would each repeat it
    rc = moe_launch_quant_act(h, S, I, hq, sh, s, MOE_PROF_QUANT_H);
    if (rc) return rc;
  }
  GemmArgs g2{qh ? (const uint8_t*)h : hq, qh ? nullptr : sh, w2, s2, perm, tiles, n_tiles, topk_w, pairs, I, H, k,
              nullptr, nullptr, nullptr, tok_cnt, comb, residual};
  g2.exact = moe_exact_accum(H);
  if (block_m == 16)
    rc = launch_down16(g2, S, max_tiles, qh, s, g1.tile_cnt != nullptr);
  else if (block_m == 32)
    rc = launch_gemm<MODE_DOWN, 2, 1, 2, true>(g2, max_tiles, s);
  else
    rc = launch_gemm<MODE_DOWN, 4, 1>(g2, max_tiles, s);
  return rc;
}

// Single-token decode (one row per routing slot, S = T * k <= 2 E): gate_up routes its own slot
// from the router GEMM's K-split partials (no top-k or sort launch) and writes the routing
// outputs, the identity slot order and the one-row tile list; then the down GEMM of the 16-row
// tiles, which quantises h itself (else gate_up does, through tile_cnt), with the in-launch token
// combine (tile_cnt and tok_cnt zero on entry).
// Every expert GEMM row is computed as on the sorted path, so the bits are the same.
int moe_launch_grouped_gemms_routed(const uint8_t* xq, const float* sx, const uint8_t* w13, const float* s13,
                                    const uint8_t* w2, const float* s2, const float* part, int ksplit, int T, int E,
                                    int renorm, uint16_t* logits, void* ids, int id_bytes, uint16_t* wts,
                                    int32_t* perm, int32_t* tiles, int32_t* n_tiles, uint16_t* h, uint8_t* hq,
                                    float* sh, uint16_t* pairs, int H, int I, int k, hipStream_t s, int32_t* tile_cnt,
                                    int32_t* tok_cnt, uint16_t* comb, const uint16_t* residual) {
  const int S = T * k;
  const bool qh = down_quantises_h(S, I);
  GemmArgs g1{xq, sx, w13, s13, perm, tiles, n_tiles, nullptr, h, H, I, k, qh ? nullptr : tile_cnt, hq, sh,
              nullptr, nullptr, nullptr, part, ksplit, T, E, renorm, logits, ids, id_bytes, wts, perm, tiles, n_tiles};
  g1.exact = moe_exact_accum(H);
  // gate_up with the wave's 3 or 4 K blocks unrolled (Qwen3-30B-A3B layer, 1 / 2 / 4 tokens:
  // gate_up 17.5 / 20.5 / 32.7 -> 16.2 / 20.1 / 31.0 us)
  const int KB1 = H / MOE_GROUP;
  int rc = KB1 == 16   ? launch_gemm_nkw<MODE_GATE_UP, 1, 4, 1, false, true, 4>(g1, S, s)
           : KB1 == 12 ? launch_gemm_nkw<MODE_GATE_UP, 1, 4, 1, false, true, 3>(g1, S, s)
                       : launch_gemm<MODE_GATE_UP, 1, 4, 1, false, true>(g1, S, s);
  if (rc) return rc;
  GemmArgs g2{qh ? (const uint8_t*)h : hq, qh ? nullptr : sh, w2, s2, perm, tiles, n_tiles, wts, pairs, I, H, k,
              nullptr, nullptr, nullptr, tok_cnt, comb, residual};
  g2.exact = moe_exact_accum(H);
  if (!qh && tile_cnt == nullptr) {
    rc = moe_launch_quant_act(h, S, I, hq, sh, s, MOE_PROF_QUANT_H);
    if (rc) return rc;
  }
  return launch_down16(g2, S, S, qh, s, g1.tile_cnt != nullptr);
}

// The 16-row decode GEMMs on expert-bucket tiles (moe_launch_route_buckets: no sort launch): the
// top-k kernel's last workgroup wrote the tile list, whose 4th field locates the tile's pairs in
// the buckets; h rows are dense in expert order, as on the sorted path.  Same hand-offs as
// moe_launch_grouped_gemms (h quantised by the down GEMM where down_quantises_h, else through
// tile_cnt up to 2 pairs per expert or a quant_h launch; tok_cnt for the token combine), and the
// same bits.
int moe_launch_grouped_gemms_buckets(const uint8_t* xq, const float* sx, const uint8_t* w13, const float* s13,
                                     const uint8_t* w2, const float* s2, const int32_t* bucket, const int32_t* tiles,
                                     const int32_t* n_tiles, int T, int max_tiles, const uint16_t* topk_w,
                                     uint16_t* h, uint8_t* hq, float* sh, uint16_t* pairs, int H, int I, int k,
                                     hipStream_t s, int32_t* tile_cnt, int32_t* tok_cnt, uint16_t* comb,
                                     const uint16_t* residual) {
  const int S = T * k;
  const bool qh = down_quantises_h(S, I);
  GemmArgs g1{xq, sx, w13, s13, nullptr, tiles, n_tiles, nullptr, h, H, I, k, qh ? nullptr : tile_cnt, hq, sh,
              nullptr, nullptr, nullptr};
  g1.exact = moe_exact_accum(H);
  g1.bucket = bucket;
  int rc = launch_gemm<MODE_GATE_UP, 1, 4>(g1, max_tiles, s);
  if (rc) return rc;
  if (tile_cnt == nullptr && !qh) {
    rc = moe_launch_quant_act(h, S, I, hq, sh, s, MOE_PROF_QUANT_H);
    if (rc) return rc;
  }
  GemmArgs g2{qh ? (const uint8_t*)h : hq, qh ? nullptr : sh, w2, s2, nullptr, tiles, n_tiles, topk_w, pairs, I, H, k,
              nullptr, nullptr, nullptr, tok_cnt, comb, residual};
  g2.exact = moe_exact_accum(H);
  g2.bucket = bucket;
  return launch_down16(g2, S, max_tiles, qh, s, g1.tile_cnt != nullptr);
}
