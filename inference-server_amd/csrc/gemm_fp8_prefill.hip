// Grouped FP8 GEMMs for prefill chunks (many rows per expert): LDS-tiled, persistent,
// XCD-aware, software-pipelined, MFMA-bound.
//
// Tile: 128 sorted rows of one expert x 256 weight rows x 128-deep K blocks.
//   gate_up: the 256 weight rows are 128 gate rows [n0, n0+128) and the matching 128 up
//            rows [I+n0, I+n0+128), so one tile yields 128 complete h columns = exactly
//            one 128-column quantisation group.  The epilogue computes h = silu(g)*u in
//            the reference's bf16 rounding order, the per-row group amax, and writes the
//            e4m3 intermediate and its scale directly (no bf16 h round trip through HBM).
//   down:    256 output columns; epilogue bf16(z) * routing weight, stored at the pair's
//            original row t*k+j.
//
// Workgroup: 8 waves, two per SIMD, in a 2 (rows) x 4 (weight rows) grid; a wave owns 64
// rows x 64 weight rows = 4 x 4 v_mfma_f32_16x16x128_f8f6f4 tiles per K block, each folded
// into the fp32 accumulator with the (activation row scale x weight tile scale) product.
//
// Pipeline, per K block kb: one barrier, after which (1) the DMA of K block kb+3 is issued
// into the LDS stage kb just vacated, (2) the fragments of K block kb+1 are read from LDS
// into the second register set, (3) the 16 MFMAs of K block kb run on the first set, with
// the scale FMAs of each MFMA trailing it.  LDS reads, DMA and MFMA/VALU of one wave thus
// overlap instead of alternating across barriers.
//
// Operands are staged through a ring of three 48.5 KB LDS stages (A 16 KB + B 32 KB +
// 512 B of activation scales) filled by global->LDS DMA without touching VGPRs.  LDS rows
// are 128 bytes, XOR-swizzled in 16-byte chunks (swz_key below) so that the lanes sharing an
// LDS cycle in a ds_read_b128 of an MFMA fragment hit distinct banks.
//
// Persistent grid: one workgroup per CU (the LDS footprint allows one).  Work items
// (tile, column block) are handed out so that the workgroups resident on one XCD
// (hardware places workgroup w on XCD w % 8) take consecutive items: they share the
// expert's weights and the tile's activations in that XCD's L2.
#include "common.h"
#include "lds_dma.h"

namespace {
using namespace moe_lds;

enum { PF_GATE_UP = 0, PF_DOWN = 1 };

constexpr int PBM = 128;             // rows per tile
constexpr int PBN = 256;             // weight rows per tile
constexpr int PBK = 128;             // K block (one scale block)
constexpr int P_A = PBM * PBK;       // 16 KB
constexpr int P_B = PBN * PBK;       // 32 KB
constexpr int P_STAGE = P_A + P_B;   // 48 KB
constexpr int kMaxKB = 32;           // K <= 4096
constexpr int P_WAVES = 8;            // two per SIMD: 2 (rows) x 4 (weight columns)
constexpr int P_THREADS = 64 * P_WAVES;

struct PrefillArgs {
  const uint8_t* a;        // gate_up: xq [T, K] (token rows); down: hq [S, K] (sorted rows)
  const float* sa;         // activation scales [rows, K/128]
  const uint8_t* w;        // [E, Nw, K]
  const float* sw;         // [E, Nw/128, K/128]
  const int32_t* perm;     // sorted row -> flat pair
  const int32_t* tiles;    // {expert, first sorted row, rows, 0}
  const int32_t* n_tiles;
  const uint16_t* topk_w;  // down: routing weights [S] (bf16)
  uint16_t* pairs;         // down: output [S, N] by flat pair
  uint8_t* hq;             // gate_up: e4m3 intermediate [S, N]
  float* sh;               // gate_up: its scales [S, N/128]
  uint16_t* h;             // bf16 weights, gate_up: the bf16 intermediate [S, N]
  int K;                   // reduction length (elements)
  int N;                   // gate_up: I; down: H
  int topk;
  int n_nblk;              // column blocks per tile: gate_up I/128, down H/256
  int exact;               // e4m3 operands widened to bf16 for exact bf16 MFMAs (moe_exact_accum)
};

constexpr int P_SA = PBM * 4;                 // 512 B of activation scales per stage
constexpr int P_STAGE3 = P_STAGE + P_SA;      // 49664 B
constexpr int P_DMA_A = P_A / 1024 / P_WAVES;  // 2 per wave
constexpr int P_DMA_B = P_B / 1024 / P_WAVES;  // 4 per wave
constexpr int P_DMA_PER_STEP = P_DMA_A + P_DMA_B + 1;  // + one activation-scale load

struct PfItem {
  int e, row0, rows, nb;
};

__device__ __forceinline__ PfItem pf_item(const PrefillArgs& p, int item) {
  const int tile = item / p.n_nblk;
  const int4 ti = const_ld4(p.tiles, tile);
  return {ti.x, ti.y, ti.z, item - tile * p.n_nblk};
}

// Splits one lane's 32-byte fragment of a 128-byte K block into the two 16-byte operands of the
// bf16 MFMAs (chunks 2 g and 2 g + 1 of the row for lane group g).
__device__ __forceinline__ v8bf frag_half(const v8i& f, int h) {
  return __builtin_bit_cast(v8bf, make_uint4(f[4 * h], f[4 * h + 1], f[4 * h + 2], f[4 * h + 3]));
}

// BF: bf16 activations and weights (a bf16 checkpoint).  A K block is then 64 elements, still 128
// bytes per row, so the LDS layout, the DMA and the fragment reads are the same; each fragment
// feeds two v_mfma_f32_16x16x32_bf16 (lane group g supplies K chunks 2 g and 2 g + 1, the same
// K permutation for both operands), which accumulate in fp32 in the MFMA: no scales, no FMAs.
// EX: e4m3 operands, each 128-deep K block as four exact bf16 MFMAs on the widened codes (see
// mfma_e4m3_exact) instead of one f8f6f4 MFMA.  The step runs in two halves of two weight
// fragments each; within a half, quarter jj of the four activation fragments is widened once and
// serves both weight fragments (a slot pair: 8 MFMAs, each of the 8 chains accumulating over jj
// in the MFMA), so a step widens 192 code pairs per lane instead of 320 with one activation
// widening per MFMA (the conversions, not the MFMAs, bounded that form: 235B prefill gate_up
// 845 -> 700 us, down 439 -> 370 us, same bits).  Half 1's first slots fold half 0's chains into
// the accumulators just before reusing their registers.  Widening whole fragments up front
// spilled ~50 registers.
template <int MODE, bool BF, bool EX = false>
__global__ __launch_bounds__(P_THREADS, 1) void grouped_gemm_fp8_prefill_kernel(PrefillArgs p) {
  static_assert(!(BF && EX), "exact accumulation is for e4m3 operands");
  __shared__ __attribute__((aligned(16))) uint8_t s_ab[3][P_STAGE3];
  __shared__ __attribute__((aligned(16))) int s_perm[2][PBM];  // perm rows of the item, by item parity
  __shared__ __attribute__((aligned(16))) float s_swt[2][2][kMaxKB];  // its weight tile scales, per K block
  __shared__ float s_amax[4][PBM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keep it in an SGPR
  const int wm = wave & 1, wn = wave >> 1;  // 2 x 4 waves: rows wm*64, weight-column quarter wn
  const int lr = lane & 15, lg = lane >> 4;
  const int c0 = 2 * lg;
  const int K = BF ? 2 * p.K : p.K;  // bytes per operand row
  const int KB = K / PBK;              // 128-byte K blocks
  constexpr int DPS = BF ? P_DMA_A + P_DMA_B : P_DMA_PER_STEP;  // DMA instructions per step and wave
  const int Nw = MODE == PF_GATE_UP ? 2 * p.N : p.N;
  const int nblk128 = Nw / PBK;
  const int n_items = const_ld(p.n_tiles, 0) * p.n_nblk;
  const int G = gridDim.x;  // a multiple of 8
  const int my_slot = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  if (my_slot >= n_items) return;  // workgroup-uniform
  const int n_my = (n_items - my_slot + G - 1) / G;  // items of this workgroup: my_slot + j G
  const int S_tot = n_my * KB;                        // K-block steps over all of them
  const uint32_t lds_stage0 = __builtin_amdgcn_readfirstlane(lds_u32(&s_ab[0][0]));
  const uint32_t lds_perm0 = __builtin_amdgcn_readfirstlane(lds_u32(&s_perm[0][0]));
  const uint32_t lds_swt0 = __builtin_amdgcn_readfirstlane(lds_u32(&s_swt[0][0][0]));

  // DMA lane assignment: one instruction fills 8 rows x 128 B (block jb = rows 8jb..8jb+7).
  // Lane L writes position L & 7 of row 8 jb + (L >> 3), which holds logical chunk
  // (L & 7) ^ swz_key(row) = (L & 7) ^ ((L >> 3) ^ (jb & 1)).  This wave fills blocks
  // jb = wave + 8 i, so jb & 1 = wave & 1 for all of them.
  const int dma_r = lane >> 3;
  const int dma_lc = (lane & 7) ^ ((dma_r ^ (wave & 1)) & 7);
  // this lane's byte offset within a 16-row fragment group, for chunk columns c0 and c0 + 1
  const int frag_off0 = lr * 128 + ((c0 ^ swz_key(lr)) << 4);
  const int frag_off1 = lr * 128 + (((c0 + 1) ^ swz_key(lr)) << 4);
  // per-lane B offsets (from the item's weight base) of this wave's blocks wave + 8 i:
  // gate_up tile rows 128.. are the up rows, I - 128 rows further on
  uint32_t b_voff[P_DMA_B];
#pragma unroll
  for (int i = 0; i < P_DMA_B; ++i) {
    const int br = 8 * (wave + 8 * i);
    const int wrow = MODE == PF_GATE_UP && br >= 128 ? p.N - 128 + br : br;
    b_voff[i] = (uint32_t)((wrow + dma_r) * K + dma_lc * 16);
  }

  // MFMA operand order: the weight fragment is the MFMA's A operand and the activation
  // fragment its B operand, so the 16x16 result tile is (weight column n, token row m) and
  // lane l holds columns n = 4 (l >> 4) + q, q = 0..3, of token row m = l & 15: four
  // consecutive output columns of one row per lane.
  // Weight row (within the 256-row tile) of fragment ni of this wave: gate_up gate rows
  // wn*32 + 16 ni (ni < 2) and the matching up rows 128 + wn*32 + 16 (ni - 2); down wn*64 + 16 ni.
#define PF_BROW(ni) \
  ((MODE == PF_GATE_UP ? ((ni) < 2 ? wn * 32 + (ni) * 16 : 128 + wn * 32 + ((ni) - 2) * 16) : wn * 64 + (ni) * 16) + lr)

  // ---- issue side: the item whose K blocks are being loaded ----
  uint32_t a_voff[P_DMA_A];  // per-lane A byte offsets of this wave's DMA blocks (wave + 8 i)
  uint32_t sa_voff;          // per-lane activation-scale byte offset (lanes < 16)
  const uint8_t* wbase;      // uniform: weight row of tile row 0 (gate_up: the gate half)

  // tables of item j -> slot j & 1: its perm rows (rows past the tile end repeat the last
  // row) and the weight tile scales of all its K blocks (waves 0 and 1: gate_up gate block nb
  // and up block I/128 + nb; down blocks 2 nb and 2 nb + 1, the two 128-row halves)
#define PF_TABLE(it_, j_)                                                                         \
  do {                                                                                            \
    const int r_ = 16 * wave + lr;                                                                \
    if (lane < 16)                                                                                \
      dma_b32<0>((uint32_t)((it_).row0 + min(r_, (it_).rows - 1)) * 4u, p.perm,                  \
                 lds_perm0 + ((j_) & 1) * (PBM * 4) + 64 * wave);                                 \
    if (!BF && wave < 2 && lane < KB) {                                                           \
      const int blk_ = MODE == PF_GATE_UP ? (wave == 0 ? (it_).nb : p.N / PBK + (it_).nb) : 2 * (it_).nb + wave; \
      dma_b32<0>((uint32_t)(((it_).e * nblk128 + blk_) * KB + lane) * 4u, p.sw,                  \
                 lds_swt0 + (((j_) & 1) * 2 + wave) * (kMaxKB * 4));                              \
    }                                                                                             \
  } while (0)

  // per-lane DMA offsets of item it_ (its table is in s_perm[j_ & 1] and visible)
#define PF_DESC(it_, j_)                                                                          \
  do {                                                                                            \
    _Pragma("unroll") for (int i = 0; i < P_DMA_A; ++i) {                                         \
      const int r_ = 8 * (wave + 8 * i) + dma_r;                                                  \
      const int arow_ = MODE == PF_GATE_UP ? s_perm[(j_) & 1][r_] / p.topk                        \
                                           : (it_).row0 + min(r_, (it_).rows - 1);                \
      a_voff[i] = (uint32_t)(arow_ * K + dma_lc * 16);                                            \
    }                                                                                             \
    const int rs_ = 16 * wave + lr;                                                               \
    const int srow_ = MODE == PF_GATE_UP ? s_perm[(j_) & 1][rs_] / p.topk                         \
                                         : (it_).row0 + min(rs_, (it_).rows - 1);                 \
    sa_voff = (uint32_t)(srow_ * KB) * 4u;                                                        \
    wbase = p.w + ((long)(it_).e * Nw + (long)(it_).nb * (MODE == PF_GATE_UP ? 128 : 256)) * K;   \
  } while (0)

  // one of the 7 DMA instructions of a K block, by index d_ (0..1 A, 2..5 B, 6 scales), with
  // the bases of the K block computed (sbw_: this wave's first block in the stage)
#define PF_DMA_ONE(d_, ab_, bb_, sab_, sbw_)                                                      \
  do {                                                                                            \
    if constexpr ((d_) < P_DMA_A) dma_b128<(d_) * 8192>(a_voff[d_], ab_, sbw_);                   \
    else if constexpr ((d_) < P_DMA_A + P_DMA_B)                                                  \
      dma_b128<P_A + ((d_) - P_DMA_A) * 8192>(b_voff[(d_) - P_DMA_A], bb_, sbw_);                 \
    else if (!BF && lane < 16) dma_b32<0>(sa_voff, sab_, (sbw_) - 1024 * wave + P_STAGE + 64 * wave); \
  } while (0)

  // weight tile scales of K block kb_ of item j_ for this wave: gate_up (gate, up); down the
  // 128-row half of the wave's columns
#define PF_SW(SW_, j_, kb_)                                                                       \
  do {                                                                                            \
    if constexpr (BF) {                                                                           \
    } else if constexpr (MODE == PF_GATE_UP) {                                                    \
      SW_[0] = s_swt[(j_) & 1][0][kb_];                                                           \
      SW_[1] = s_swt[(j_) & 1][1][kb_];                                                           \
    } else {                                                                                      \
      SW_[0] = SW_[1] = s_swt[(j_) & 1][wn >> 1][kb_];                                            \
    }                                                                                             \
  } while (0)

  // fragments and activation scales of the K block in stage st_ (the four token rows
  // wm*64 + mi*16 + lr of this lane)
#define PF_READ(A_, B_, SV_, st_)                                                                 \
  do {                                                                                            \
    const uint8_t* sA_ = s_ab[st_];                                                               \
    const uint8_t* sB_ = sA_ + P_A;                                                               \
    const float* sS_ = (const float*)(sA_ + P_STAGE);                                             \
    _Pragma("unroll") for (int mi = 0; mi < 4; ++mi) A_[mi] = lds_frag(sA_, wm * 64 + mi * 16 + lr, c0); \
    _Pragma("unroll") for (int ni = 0; ni < 4; ++ni) B_[ni] = lds_frag(sB_, PF_BROW(ni), c0);     \
    if constexpr (!BF) {                                                                          \
      _Pragma("unroll") for (int mi = 0; mi < 4; ++mi) SV_[mi] = sS_[wm * 64 + mi * 16 + lr];     \
    }                                                                                             \
  } while (0)

  // One step's 16 MFMAs (A fragments AC, B fragments B, scales SC/WC; MFMA order ni-major)
  // with the LDS reads of the next step's fragments (A into AN; each B fragment in place
  // two slots after its last MFMA of this step), the DMA of K block s+3 and the scale FMAs
  // interleaved in a fixed order: per slot an MFMA, one LDS read, every other slot a DMA,
  // then the FMAs of the MFMA three slots back (its result is ready by then).
  // sched_barrier pins the order.
#define PF_RD_A(AN_, mi_, h_)                                                                     \
  do {                                                                                            \
    const uint4 v_ = *(const uint4*)(sA_ + (wm * 64 + (mi_) * 16) * 128 + ((h_) ? frag_off1 : frag_off0)); \
    AN_[mi_][4 * (h_)] = v_.x; AN_[mi_][4 * (h_) + 1] = v_.y; AN_[mi_][4 * (h_) + 2] = v_.z; AN_[mi_][4 * (h_) + 3] = v_.w; \
  } while (0)
#define PF_RD_B(B_, ni_, h_)                                                                      \
  do {                                                                                            \
    const uint4 v_ = *(const uint4*)(sB_ + (PF_BROW(ni_) - lr) * 128 + ((h_) ? frag_off1 : frag_off0)); \
    B_[ni_][4 * (h_)] = v_.x; B_[ni_][4 * (h_) + 1] = v_.y; B_[ni_][4 * (h_) + 2] = v_.z; B_[ni_][4 * (h_) + 3] = v_.w; \
  } while (0)
// An empty volatile asm that takes and returns v_: the value is computed before this point
// and the volatile asm statements keep their order, which holds each MFMA and each scale FMA in
// its slot (sched_barrier alone binds only the machine scheduler: without the pins the FMAs
// were sunk below all 16 MFMAs, every MFMA result stayed live and the step lost its overlap).
#define PF_PIN(v_) asm volatile("" : "+v"(v_))
#define PF_STEP_BODY(AC, AN, B, SC, SN, WC, WN, st_, j1_, kb1_, ab_, bb_, sab_, sbw_)             \
  do {                                                                                            \
    const uint8_t* sA_ = s_ab[st_];                                                               \
    const uint8_t* sB_ = sA_ + P_A;                                                               \
    const float* sS_ = (const float*)(sA_ + P_STAGE);                                             \
    float sca_[4], scb_[4];                                                                       \
    _Pragma("unroll") for (int mi = 0; mi < 4; ++mi) {                                            \
      sca_[mi] = SC[mi] * WC[0];                                                                  \
      scb_[mi] = MODE == PF_GATE_UP ? SC[mi] * WC[1] : sca_[mi];                                  \
    }                                                                                             \
    v4f t_[4];                                                                                    \
    v4f tx_[2][4];                                                                                \
    v8bf aq_[4];                                                                                  \
    _Pragma("unroll") for (int it = 0; it < 21; ++it) {                                           \
      if (it < 16 && !EX) {                                                                       \
        const int ni = it >> 2, mi = it & 3;                                                      \
        t_[it & 3] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(B[ni], AC[mi], zero4, 0, 0, 0, 0, 0, 0); \
        PF_PIN(t_[it & 3]);                                                                       \
      }                                                                                           \
      if (it < 16 && EX) {                                                                        \
        /* slot (h, jj, nl): weight fragment ni = 2 h + nl, 32-deep quarter jj of the K block. */ \
        /* The quarter of the four activation fragments is widened once per (h, jj) and shared */ \
        /* by the slot pair; each of the pair's eight chains runs over jj in one register set. */ \
        /* Half 1 folds half 0's chain (same registers) just before overwriting it. */           \
        const int h = it >> 3, jj = (it >> 1) & 3, nl = it & 1, ni = 2 * h + nl;                  \
        if (nl == 0) {                                                                            \
          _Pragma("unroll") for (int mi = 0; mi < 4; ++mi) {                                      \
            uint32_t a0_ = (uint32_t)AC[mi][2 * jj], a1_ = (uint32_t)AC[mi][2 * jj + 1];          \
            asm volatile("" : "+v"(a0_), "+v"(a1_));                                              \
            aq_[mi] = e4m3x8_to_bf16(a0_, a1_);                                                   \
          }                                                                                       \
        }                                                                                         \
        uint32_t b0_ = (uint32_t)B[ni][2 * jj], b1_ = (uint32_t)B[ni][2 * jj + 1];                \
        asm volatile("" : "+v"(b0_), "+v"(b1_));                                                  \
        const v8bf bw_ = e4m3x8_to_bf16(b0_, b1_);                                                \
        _Pragma("unroll") for (int mi = 0; mi < 4; ++mi) {                                        \
          if (h == 1 && jj == 0) {                                                                \
            _Pragma("unroll") for (int q = 0; q < 4; ++q)                                         \
              acc[mi][nl][q] = fmaf(tx_[nl][mi][q], sca_[mi], acc[mi][nl][q]);                    \
            PF_PIN(acc[mi][nl]);                                                                  \
          }                                                                                       \
          tx_[nl][mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bw_, aq_[mi], jj == 0 ? zero4 : tx_[nl][mi], 0, 0, 0); \
          PF_PIN(tx_[nl][mi]);                                                                    \
        }                                                                                         \
      }                                                                                           \
      if constexpr (EX) {                                                                         \
        /* B fragment parts are reloaded one slot or more after their last quarter's MFMAs */   \
        switch (it) {                                                                             \
          case 0: PF_RD_A(AN, 0, 0); break;                                                       \
          case 1: PF_RD_A(AN, 0, 1); break;                                                       \
          case 2: PF_RD_A(AN, 1, 0); break;                                                       \
          case 3: PF_RD_A(AN, 1, 1); break;                                                       \
          case 4: PF_RD_B(B, 0, 0); break;                                                        \
          case 5: PF_RD_B(B, 1, 0); break;                                                        \
          case 6: PF_RD_A(AN, 2, 0); break;                                                       \
          case 7: PF_RD_B(B, 0, 1); break;                                                        \
          case 8: PF_RD_B(B, 1, 1); break;                                                        \
          case 9: PF_RD_A(AN, 2, 1); break;                                                       \
          case 10: PF_RD_A(AN, 3, 0); break;                                                      \
          case 11: PF_RD_A(AN, 3, 1); break;                                                      \
          case 12: SN[0] = sS_[wm * 64 + lr]; break;                                              \
          case 13: PF_RD_B(B, 2, 0); break;                                                       \
          case 14: PF_RD_B(B, 3, 0); break;                                                       \
          case 15: SN[1] = sS_[wm * 64 + 16 + lr]; break;                                         \
          case 16: PF_RD_B(B, 2, 1); break;                                                       \
          case 17: PF_RD_B(B, 3, 1); break;                                                       \
          case 18: SN[2] = sS_[wm * 64 + 32 + lr]; break;                                         \
          case 19: SN[3] = sS_[wm * 64 + 48 + lr]; break;                                         \
          default: PF_SW(WN, j1_, kb1_); break;                                                   \
        }                                                                                         \
      } else {                                                                                    \
        switch (it) {                                                                             \
          case 0: PF_RD_A(AN, 0, 0); break;                                                       \
          case 1: PF_RD_A(AN, 0, 1); break;                                                       \
          case 2: PF_RD_A(AN, 1, 0); break;                                                       \
          case 3: PF_RD_A(AN, 1, 1); break;                                                       \
          case 4: PF_RD_A(AN, 2, 0); break;                                                       \
          case 5: PF_RD_B(B, 0, 0); break;                                                        \
          case 6: PF_RD_B(B, 0, 1); break;                                                        \
          case 7: PF_RD_A(AN, 2, 1); break;                                                       \
          case 8: PF_RD_A(AN, 3, 0); break;                                                       \
          case 9: PF_RD_B(B, 1, 0); break;                                                        \
          case 10: PF_RD_B(B, 1, 1); break;                                                       \
          case 11: PF_RD_A(AN, 3, 1); break;                                                      \
          case 12: SN[0] = sS_[wm * 64 + lr]; break;                                              \
          case 13: PF_RD_B(B, 2, 0); break;                                                       \
          case 14: PF_RD_B(B, 2, 1); break;                                                       \
          case 15: SN[1] = sS_[wm * 64 + 16 + lr]; break;                                         \
          case 16: SN[2] = sS_[wm * 64 + 32 + lr]; break;                                         \
          case 17: PF_RD_B(B, 3, 0); break;                                                       \
          case 18: PF_RD_B(B, 3, 1); break;                                                       \
          case 19: SN[3] = sS_[wm * 64 + 48 + lr]; break;                                         \
          default: PF_SW(WN, j1_, kb1_); break;                                                   \
        }                                                                                         \
      }                                                                                           \
      if (it == 1) PF_DMA_ONE(0, ab_, bb_, sab_, sbw_);                                           \
      if (it == 3) PF_DMA_ONE(1, ab_, bb_, sab_, sbw_);                                           \
      if (it == 5) PF_DMA_ONE(2, ab_, bb_, sab_, sbw_);                                           \
      if (it == 7) PF_DMA_ONE(3, ab_, bb_, sab_, sbw_);                                           \
      if (it == 9) PF_DMA_ONE(4, ab_, bb_, sab_, sbw_);                                           \
      if (it == 11) PF_DMA_ONE(5, ab_, bb_, sab_, sbw_);                                          \
      if (it == 13) PF_DMA_ONE(6, ab_, bb_, sab_, sbw_);                                          \
      if (!EX && it >= 3 && it < 19) {                                                            \
        const int j = it - 3, ni = j >> 2, mi = j & 3;                                            \
        const float sc_ = (MODE == PF_GATE_UP && ni >= 2) ? scb_[mi] : sca_[mi];                  \
        _Pragma("unroll") for (int q = 0; q < 4; ++q) acc[mi][ni][q] = fmaf(t_[j & 3][q], sc_, acc[mi][ni][q]); \
        PF_PIN(acc[mi][ni]);                                                                      \
      }                                                                                           \
      if (EX && (it == 16 || it == 17)) {                                                         \
        /* half 1's chains (weight fragments 2 and 3), one slot after their last quarter */      \
        const int nl = it - 16, ni = 2 + nl;                                                      \
        _Pragma("unroll") for (int mi = 0; mi < 4; ++mi) {                                        \
          const float sc_ = MODE == PF_GATE_UP ? scb_[mi] : sca_[mi];                             \
          _Pragma("unroll") for (int q = 0; q < 4; ++q)                                           \
            acc[mi][ni][q] = fmaf(tx_[nl][mi][q], sc_, acc[mi][ni][q]);                           \
          PF_PIN(acc[mi][ni]);                                                                    \
        }                                                                                         \
      }                                                                                           \
      __builtin_amdgcn_sched_barrier(0);                                                          \
    }                                                                                             \
  } while (0)

  // bf16: 32 MFMAs per step, for each weight fragment ni its low halves (mi = 0..3) then its
  // high halves, so that an accumulator's two MFMAs are four MFMAs apart; the next step's A
  // fragments are read in slots 0-7 and each B fragment is reloaded in place after its last MFMA
#define PF_STEP_BODY_BF(AC, AN, B, st_, ab_, bb_, sab_, sbw_)                                     \
  do {                                                                                            \
    const uint8_t* sA_ = s_ab[st_];                                                               \
    const uint8_t* sB_ = sA_ + P_A;                                                               \
    _Pragma("unroll") for (int it = 0; it < 34; ++it) {                                           \
      if (it < 32) {                                                                              \
        const int ni = it >> 3, hh = (it >> 2) & 1, mi = it & 3;                                  \
        acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(frag_half(B[ni], hh), frag_half(AC[mi], hh), \
                                                              acc[mi][ni], 0, 0, 0);             \
      }                                                                                           \
      if (it < 8) PF_RD_A(AN, it >> 1, it & 1);                                                   \
      if (it == 8 || it == 9) PF_RD_B(B, 0, it - 8);                                              \
      if (it == 16 || it == 17) PF_RD_B(B, 1, it - 16);                                           \
      if (it == 24 || it == 25) PF_RD_B(B, 2, it - 24);                                           \
      if (it == 32 || it == 33) PF_RD_B(B, 3, it - 32);                                           \
      if (it == 1) PF_DMA_ONE(0, ab_, bb_, sab_, sbw_);                                           \
      if (it == 3) PF_DMA_ONE(1, ab_, bb_, sab_, sbw_);                                           \
      if (it == 5) PF_DMA_ONE(2, ab_, bb_, sab_, sbw_);                                           \
      if (it == 7) PF_DMA_ONE(3, ab_, bb_, sab_, sbw_);                                           \
      if (it == 9) PF_DMA_ONE(4, ab_, bb_, sab_, sbw_);                                           \
      if (it == 11) PF_DMA_ONE(5, ab_, bb_, sab_, sbw_);                                          \
      __builtin_amdgcn_sched_barrier(0);                                                          \
    }                                                                                             \
  } while (0)

  const v4f zero4 = {0.f, 0.f, 0.f, 0.f};
  v4f acc[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = zero4;
  v8i a0[4], a1[4], bf[4];
  float sv0[4], sv1[4];
  float sw_0[2], sw_1[2];

  // ---- prologue: item 0's table, its descriptors, K blocks 0..2 in flight ----
  PfItem it_c = pf_item(p, my_slot);  // the item being computed
  PfItem it_i = it_c;                 // the item being issued
  PF_TABLE(it_c, 0);
  wait_vm<0>();
  lds_wait_barrier();
  PF_DESC(it_i, 0);
  // K blocks 0..2 of item 0 (the pipelined path needs KB >= 4, checked by the launcher)
#pragma unroll
  for (int k0 = 0; k0 < 3; ++k0) {
    const uint8_t* ab_ = p.a + (long)k0 * PBK;
    const uint8_t* bb_ = wbase + (long)k0 * PBK;
    const float* sab_ = p.sa + k0;
    const uint32_t sbw_ = lds_stage0 + k0 * P_STAGE3 + 1024 * wave;
    PF_DMA_ONE(0, ab_, bb_, sab_, sbw_);
    PF_DMA_ONE(1, ab_, bb_, sab_, sbw_);
    PF_DMA_ONE(2, ab_, bb_, sab_, sbw_);
    PF_DMA_ONE(3, ab_, bb_, sab_, sbw_);
    PF_DMA_ONE(4, ab_, bb_, sab_, sbw_);
    PF_DMA_ONE(5, ab_, bb_, sab_, sbw_);
    PF_DMA_ONE(6, ab_, bb_, sab_, sbw_);
  }
  wait_vm<2 * DPS>();
  lds_wait_barrier();
  PF_READ(a0, bf, sv0, 0);
  PF_SW(sw_0, 0, 0);

  // step counters (uniform): compute step s = K block kb of item j in stage st; issue
  // target s+3 = K block kb3 of item j3, also into stage st
  int s = 0, j = 0, kb = 0, st = 0, j3 = 0, kb3 = 3;

  // Step s: wait until K block s+1 has landed (s+2 may stay in flight) and this wave's
  // fragment reads of s are done; at kb = 0 start the table DMA of item j+1; refill stage
  // st with K block s+3 (switching the issue side to item j+1 at its first K block) and
  // read the fragments of s+1 while computing s; at kb = KB-1 run item j's epilogue.
  // Loads complete in order, so the wait counts are exact.
#define PF_STEP(AC, AN, SC, SN, WC, WN)                                                           \
  do {                                                                                            \
    if (s + 2 < S_tot)                                                                            \
      wait_vm<DPS>();                                                                             \
    else                                                                                          \
      wait_vm<0>();                                                                               \
    lds_wait_barrier();                                                                           \
    if (kb == 0 && j + 1 < n_my) {                                                                \
      const PfItem nx_ = pf_item(p, my_slot + (j + 1) * G);                                       \
      PF_TABLE(nx_, j + 1);                                                                       \
    }                                                                                             \
    /* DMA target: K block s+3; past the last step the stage just freed is refilled with */      \
    /* a valid block again (no branch in the step body), waited for by the tail's vmcnt(0) */     \
    const int live_ = s + 3 < S_tot;                                                              \
    if (live_ && kb3 == 0) {                                                                      \
      it_i = pf_item(p, my_slot + j3 * G);                                                        \
      PF_DESC(it_i, j3);                                                                          \
    }                                                                                             \
    const int kbi_ = live_ ? kb3 : KB - 1;                                                        \
    const uint8_t* ab_ = p.a + (long)kbi_ * PBK;                                                  \
    const uint8_t* bb_ = wbase + (long)kbi_ * PBK;                                                \
    const float* sab_ = p.sa + kbi_;                                                              \
    const uint32_t sbw_ = lds_stage0 + st * P_STAGE3 + 1024 * wave;                               \
    if (live_ && ++kb3 == KB) {                                                                   \
      kb3 = 0;                                                                                    \
      ++j3;                                                                                       \
    }                                                                                             \
    const int last_ = kb == KB - 1;                                                               \
    const int st1_ = st == 2 ? 0 : st + 1;                                                        \
    /* fragments of step s+1 (past the last step: a harmless read of a stale stage) */           \
    if constexpr (BF)                                                                             \
      PF_STEP_BODY_BF(AC, AN, bf, st1_, ab_, bb_, sab_, sbw_);                                    \
    else                                                                                          \
      PF_STEP_BODY(AC, AN, bf, SC, SN, WC, WN, st1_, j + last_, last_ ? 0 : kb + 1, ab_, bb_, sab_, sbw_); \
    if (last_) {                                                                                  \
      pf_epilogue(j);                                                                             \
      _Pragma("unroll") for (int mi = 0; mi < 4; ++mi)                                            \
        _Pragma("unroll") for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = zero4;                     \
      ++j;                                                                                        \
      kb = 0;                                                                                     \
      if (j < n_my) it_c = pf_item(p, my_slot + j * G);                                           \
    } else {                                                                                      \
      ++kb;                                                                                       \
    }                                                                                             \
    st = st1_;                                                                                    \
    ++s;                                                                                          \
  } while (0)

  // epilogue of item j (it_c), straight from the accumulators: lane holds, for token rows
  // r = wm*64 + mi*16 + lr, the columns 16 ni + 4 lg + q of this wave's weight rows
  auto pf_epilogue = [&](int jj) __attribute__((always_inline)) {
    const int row0 = it_c.row0, rows = it_c.rows, nb = it_c.nb;
    if constexpr (MODE == PF_GATE_UP && BF) {
      // h = bf16(bf16(silu(bf16 g)) * bf16 u) in bf16, four consecutive h columns per lane and row
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        if (wm * 64 + mi * 16 >= rows) continue;  // the 16-row group lies past the tile (uniform)
        const int r = wm * 64 + mi * 16 + lr;
        if (r >= rows) continue;
        uint16_t* dst = p.h + (long)(row0 + r) * p.N + nb * 128 + wn * 32 + 4 * lg;
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
          uint2 v;
          v.x = (uint32_t)f32_to_bf16(silu_mul_bf16(acc[mi][ni][0], acc[mi][ni + 2][0])) |
                ((uint32_t)f32_to_bf16(silu_mul_bf16(acc[mi][ni][1], acc[mi][ni + 2][1])) << 16);
          v.y = (uint32_t)f32_to_bf16(silu_mul_bf16(acc[mi][ni][2], acc[mi][ni + 2][2])) |
                ((uint32_t)f32_to_bf16(silu_mul_bf16(acc[mi][ni][3], acc[mi][ni + 2][3])) << 16);
          *(uint2*)(dst + ni * 16) = v;
        }
      }
    } else if constexpr (MODE == PF_GATE_UP) {
      // h = bf16(bf16(silu(bf16 g)) * bf16 u): gate frags 0, 1 pair with up frags 2, 3, so
      // this wave holds h columns wn*32 + 16 ni + 4 lg + q
      float rmax[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        float m = 0.f;
        rmax[mi] = 0.f;
        // a 16-row group past the tile's end computes nothing (wave-uniform): its rows are
        // never stored, and its amax slots are read only for its own rows
        if (wm * 64 + mi * 16 >= rows) continue;
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float h = silu_mul_bf16(acc[mi][ni][q], acc[mi][ni + 2][q]);
            acc[mi][ni][q] = h;
            m = fmaxf(m, fabsf(h));
          }
        // the four lanes lr, lr+16, lr+32, lr+48 share the row
        m = fmaxf(m, __shfl_xor(m, 16));
        m = fmaxf(m, __shfl_xor(m, 32));
        rmax[mi] = m;
      }
      if (lg == 0) {
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) s_amax[wn][wm * 64 + mi * 16 + lr] = rmax[mi];
      }
      lds_wait_barrier();
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        if (wm * 64 + mi * 16 >= rows) continue;
        const int r = wm * 64 + mi * 16 + lr;
        const float amax = fmaxf(fmaxf(s_amax[0][r], s_amax[1][r]), fmaxf(s_amax[2][r], s_amax[3][r]));
        const float sc = amax > 0.f ? amax / MOE_FP8_MAX : 1.0f;
        if (r < rows) {
          const long srow = row0 + r;
          // h / s rounded as the oracle's division (div_rn): h and amax are bf16, so 448 h / amax
          // often lands exactly on an e4m3 rounding midpoint, where h * (1 / s) (two roundings)
          // falls on either side (0.05% of the codes differed that way)
          uint8_t* dst = p.hq + srow * p.N + nb * 128 + wn * 32 + 4 * lg;
#pragma unroll
          for (int ni = 0; ni < 2; ++ni)
            *(uint32_t*)(dst + ni * 16) = pack4_e4m3(clamp_fp8(div_rn(acc[mi][ni][0], sc)), clamp_fp8(div_rn(acc[mi][ni][1], sc)),
                                                     clamp_fp8(div_rn(acc[mi][ni][2], sc)),
                                                     clamp_fp8(div_rn(acc[mi][ni][3], sc)));
          if (wn == 0 && lg == 0) p.sh[srow * (p.N / PBK) + nb] = sc;
        }
      }
    } else {
      // bf16(z) at the pair's row; the combine applies the routing weight
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        if (wm * 64 + mi * 16 >= rows) continue;
        const int r = wm * 64 + mi * 16 + lr;
        if (r < rows) {
          const long pr = s_perm[jj & 1][r];
          uint16_t* dst = p.pairs + pr * p.N + nb * 256 + wn * 64 + 4 * lg;
#pragma unroll
          for (int ni = 0; ni < 4; ++ni) {
            uint2 v;
            v.x = (uint32_t)f32_to_bf16(acc[mi][ni][0]) | ((uint32_t)f32_to_bf16(acc[mi][ni][1]) << 16);
            v.y = (uint32_t)f32_to_bf16(acc[mi][ni][2]) | ((uint32_t)f32_to_bf16(acc[mi][ni][3]) << 16);
            *(uint2*)(dst + ni * 16) = v;
          }
        }
      }
    }
  };

  while (s < S_tot) {
    PF_STEP(a0, a1, sv0, sv1, sw_0, sw_1);
    if (s < S_tot) PF_STEP(a1, a0, sv1, sv0, sw_1, sw_0);
  }
#undef PF_STEP
#undef PF_STEP_BODY
#undef PF_PIN
#undef PF_STEP_BODY_BF
#undef PF_RD_A
#undef PF_RD_B
#undef PF_READ
#undef PF_SW
#undef PF_DMA_ONE
#undef PF_DESC
#undef PF_TABLE
#undef PF_BROW
}

int device_cu_count() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}

template <int MODE, bool BF = false>
int launch_prefill(const PrefillArgs& a, int max_tiles, hipStream_t s) {
  const long max_items = (long)max_tiles * a.n_nblk;
  long g = device_cu_count();
  if (g > max_items) g = max_items;
  g = (g + 7) / 8 * 8;
  if (g < 8) g = 8;
  if (!BF && a.exact)
    MOE_LAUNCH(MODE == PF_GATE_UP ? MOE_PROF_GATE_UP : MOE_PROF_DOWN, s,
               (grouped_gemm_fp8_prefill_kernel<MODE, false, true>), dim3((unsigned)g), dim3(P_THREADS), 0, s, a);
  else
    MOE_LAUNCH(MODE == PF_GATE_UP ? MOE_PROF_GATE_UP : MOE_PROF_DOWN, s, (grouped_gemm_fp8_prefill_kernel<MODE, BF>),
               dim3((unsigned)g), dim3(P_THREADS), 0, s, a);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}

}  // namespace

// gate_up (with fused SiLU*up and e4m3 re-quantisation of h) then down, for block_m = 128 tiles.
int moe_launch_grouped_gemms_prefill(const uint8_t* xq, const float* sx, const uint8_t* w13, const float* s13,
                                     const uint8_t* w2, const float* s2, const int32_t* perm, const int32_t* tiles,
                                     const int32_t* n_tiles, int max_tiles, const uint16_t* topk_w, uint8_t* hq,
                                     float* sh, uint16_t* pairs, int H, int I, int k, hipStream_t s) {
  // the DMA takes 32-bit per-lane byte offsets into the activations: rows (<= the sorted
  // row capacity) x K must stay below 2^32
  const long max_rows = (long)max_tiles * PBM;
  if (max_rows * (H > I ? H : I) >= (1L << 32)) return MOE_ERR_INVALID_ARG;
  // the cross-item DMA pipeline needs at least 4 K blocks per GEMM
  if (H / PBK < 4 || I / PBK < 4 || H % PBN != 0) return MOE_ERR_INVALID_ARG;
  PrefillArgs g1{xq, sx, w13, s13, perm, tiles, n_tiles, nullptr, nullptr, hq, sh, nullptr, H, I, k, I / PBK,
                 moe_exact_accum(H)};
  int rc = launch_prefill<PF_GATE_UP>(g1, max_tiles, s);
  if (rc) return rc;
  PrefillArgs g2{hq, sh, w2, s2, perm, tiles, n_tiles, topk_w, pairs, nullptr, nullptr, nullptr, I, H, k, H / PBN,
                 moe_exact_accum(H)};
  return launch_prefill<PF_DOWN>(g2, max_tiles, s);
}

// Whether bf16 experts of this shape can take the 128-row tiles (bf16 K blocks are 64 deep).
bool moe_prefill_bf16_ok(int H, int I, long max_rows) {
  return H % PBN == 0 && H / 64 >= 4 && I / 64 >= 4 && I % MOE_GROUP == 0 &&
         max_rows * 2 * (H > I ? H : I) < (1L << 32);
}

// The same pair of GEMMs for bf16 weights: gate_up writes bf16 h [S, I], down bf16(z) pair rows
// (the combine applies the routing weight).
int moe_launch_grouped_gemms_prefill_bf16(const uint16_t* x, const uint16_t* w13, const uint16_t* w2,
                                          const int32_t* perm, const int32_t* tiles, const int32_t* n_tiles,
                                          int max_tiles, uint16_t* h, uint16_t* pairs, int H, int I, int k,
                                          hipStream_t s) {
  if (!moe_prefill_bf16_ok(H, I, (long)max_tiles * PBM)) return MOE_ERR_INVALID_ARG;
  PrefillArgs g1{(const uint8_t*)x, nullptr, (const uint8_t*)w13, nullptr, perm, tiles, n_tiles, nullptr, nullptr,
                 nullptr, nullptr, h, H, I, k, I / PBK};
  int rc = launch_prefill<PF_GATE_UP, true>(g1, max_tiles, s);
  if (rc) return rc;
  PrefillArgs g2{(const uint8_t*)h, nullptr, (const uint8_t*)w2, nullptr, perm, tiles, n_tiles, nullptr, pairs,
                 nullptr, nullptr, nullptr, I, H, k, H / PBN};
  return launch_prefill<PF_DOWN, true>(g2, max_tiles, s);
}
