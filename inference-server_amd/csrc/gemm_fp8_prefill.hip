// Grouped FP8 GEMMs for prefill chunks (many rows per expert): LDS-tiled, persistent,
// XCD-aware, MFMA-bound.
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
// Workgroup: 8 waves (2 per SIMD) in a 2x4 grid; a wave owns 64 rows x 64 weight rows
// = 4 x 4 v_mfma_f32_16x16x128_f8f6f4 tiles per K block, each folded into the fp32
// accumulator with the (activation row scale x weight tile scale) product.  Two waves
// per SIMD let one wave's scale FMAs and LDS reads run under the other's MFMAs.
//
// Operands are staged through a ring of three 48.5 KB LDS stages (A 16 KB + B 32 KB +
// 512 B of activation scales) filled by global->LDS DMA without touching VGPRs: K block
// kb+2 is in flight while kb is computed, so a load has two compute phases to land; one
// barrier per K block.  LDS rows are 128 bytes;
// 16-byte chunk c of row r is stored at chunk c ^ (r & 7), so the 8 lanes that share a
// LDS cycle in a ds_read_b128 of an MFMA fragment hit 8 different bank groups.
//
// Persistent grid: one workgroup per CU (the LDS footprint allows one).  Work items
// (tile, column block) are handed out so that the workgroups resident on one XCD
// (hardware places workgroup w on XCD w % 8) take consecutive items: they share the
// expert's weights and the tile's activations in that XCD's L2.
#include "common.h"

namespace {

enum { PF_GATE_UP = 0, PF_DOWN = 1 };

constexpr int PBM = 128;             // rows per tile
constexpr int PBN = 256;             // weight rows per tile
constexpr int PBK = 128;             // K block (one scale block)
constexpr int P_A = PBM * PBK;       // 16 KB
constexpr int P_B = PBN * PBK;       // 32 KB
constexpr int P_STAGE = P_A + P_B;   // 48 KB
constexpr int kMaxKB = 32;           // K <= 4096

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
  int K;                   // reduction length
  int N;                   // gate_up: I; down: H
  int topk;
  int n_nblk;              // column blocks per tile: gate_up I/128, down H/256
};

// LDS rows are 128 bytes = 32 of the 64 four-byte banks, so an MFMA fragment read (16
// lanes on 16 consecutive rows, one 16-byte chunk each) covers all 64 banks only if the 8
// even rows and the 8 odd rows each use 8 different chunk positions: chunk c of row r is
// stored at position c ^ ((r >> 1) & 7).
__device__ __forceinline__ int swz(int row, int chunk) { return row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4); }

__device__ __forceinline__ v8i lds_frag(const uint8_t* base, int row, int c0) {
  const uint4 lo = *(const uint4*)(base + swz(row, c0));
  const uint4 hi = *(const uint4*)(base + swz(row, c0 + 1));
  v8i r;
  r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w;
  r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
  return r;
}

#define LDS_AS __attribute__((address_space(3)))

__device__ __forceinline__ uint32_t lds_u32(const void* p) { return (uint32_t)(uintptr_t)((LDS_AS const void*)p); }

// Global -> LDS DMA (gfx950 global_load_lds_dwordx4 / _dword): lane i of the wave writes
// LDS [m0 + 16 i] (resp. [m0 + 4 i]).  Issued from inline asm so the compiler's
// wait-count pass does not serialise every LDS read behind it; the kernel waits on
// vmcnt itself.  M0 is saved and restored around the load.
__device__ __forceinline__ void dma_b128(const void* g, uint32_t lds) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(g), "s"(lds) : "memory");
}
__device__ __forceinline__ void dma_b32(const void* g, uint32_t lds) {
  uint32_t saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved) : "v"(g), "s"(lds) : "memory");
}

constexpr int P_SA = PBM * 4;                 // 512 B of activation scales per stage
constexpr int P_STAGE3 = P_STAGE + P_SA;      // 49664 B
constexpr int P_DMA_PER_STEP = 7;             // per wave: 2 A + 4 B + 1 scale loads per K block

// Wait until at most N of this wave's vector loads are outstanding and every LDS access
// has completed, then barrier.  Loads complete in order, so N = loads issued for the
// next-but-one K block leaves exactly those in flight.
template <int N>
__device__ __forceinline__ void wait_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

template <int MODE>
__global__ __launch_bounds__(512, 1) void grouped_gemm_fp8_prefill_kernel(PrefillArgs p) {
  __shared__ __attribute__((aligned(16))) uint8_t s_ab[3][P_STAGE3];
  __shared__ int s_arow[PBM];
  __shared__ int s_pair[PBM];
  __shared__ float s_wt[PBM];
  __shared__ float s_amax[4][PBM];
  __shared__ float s_sw[3][kMaxKB];  // weight tile scales of the item: gate / up (or the two down blocks)

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: keep it in an SGPR
  const int wm = wave & 1, wn = wave >> 1;  // 2 x 4 waves: rows wm*64, column quarter wn
  const int lr = lane & 15, lg = lane >> 4;
  const int c0 = 2 * lg;
  const int K = p.K, KB = K / PBK;
  const int Nw = MODE == PF_GATE_UP ? 2 * p.N : p.N;
  const int n_items = p.n_tiles[0] * p.n_nblk;
  const int G = gridDim.x;  // a multiple of 8
  const int my_slot = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
  const uint32_t lds_stage0 = __builtin_amdgcn_readfirstlane(lds_u32(&s_ab[0][0]));

  // DMA lane assignment: one instruction fills 8 rows x 128 B (block j = rows 8j..8j+7).
  // Lane L writes position L & 7 of row 8j + (L >> 3), which holds logical chunk
  // (L & 7) ^ ((row >> 1) & 7); every block this wave fills has j = wave (mod 2).
  const int dma_r = lane >> 3;
  const int dma_lc = (lane & 7) ^ ((4 * (wave & 1) + (dma_r >> 1)) & 7);

  // B row of fragment ni of this wave (within the 256-row B tile)
#define PF_BROW(ni) \
  ((MODE == PF_GATE_UP ? ((ni) < 2 ? wn * 32 + (ni) * 16 : 128 + wn * 32 + ((ni) - 2) * 16) : wn * 64 + (ni) * 16) + lr)

  for (int base = 0;; base += G) {
    const int item = base + my_slot;
    if (item >= n_items) break;  // workgroup-uniform
    const int tile = item / p.n_nblk, nb = item - tile * p.n_nblk;
    const int4 ti = *(const int4*)(p.tiles + 4 * tile);
    const int e = ti.x, row0 = ti.y, rows = ti.z;

    __syncthreads();  // the previous item's epilogue is done with the row tables
    if (tid < PBM) {
      const int rr = row0 + min(tid, rows - 1);  // rows past the tile end repeat the last row
      if constexpr (MODE == PF_GATE_UP) {
        s_arow[tid] = p.perm[rr] / p.topk;
      } else {
        s_arow[tid] = rr;
        const int pr = p.perm[rr];
        s_pair[tid] = pr;
        s_wt[tid] = bf16_to_f32(p.topk_w[pr]);
      }
    } else if (tid < PBM + 2 * kMaxKB) {
      // weight tile scales for every K block: gate_up -> gate block nb and up block I/128 + nb;
      // down -> blocks 2 nb and 2 nb + 1 (the two 128-row halves of the 256 columns)
      const int j = tid - PBM, which = j / kMaxKB, kb = j % kMaxKB;
      const int nblk128 = Nw / PBK;
      const int blk = MODE == PF_GATE_UP ? (which == 0 ? nb : p.N / PBK + nb) : 2 * nb + which;
      if (kb < KB) s_sw[which][kb] = p.sw[((long)e * nblk128 + blk) * KB + kb];
    }
    __syncthreads();

    // per-lane source rows of this wave's DMA instructions (A: blocks wave, wave+8;
    // B: blocks wave + 8 i; scales: rows 16 wave + lane for lane < 16)
    const uint8_t* a_src0 = p.a + (long)s_arow[8 * wave + dma_r] * K + dma_lc * 16;
    const uint8_t* a_src1 = p.a + (long)s_arow[8 * (wave + 8) + dma_r] * K + dma_lc * 16;
    const uint8_t* b_src[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int br = 8 * (wave + 8 * i) + dma_r;
      long wrow;
      if constexpr (MODE == PF_GATE_UP)
        wrow = br < 128 ? nb * 128 + br : p.N + nb * 128 + (br - 128);
      else
        wrow = (long)nb * 256 + br;
      b_src[i] = p.w + ((long)e * Nw + wrow) * K + dma_lc * 16;
    }
    const float* sa_src = p.sa + (long)s_arow[16 * wave + (lane & 15)] * KB;

    // this wave's weight scale rows in s_sw: gate_up (gate, up); down (its 128-column half)
    const float* sw0 = MODE == PF_GATE_UP ? s_sw[0] : s_sw[wn >> 1];
    const float* sw1 = MODE == PF_GATE_UP ? s_sw[1] : s_sw[wn >> 1];

#define PF_ISSUE(kb_)                                                                          \
  do {                                                                                         \
    const int st_ = (kb_) % 3;                                                                 \
    const uint32_t sb = lds_stage0 + st_ * P_STAGE3;                                           \
    const long ko = (long)(kb_) * PBK;                                                         \
    dma_b128(a_src0 + ko, sb + 1024 * wave);                                                   \
    dma_b128(a_src1 + ko, sb + 1024 * (wave + 8));                                             \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) dma_b128(b_src[i] + ko, sb + P_A + 1024 * (wave + 8 * i)); \
    if (lane < 16) dma_b32(sa_src + (kb_), sb + P_STAGE + 64 * wave);                          \
  } while (0)

    v4f acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = (v4f){0.f, 0.f, 0.f, 0.f};

    PF_ISSUE(0);
    if (KB > 1) {
      PF_ISSUE(1);
      wait_barrier<P_DMA_PER_STEP>();
    } else {
      wait_barrier<0>();
    }
    for (int kb = 0; kb < KB; ++kb) {
      const bool issue = kb + 2 < KB;
      if (issue) PF_ISSUE(kb + 2);
      const uint8_t* sA = s_ab[kb % 3];
      const uint8_t* sB = sA + P_A;
      const float* sSa = (const float*)(sA + P_STAGE);
      v8i a[4], b[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) a[mi] = lds_frag(sA, wm * 64 + mi * 16 + lr, c0);
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) b[ni] = lds_frag(sB, PF_BROW(ni), c0);
      float4 sv[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) sv[mi] = *(const float4*)&sSa[wm * 64 + mi * 16 + 4 * lg];
      const float sw_a = sw0[kb], sw_b = sw1[kb];
      // combined (activation row x weight tile) scale of every accumulator row, per B half
      float sca[4][4], scb[4][4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        const float s4[4] = {sv[mi].x, sv[mi].y, sv[mi].z, sv[mi].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          sca[mi][q] = s4[q] * sw_a;
          scb[mi][q] = MODE == PF_GATE_UP ? s4[q] * sw_b : sca[mi][q];
        }
      }
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
          const v4f zero = {0.f, 0.f, 0.f, 0.f};
          const v4f t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[mi], b[ni], zero, 0, 0, 0, 0, 0, 0);
#pragma unroll
          for (int q = 0; q < 4; ++q)
            acc[mi][ni][q] = fmaf(t[q], (MODE == PF_GATE_UP && ni >= 2) ? scb[mi][q] : sca[mi][q], acc[mi][ni][q]);
        }
      }
      if (issue)
        wait_barrier<P_DMA_PER_STEP>();
      else
        wait_barrier<0>();
    }
#undef PF_ISSUE

    if constexpr (MODE == PF_GATE_UP) {
      // h = bf16(bf16(silu(bf16 g)) * bf16 u) in acc[..][0..1]; gate frags 0,1 pair with up frags 2,3
      float rmax[4][4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float m = 0.f;
#pragma unroll
          for (int ni = 0; ni < 2; ++ni) {
            const float h = silu_mul_bf16(acc[mi][ni][q], acc[mi][ni + 2][q]);
            acc[mi][ni][q] = h;
            m = fmaxf(m, fabsf(h));
          }
          rmax[mi][q] = group_max<16>(m);  // the 16 lanes sharing these rows
        }
      if (lr == 0) {
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
          for (int q = 0; q < 4; ++q) s_amax[wn][wm * 64 + mi * 16 + 4 * lg + q] = rmax[mi][q];
      }
      __syncthreads();
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = wm * 64 + mi * 16 + 4 * lg + q;
          const float amax = fmaxf(fmaxf(s_amax[0][r], s_amax[1][r]), fmaxf(s_amax[2][r], s_amax[3][r]));
          const float s = amax > 0.f ? amax / MOE_FP8_MAX : 1.0f;
          if (r < rows) {
            const long srow = row0 + r;
            uint8_t* dst = p.hq + srow * p.N + nb * 128 + wn * 32 + lr;
            // h * (1/s) with a correctly rounded 1/s: within one fp32 ulp of h / s
            const float inv_s = 1.0f / s;
            const int code = __builtin_amdgcn_cvt_pk_fp8_f32(clamp_fp8(acc[mi][0][q] * inv_s),
                                                             clamp_fp8(acc[mi][1][q] * inv_s), 0, false);
            dst[0] = (uint8_t)(code & 0xff);
            dst[16] = (uint8_t)((code >> 8) & 0xff);
            if (wn == 0 && lr == 0) p.sh[srow * (p.N / PBK) + nb] = s;
          }
        }
    } else {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int r = wm * 64 + mi * 16 + 4 * lg + q;
          if (r >= rows) continue;
          const long pr = s_pair[r];
          const float wt = s_wt[r];
          uint16_t* dst = p.pairs + pr * p.N + nb * 256 + wn * 64 + lr;
#pragma unroll
          for (int ni = 0; ni < 4; ++ni) dst[ni * 16] = f32_to_bf16(round_bf16(acc[mi][ni][q]) * wt);
        }
    }
  }
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

template <int MODE>
int launch_prefill(const PrefillArgs& a, int max_tiles, hipStream_t s) {
  const long max_items = (long)max_tiles * a.n_nblk;
  long g = device_cu_count();
  if (g > max_items) g = max_items;
  g = (g + 7) / 8 * 8;
  if (g < 8) g = 8;
  MOE_LAUNCH(MODE == PF_GATE_UP ? MOE_PROF_GATE_UP : MOE_PROF_DOWN, s, grouped_gemm_fp8_prefill_kernel<MODE>,
             dim3((unsigned)g), dim3(512), 0, s, a);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}

}  // namespace

// gate_up (with fused SiLU*up and e4m3 re-quantisation of h) then down, for block_m = 128 tiles.
int moe_launch_grouped_gemms_prefill(const uint8_t* xq, const float* sx, const uint8_t* w13, const float* s13,
                                     const uint8_t* w2, const float* s2, const int32_t* perm, const int32_t* tiles,
                                     const int32_t* n_tiles, int max_tiles, const uint16_t* topk_w, uint8_t* hq,
                                     float* sh, uint16_t* pairs, int H, int I, int k, hipStream_t s) {
  PrefillArgs g1{xq, sx, w13, s13, perm, tiles, n_tiles, nullptr, nullptr, hq, sh, H, I, k, I / PBK};
  int rc = launch_prefill<PF_GATE_UP>(g1, max_tiles, s);
  if (rc) return rc;
  PrefillArgs g2{hq, sh, w2, s2, perm, tiles, n_tiles, topk_w, pairs, nullptr, nullptr, I, H, k, H / PBN};
  return launch_prefill<PF_DOWN>(g2, max_tiles, s);
}
