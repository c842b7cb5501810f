// Shared device helpers for the gfx950 MoE kernels: bf16 / e4m3 conversions,
// wave64 reductions and the MFMA operand types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_mi355x.h"

#define MOE_WAVE 64
#define MOE_GROUP 128      // quantisation group / block size
#define MOE_FP8_MAX 448.0f

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// bf16 <-> fp32 (bit patterns carried as uint16)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// Round to nearest even (gfx950 v_cvt_pk_bf16_f32); NaN stays NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const __bf16 b = (__bf16)f;
  return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ float round_bf16(float f) { return (float)(__bf16)f; }

// ---------------------------------------------------------------------------
// Exact e4m3 dot products.  v_mfma_scale_f32_16x16x128_f8f6f4 aligns its 128 products to
// the largest one and truncates the rest (about 2^-15 of the largest product is lost per
// MFMA, always toward zero), so over a 4096-deep reduction the fp32 result drifts ~2^-14
// of its value from the exact sum.  Widening the codes to bf16 (every e4m3 value is a bf16
// value) and using v_mfma_f32_16x16x32_bf16, whose 8-bit x 8-bit products and their sum
// are exact before the one fp32 rounding, gives the dequantise-then-fp32 result to fp32
// rounding.  Each lane's 32-byte fragment (row l % 16, K bytes [32 (l / 16), +32)) feeds
// four bf16 MFMAs, MFMA j taking bytes [8 j, 8 j + 8): the same K permutation for both
// operands, and the same 16x16 result layout as the f8f6f4 MFMA.
// ---------------------------------------------------------------------------
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// 8 e4m3 codes (two dwords) -> 8 bf16 values, exactly (v_cvt_scalef32_pk_bf16_fp8, scale 1)
__device__ __forceinline__ v8bf e4m3x8_to_bf16(uint32_t lo, uint32_t hi) {
  const v2bf a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
  const v2bf b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
  const v2bf c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
  const v2bf d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
  return (v8bf){a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// The 16x16 block of sum_k a[k] b[k] over one 128-deep K block of e4m3 codes, exact up to fp32
// rounding (a is the MFMA's A operand: rows of the result).  Both operands are widened just
// before each MFMA: the code dwords pass through an empty volatile asm after the previous MFMA,
// so the compiler cannot hoist the conversions of all four MFMAs ahead of the first (8 live
// registers for the widened operands instead of 32; the kernels run at their register bounds).
__device__ __forceinline__ v4f mfma_e4m3_exact(const v8i& a, const v8i& b) {
  v4f t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t a0 = (uint32_t)a[2 * j], a1 = (uint32_t)a[2 * j + 1];
    uint32_t b0 = (uint32_t)b[2 * j], b1 = (uint32_t)b[2 * j + 1];
    asm volatile("" : "+v"(a0), "+v"(a1), "+v"(b0), "+v"(b1));
    t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(e4m3x8_to_bf16(a0, a1), e4m3x8_to_bf16(b0, b1), t, 0, 0, 0);
    asm volatile("" : "+v"(t));
  }
  return t;
}

// Whether the expert GEMMs of a layer with hidden size H accumulate exactly.  With the
// f8f6f4 MFMA's truncation the gate_up result of a 4096-deep reduction moves by ~2^-14 of its
// value, enough to move bf16 h across an e4m3 rounding boundary of its re-quantisation for
// ~0.2% of the intermediate codes; under a heavy routing weight one moved code shifts an
// output of the Qwen3-235B-A22B layer (outputs up to ~2.9) by up to 3 bf16 ulps (2.3e-2).  At
// H = 2048 (Qwen3-30B-A3B) the drift is half as large and outputs stay well within 2e-2, so the
// f8f6f4 MFMA (twice the bf16 rate) is kept there.
__host__ __device__ inline bool moe_exact_accum(int H) { return H > 2048; }

// silu(gate) * up on bf16 values, in the reference's rounding order: the grouped GEMM
// output is bf16, silu(gate) is rounded to bf16, the product is rounded again
// (TF/integrations/moe.py:509-520).  silu(g) = g / (1 + exp(-g)) with exp from v_exp_f32 (a few
// ulps for the bf16 g of a layer) and the corrected quotient div_rn: silu(g) in fp32 is within a
// few ulps of the reference's, and its bf16 rounding differs only where that value sits that close
// to a bf16 rounding boundary.  The library expf was measured as well: ~30 more instructions per h
// element (the 4096-token prefill gate_up 170 -> 198 us) for no measurable change in the e4m3
// codes of h.
__device__ __forceinline__ float div_rn(float a, float b);
__device__ __forceinline__ float silu_mul_bf16(float gate_acc, float up_acc) {
  const float g = round_bf16(gate_acc);
  const float u = round_bf16(up_acc);
  const float e = __builtin_amdgcn_exp2f(-g * 1.4426950408889634f);
  const float sg = round_bf16(div_rn(g, 1.0f + e));
  return round_bf16(sg * u);
}

// a / b for finite b != 0 away from the fp32 range limits (callers: |a| <= 2^64, b a group scale
// or 1 + exp(-g) for a bf16 g): the v_rcp_f32 quotient with one residual correction.  The fma
// residual a - q b is exact, so the corrected quotient is the correctly rounded one in all but
// rare cases, and an exactly representable quotient (an e4m3 midpoint, say) always comes out
// exact; the IEEE division sequence costs about three times as many instructions, which showed in
// the prefill GEMM's epilogue (gate_up at 4096 tokens 170 -> 209 us).
__device__ __forceinline__ float div_rn(float a, float b) {
  const float r = __builtin_amdgcn_rcpf(b);
  const float q = a * r;
  const float e = fmaf(-q, b, a);
  return fmaf(e, r, q);
}

// ---------------------------------------------------------------------------
// fp32 -> OCP e4m3fn.  Inputs are clamped to [-448, 448] by the callers, so the
// conversion only has to round (to nearest even, the hardware default mode).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pack4_e4m3(float a, float b, float c, float d) {
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  int both = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
  return (uint32_t)both;
}

__device__ __forceinline__ float clamp_fp8(float v) {
  return __builtin_amdgcn_fmed3f(v, -MOE_FP8_MAX, MOE_FP8_MAX);
}

// ---------------------------------------------------------------------------
// Wave64 reductions (butterfly over all 64 lanes; every lane gets the result)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, MOE_WAVE));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, MOE_WAVE);
  return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    uint32_t o = (uint32_t)__shfl_xor((int)v, m, MOE_WAVE);
    v = o > v ? o : v;
  }
  return v;
}

// Wave-uniform reductions on the VALU only: DPP row rotations reduce each 16-lane row
// (every lane ends with its row's result), v_readlane combines the four rows.  No LDS
// crossbar traffic, unlike ds_bpermute-based shuffles.
template <int N>
__device__ __forceinline__ uint32_t row_ror(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x120 + N, 0xf, 0xf, false);
}

__device__ __forceinline__ uint32_t wave_max_u32_uniform(uint32_t v) {
  uint32_t o;
  o = row_ror<1>(v); v = o > v ? o : v;
  o = row_ror<2>(v); v = o > v ? o : v;
  o = row_ror<4>(v); v = o > v ? o : v;
  o = row_ror<8>(v); v = o > v ? o : v;
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
  const uint32_t a = r0 > r1 ? r0 : r1, b = r2 > r3 ? r2 : r3;
  return a > b ? a : b;
}

__device__ __forceinline__ float wave_max_uniform(float v) {
  v = fmaxf(v, __uint_as_float(row_ror<1>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(row_ror<2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(row_ror<4>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(row_ror<8>(__float_as_uint(v))));
  return fmaxf(fmaxf(__uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0)),
                     __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16))),
               fmaxf(__uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 32)),
                     __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 48))));
}

__device__ __forceinline__ float wave_sum_uniform(float v) {
  v += __uint_as_float(row_ror<1>(__float_as_uint(v)));
  v += __uint_as_float(row_ror<2>(__float_as_uint(v)));
  v += __uint_as_float(row_ror<4>(__float_as_uint(v)));
  v += __uint_as_float(row_ror<8>(__float_as_uint(v)));
  return (__uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 0)) +
          __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 16))) +
         (__uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 32)) +
          __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), 48)));
}

// max over aligned groups of `width` lanes (width a power of two <= 64)
template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int m = WIDTH / 2; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, MOE_WAVE));
  return v;
}

// Dynamic e4m3 quantisation of one 128-value group held by 16 adjacent lanes x 8 bf16
// values (the 16 bytes `raw`): s = amax/448 (1 if amax == 0), q = e4m3(clamp(x / s)).
// Writes 8 codes per lane and, from lane sub == 0, the group scale.
__device__ __forceinline__ void quant_group16_raw(uint4 raw, uint8_t* dst, float* sdst, int sub) {
  float v[8];
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = group_max<16>(amax);
  const float s = amax > 0.f ? amax / MOE_FP8_MAX : 1.0f;
  uint2 out;  // correctly rounded x / s, as the oracle
  out.x = pack4_e4m3(clamp_fp8(v[0] / s), clamp_fp8(v[1] / s), clamp_fp8(v[2] / s), clamp_fp8(v[3] / s));
  out.y = pack4_e4m3(clamp_fp8(v[4] / s), clamp_fp8(v[5] / s), clamp_fp8(v[6] / s), clamp_fp8(v[7] / s));
  *(uint2*)dst = out;
  if (sub == 0) *sdst = s;
}

__device__ __forceinline__ void quant_group16(const uint16_t* src, uint8_t* dst, float* sdst, int sub) {
  quant_group16_raw(*(const uint4*)src, dst, sdst, sub);
}

// ---------------------------------------------------------------------------
// Hand-off between the workgroups of one launch ("the last workgroup finishes"): data that
// another workgroup will read is stored and loaded as device-scope relaxed atomics, which on
// gfx950 are the sc1 forms of the stores and loads (coherent across the XCDs' L2 caches); a
// workgroup waits for its stores to complete, then counts in with a device-scope atomic add,
// and the workgroup whose add completes the count reads the data.  No L2 writeback or
// invalidate is needed, unlike a device-scope release / acquire fence (measured: a fence in
// every workgroup costs 6-60 us per launch at 96-1024 workgroups; this hand-off under 1 us).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void xwg_store32(void* p, uint32_t v) {
  __hip_atomic_store((uint32_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void xwg_store64(void* p, uint64_t v) {
  __hip_atomic_store((uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t xwg_load64(const void* p) {
  return __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint4 xwg_load128(const void* p) {
  const uint64_t a = xwg_load64(p), b = xwg_load64((const char*)p + 8);
  return make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
}
// Every memory operation this wave issued has completed (its xwg stores are visible).
__device__ __forceinline__ void xwg_wait_stores() { __builtin_amdgcn_s_waitcnt(0); }
// Count in; returns the counter's value before this add.
__device__ __forceinline__ int xwg_count_in(int32_t* cnt, int n = 1) {
  return __hip_atomic_fetch_add(cnt, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t lanemask_lt() {
  const int lane = __lane_id();
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// The token combine of a down-GEMM workgroup on the hand-off path, run by its last result wave
// once the workgroup's pair rows (columns [bx CB, (bx + 1) CB) of its tile's rows, whose pairs
// are rowpair[0 .. rows)) are stored device-scope: one tile row (pair) per lane counts in for its token's column block in tok_cnt
// [T, nbx] (zero on entry); the lanes whose count completes the token's k slots list their
// tokens (s_tok, one int per lane), and the wave sums each listed token's k pair rows over the
// block's columns: fp32 in slot order, + residual (bf16, when non-null) after one bf16 rounding,
// one bf16 rounding into comb [T, N] (combine_kernel's arithmetic).
template <int CB>
__device__ __forceinline__ void handoff_combine(const int32_t* rowpair, int topk, int rows, int32_t* tok_cnt,
                                                int nbx, int bx, const uint16_t* pairs, int N,
                                                const uint16_t* residual, uint16_t* comb, int* s_tok) {
  const int lane = threadIdx.x & 63;
  bool done = false;
  int t = 0;
  if (lane < rows) {
    t = rowpair[lane] / topk;
    done = xwg_count_in(tok_cnt + (long)t * nbx + bx) == topk - 1;
  }
  const uint64_t mask = __ballot(done);
  if (done) s_tok[__popcll(mask & lanemask_lt())] = t;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const int ntok = __popcll(mask);
  constexpr int PER_TOK = CB / 8;
  for (int u = lane; u < ntok * PER_TOK; u += MOE_WAVE) {
    const int tt = s_tok[u / PER_TOK];
    const int c0 = bx * CB + (u % PER_TOK) * 8;
    float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < topk; j0 += 8) {
      uint4 rv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) rv[j] = xwg_load128(pairs + (long)(tt * topk + min(j0 + j, topk - 1)) * N + c0);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j0 + j >= topk) break;
        const uint32_t w4[4] = {rv[j].x, rv[j].y, rv[j].z, rv[j].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sum[2 * i] += __uint_as_float(w4[i] << 16);
          sum[2 * i + 1] += __uint_as_float(w4[i] & 0xffff0000u);
        }
      }
    }
    if (residual != nullptr) {
      const uint4 r4 = *(const uint4*)(residual + (long)tt * N + c0);
      const uint32_t ru[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sum[2 * i] = __uint_as_float(ru[i] << 16) + round_bf16(sum[2 * i]);
        sum[2 * i + 1] = __uint_as_float(ru[i] & 0xffff0000u) + round_bf16(sum[2 * i + 1]);
      }
    }
    uint4 o4;
    o4.x = (uint32_t)f32_to_bf16(sum[0]) | ((uint32_t)f32_to_bf16(sum[1]) << 16);
    o4.y = (uint32_t)f32_to_bf16(sum[2]) | ((uint32_t)f32_to_bf16(sum[3]) << 16);
    o4.z = (uint32_t)f32_to_bf16(sum[4]) | ((uint32_t)f32_to_bf16(sum[5]) << 16);
    o4.w = (uint32_t)f32_to_bf16(sum[6]) | ((uint32_t)f32_to_bf16(sum[7]) << 16);
    *(uint4*)(comb + (long)tt * N + c0) = o4;
  }
}

// Read an expert id stored as int32 or int64.
__device__ __forceinline__ int load_id(const void* ids, int id_bytes, int i) {
  return id_bytes == 8 ? (int)((const int64_t*)ids)[i] : ((const int32_t*)ids)[i];
}

// ---------------------------------------------------------------------------
// Host-side helpers shared by the entry points
// ---------------------------------------------------------------------------
static inline size_t moe_align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

static inline bool moe_aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
// a 1-D grid of n workgroups fits the launch (gridDim.x is 32-bit; kernels index workgroups as int)
static inline bool moe_grid_fits(long n) { return n >= 0 && n < (1L << 31); }

#define MOE_CHECK_LAUNCH()                          \
  do {                                              \
    hipError_t _e = hipGetLastError();              \
    if (_e != hipSuccess) return (int)_e;           \
  } while (0)

#define MOE_RETURN_IF(cond, code) \
  do {                            \
    if (cond) return (code);      \
  } while (0)

// Workspace carving: successive 256-byte aligned slices of one caller buffer.
struct WsCarver {
  char* base;
  size_t off;
  __host__ explicit WsCarver(void* b) : base((char*)b), off(0) {}
  template <typename T>
  __host__ T* take(size_t count) {
    off = moe_align_up(off, 256);
    T* p = base ? (T*)(base + off) : nullptr;
    off += count * sizeof(T);
    return p;
  }
};

// Kernel slots of the event-timing facility (prof.hip).
enum {
  MOE_PROF_ROUTER_GEMM = 0,
  MOE_PROF_TOPK = 1,
  MOE_PROF_QUANT_ACT = 2,
  MOE_PROF_ALIGN = 3,
  MOE_PROF_GATE_UP = 4,
  MOE_PROF_QUANT_H = 5,
  MOE_PROF_DOWN = 6,
  MOE_PROF_COMBINE = 7,
  MOE_PROF_LINEAR = 8,
  MOE_PROF_SLOTS = 9
};
int moe_prof_begin(int slot, hipStream_t s);
void moe_prof_end(int id, hipStream_t s);

// hipLaunchKernelGGL bracketed by the timing events of `slot` (no-op unless enabled).
#define MOE_LAUNCH(slot, stream, ...)                  \
  do {                                                \
    const int _pid = moe_prof_begin((slot), (stream)); \
    hipLaunchKernelGGL(__VA_ARGS__);                  \
    moe_prof_end(_pid, (stream));                     \
  } while (0)

// Internal launchers shared between translation units.
int moe_launch_quant_act(const void* x, int R, int C, void* q, float* scales, hipStream_t s,
                         int slot = MOE_PROF_QUANT_ACT);
int moe_launch_align(const void* ids, int id_bytes, int S, int E, int block_m, int32_t* perm,
                     int32_t* counts, int32_t* offsets, int32_t* tiles, int32_t* n_tiles,
                     void* workspace, size_t workspace_bytes, hipStream_t s, int32_t* zero = nullptr,
                     int nzero = 0);
