// LDS staging helpers of the LDS-tiled grouped GEMM (gemm_fp8_prefill.hip): the swizzled 128-byte LDS row layout, MFMA fragment reads,
// global -> LDS DMA, wait / barrier and scalar table loads.
#pragma once

#include "common.h"

namespace moe_lds {

// LDS rows are 128 bytes (eight 16-byte chunks).  Chunk c of row r is stored at position
// c ^ swz_key(r), swz_key(r) = (r ^ ((r >> 3) & 1)) & 7: a ds_read_b128 of an MFMA fragment
// (16 consecutive rows from a multiple of 16, one chunk column per 16 lanes) then runs
// without bank conflicts on gfx950 (4 LDS cycles per instruction, measured with
// SQ_LDS_BANK_CONFLICT; XOR with r & 7 or (r >> 1) & 7 alone costs 8).  The key depends on
// r & 15 only, so a lane's address within any 16-row group is the same.
__device__ __forceinline__ int swz_key(int row) { return (row ^ ((row >> 3) & 1)) & 7; }
__device__ __forceinline__ int swz(int row, int chunk) { return row * 128 + ((chunk ^ swz_key(row)) << 4); }

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

// Global -> LDS DMA (gfx950 global_load_lds_dwordx4 / _dword), address = SGPR base +
// per-lane 32-bit offset: lane i of the wave writes LDS [m0 + 16 i] (resp. [m0 + 4 i]), with
// m0 = m0base + OFF.  Issued from inline asm so the compiler does not wait on these loads
// itself; the kernel waits on vmcnt explicitly.  M0 is written with s_mov_b32 from an SGPR the
// compiler computed: an s_add inside the asm would write SCC behind the compiler's back (SCC
// cannot be declared clobbered), and the compiler does keep SCC live across these statements
// (an s_cmp before the asm feeding an s_cbranch_scc after it), which then branched on the
// add's carry.
template <int OFF>
__device__ __forceinline__ void dma_b128(uint32_t voff, const void* sbase, uint32_t m0base) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(m0base + OFF);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(sbase), "s"(m0v) : "memory", "m0");
}
template <int OFF>
__device__ __forceinline__ void dma_b32(uint32_t voff, const void* sbase, uint32_t m0base) {
  const uint32_t m0v = __builtin_amdgcn_readfirstlane(m0base + OFF);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(voff), "s"(sbase), "s"(m0v) : "memory", "m0");
}

// Wait until at most VM of this wave's vector loads are outstanding (inline asm: the
// compiler does not track the DMA loads) and every LDS access has completed, then
// barrier.  The LDS wait is the s_waitcnt builtin (vmcnt 63 = no wait, expcnt 7 = no wait,
// lgkmcnt 0), issued unconditionally, so the compiler's own wait-count tracking sees that
// every earlier LDS read is complete on every path.  Loads complete in order.
constexpr int kWaitLgkm0 = 0xF | (3 << 14) | (7 << 4);
template <int VM>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(VM) : "memory");
}
__device__ __forceinline__ void lds_wait_barrier() {
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Constant-address-space views: uniform loads through them become scalar (SMEM) loads,
// which are tracked by lgkmcnt and never wait behind the in-flight DMA loads (vmcnt).
#define CONST_AS __attribute__((address_space(4)))
__device__ __forceinline__ int const_ld(const int32_t* p, long i) { return ((const CONST_AS int32_t*)p)[i]; }
__device__ __forceinline__ int4 const_ld4(const int32_t* p, long i) {
  const CONST_AS int32_t* q = (const CONST_AS int32_t*)p + 4 * i;
  return make_int4(q[0], q[1], q[2], q[3]);
}

}  // namespace moe_lds
