// Paged GQA decode attention (one new token per sequence) for the Qwen3-MoE decoder layer,
// bf16 in and out, fp32 softmax and accumulation.
//
// Reference: eager_attention_forward, TF/models/qwen3_moe/modeling_qwen3_moe.py:96-119, as
// called by Qwen3MoeAttention.forward (:151-191) for a decode step: scores
// bf16(bf16(q . k) * head_dim^-0.5), softmax in fp32 over the keys of the sequence, the
// probabilities applied to V, output bf16.  The grouped-query heads share a key/value head
// (repeat_kv, :84-93): query head h reads key/value head h / (Hq / Hkv).
//
// KV cache (this library's layout; the reference keeps a contiguous per-layer cache): pages
// of 16 tokens.  K pages are [page][kv head][token 16][dim 128] and V pages are stored
// transposed, [page][kv head][dim 128][token 16], so that both MFMA products below take
// their operands straight from HBM with 16- and 8-byte loads.
//
// One workgroup = (sequence b, kv head g, split of up to `pps` pages); its 4 waves take the
// split's pages round robin, each with its own online-softmax state, merged in LDS at the
// end.  The grid is one-dimensional: workgroup i takes the i-th (b, g, split) that holds
// pages, in sequence order, found from the context lengths by a block-wide prefix sum; the
// workgroups past the last one leave at once.  (A (split, head, sequence) grid whose empty
// splits exit interleaved with the working ones reads the KV cache about 25% slower:
// 4.5 against 5.8 TB/s in a loads-only model of this kernel, U[512, 8192] contexts.)  Per page a wave computes
//   S^T [16 keys x 16 heads] = K [16 x 128] . Q^T [128 x 16]       (4 x mfma 16x16x32 bf16)
//   O^T [128 x 16 heads]    += V^T [128 x 16 keys] . P^T [16 keys x 16 heads]
//                                                                   (8 x mfma 16x16x16 bf16)
// where the query heads of the group fill columns 0..G-1 (G <= 16) and the rest are zero.  The
// score tile's lane layout (lane l: keys 4 (l >> 4) + i of head l & 15) is exactly the B
// operand layout of the second product, so P needs no shuffle, and the output tile again
// holds head l & 15 in lane l: the online-softmax rescale of a head is applied in the lanes
// that hold its running max.  Splits are combined by
// paged_attn_merge_kernel (log-sum-exp weights).
#include "common.h"

namespace {

typedef short v4s __attribute__((ext_vector_type(4)));

// Buffer descriptor of one (page, kv head) block of K or V (4 KB; offsets past it read 0).
// Word 3 selects the 32-bit data format: untyped buffer loads on gfx9 read zeros when the
// format field is 0.
constexpr int kKvBlockBytes = 16 * 128 * 2;
constexpr int kCachePolicyNT = 2;  // the instruction's cache-policy field: nt (streaming)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t kv_rsrc(const uint16_t* block, bool live) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)block, (short)0, live ? kKvBlockBytes : 0, 0x00020000);
}

constexpr int kHD = 128;        // head dim
constexpr int kPage = 16;       // tokens per page
constexpr int kAttnWaves = 4;

__device__ __forceinline__ float bf16_round(float f) { return (float)(__bf16)f; }

// Reductions over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the 16-lane rows of a wave) with
// gfx950's row swaps: v_permlane16_swap exchanges rows 1 and 0, 3 and 2 between its two
// operands, v_permlane32_swap the two halves, so combining the pair it returns gives every
// lane op(own, partner) without an LDS permute.  The sums associate as (r0 + r1) + (r2 + r3)
// in every lane.
__device__ __forceinline__ float rows_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Pages of a context, clamped to the block table's width (context lengths are device data:
// a value past the table would read beyond it).  Negative lengths count as empty.
__device__ __forceinline__ int attn_pages(int ctx, int max_pages) {
  return ctx <= 0 ? 0 : min((ctx + kPage - 1) / kPage, max_pages);
}

#ifndef MOE_ATTN_PART_BANDS
#define MOE_ATTN_PART_BANDS 8
#endif
constexpr int kPartBands = MOE_ATTN_PART_BANDS;
// band of a partial split of r pages (0 < r < pps <= 64): 0 for the longest
__device__ __forceinline__ int attn_part_band(int r, int pps) { return (pps - 1 - r) * kPartBands / (pps - 1); }

struct AttnArgs {
  const uint16_t* q;           // [B, Hq, 128] bf16
  const uint16_t* k_cache;     // [pages, Hkv, 16, 128] bf16
  const uint16_t* v_cache;     // [pages, Hkv, 128, 16] bf16
  const int32_t* block_tables; // [B, max_pages]
  const int32_t* context_lens; // [B]
  float* part_o;               // [B, Hkv, max_splits, G, 128] unnormalised outputs
  float* part_ml;              // [B, Hkv, max_splits, G, 2] (running max, sum)
  int B, Hq, Hkv, max_pages, max_splits, pps;
  int num_pages;               // pages in each pool: table entries outside [0, num_pages) are empty
  float scale;
};

// four waves per SIMD (at most 128 registers): each wave has one page in flight, so occupancy
// is what keeps the HBM busy
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void paged_attn_decode_kernel(AttnArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: keeps page ids and descriptors scalar
  const int lr = lane & 15, lg = lane >> 4;
  const int G = a.Hq / a.Hkv;

  // workgroup -> (b, g, split).  Items in dispatch order: every head's full splits of pps pages
  // (sequence-major), then the partial last splits, longest first in kPartBands bands of their
  // page count, so that the launch drains on short items (the slots free up one by one at the
  // end, and with the partial splits spread through the order the last items dispatched were
  // mostly full ones).  Split numbering (page order) is unchanged, so the merge is too.  Found
  // in chunks of 256 sequences: a block-wide scan of the full-split items (wave scans, then
  // across the 4 waves through LDS), and per band a wave ballot of the sequences in it (each
  // adds Hkv items); where the batch spans several chunks, a first pass sums the totals.
  __shared__ int s_w0[kAttnWaves];
  __shared__ int s_cnt[kPartBands][kAttnWaves];  // sequences per band and wave, this chunk
  __shared__ int s_tot[kPartBands], s_carry[kPartBands];  // per band: this chunk, earlier chunks
  __shared__ int s_item[4];  // sequence, phase, index within it, context length
  if (threadIdx.x == 0) s_item[0] = -1;
  {
    const int item = blockIdx.x;
    int n0 = 0, incl0 = 0, before0 = 0, tot0 = 0, band = -1, rank = 0, cl = 0;
    // this thread's sequence: full-split items and band; the chunk's scan and band counts
    auto chunk = [&](int b0) __attribute__((always_inline)) {
      const int bb = b0 + (int)threadIdx.x;
      int full = 0;
      band = -1;
      if (bb < a.B) {
        cl = a.context_lens[bb];
        const int np = attn_pages(cl, a.max_pages);
        full = np / a.pps;
        const int r = np - full * a.pps;
        band = r > 0 ? attn_part_band(r, a.pps) : -1;
      }
      n0 = full * a.Hkv;
      incl0 = n0;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int t = __shfl_up(incl0, d);
        if (lane >= d) incl0 += t;
      }
      if (lane == 63) s_w0[wave] = incl0;
      const uint64_t below = (1ull << lane) - 1;
      for (int q = 0; q < kPartBands; ++q) {  // uniform loop
        const uint64_t m = __ballot(band == q);
        if (lane == 0) s_cnt[q][wave] = __popcll(m);
        if (band == q) rank = __popcll(m & below);
      }
      __syncthreads();
      before0 = 0;
      tot0 = 0;
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) {
        before0 += w < wave ? s_w0[w] : 0;
        tot0 += s_w0[w];
      }
      if (band >= 0)
        for (int w = 0; w < wave; ++w) rank += s_cnt[band][w];
      if (threadIdx.x < kPartBands) {
        int t = 0;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) t += s_cnt[threadIdx.x][w];
        s_tot[threadIdx.x] = t;
      }
      __syncthreads();
    };
    __shared__ int s_total[kPartBands];  // per band, the whole batch
    int n_full = 0;  // full-split items of the whole batch
    if (threadIdx.x < kPartBands) {
      s_total[threadIdx.x] = 0;
      s_carry[threadIdx.x] = 0;
    }
    if (a.B > 256) {  // workgroup-uniform
      for (int b0 = 0; b0 < a.B; b0 += 256) {
        chunk(b0);
        n_full += tot0;
        if (threadIdx.x < kPartBands) s_total[threadIdx.x] += s_tot[threadIdx.x];
      }
      __syncthreads();
    }
    int carry0 = 0;
    for (int b0 = 0; b0 < a.B; b0 += 256) {  // workgroup-uniform
      chunk(b0);
      if (a.B <= 256) {
        n_full = tot0;
        if (threadIdx.x < kPartBands) s_total[threadIdx.x] = s_tot[threadIdx.x];
        __syncthreads();
      }
      const int first = carry0 + before0 + incl0 - n0;
      if (n0 > 0 && item >= first && item < first + n0) {
        s_item[0] = b0 + (int)threadIdx.x;
        s_item[1] = 0;
        s_item[2] = item - first;
        s_item[3] = cl;
      }
      if (band >= 0) {
        int off = n_full;  // items of the longer bands
        for (int q = 0; q < band; ++q) off += s_total[q] * a.Hkv;
        const int f = off + (s_carry[band] + rank) * a.Hkv;
        if (item >= f && item < f + a.Hkv) {
          s_item[0] = b0 + (int)threadIdx.x;
          s_item[1] = 1;
          s_item[2] = item - f;
          s_item[3] = cl;
        }
      }
      carry0 += tot0;
      __syncthreads();  // every thread has read s_carry
      if (threadIdx.x < kPartBands) s_carry[threadIdx.x] += s_tot[threadIdx.x];
    }
    __syncthreads();  // s_item is final
  }
  const int b = s_item[0];
  if (b < 0) return;  // workgroup-uniform: past the last item
  const int ctx = min(s_item[3], kPage * a.max_pages);  // the scan's read: no second round trip
  const int n_pages = attn_pages(ctx, a.max_pages);
  const int n_full = n_pages / a.pps;
  const bool part = s_item[1] != 0;
  const int g = part ? s_item[2] : s_item[2] / n_full;
  const int split = part ? n_full : s_item[2] % n_full;
  const int p_begin = split * a.pps;
  const int p_end = min(n_pages, p_begin + a.pps);

  // Q^T operand (B of the score product): head lr of the group, dims 32 kk + 8 lg .. +8
  v8bf qop[4];
  {
    const bool live = lr < G;
    const uint16_t* qrow = a.q + ((long)b * a.Hq + g * G + (live ? lr : 0)) * kHD;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      uint4 v = live ? *(const uint4*)(qrow + 32 * kk + 8 * lg) : make_uint4(0, 0, 0, 0);
      qop[kk] = __builtin_bit_cast(v8bf, v);
    }
  }

  const int32_t* btab = a.block_tables + (long)b * a.max_pages;
  const long kv_head_stride = (long)kHD * kPage;  // elements per (page, kv head)

  float m_run = -INFINITY, l_run = 0.f;  // of head lr (identical in the 4 lanes lr + 16 j)
  v4f o[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) o[n] = (v4f){0.f, 0.f, 0.f, 0.f};

  // operands of one page: K rows (lane: key lr, dims 32 kk + 8 lg) and V^T (lane: keys
  // 4 lg .. +4 of dim 16 n + lr).  One register set each: the next page's K is loaded as soon
  // as the score MFMAs have read this page's, its V after the output MFMAs, so both stay in
  // flight through most of an iteration without a second buffer (occupancy over depth).
  uint4 kr[4];
  uint2 vr[8];
  // page ids of this wave's pages p_begin + wave + 4 i, one per lane, fetched up front so that
  // the K / V loads of a page do not wait on a dependent block-table load
  const int my_page = (p_begin + wave + kAttnWaves * lane < p_end) ? btab[p_begin + wave + kAttnWaves * lane] : 0;
  auto page_of = [&](int p) __attribute__((always_inline)) {
    return (long)__builtin_amdgcn_readlane(my_page, (p - p_begin - wave) / kAttnWaves);
  };
  // a table entry outside the pools (a -1 pad, a stale id) is an empty page: its descriptor
  // covers 0 bytes, so its loads read zeros and touch no memory, and its keys are masked
  auto page_ok = [&](long pg) __attribute__((always_inline)) { return pg >= 0 && pg < a.num_pages; };
  // K and V are read once per step: non-temporal loads (the nt bit) keep the stream from
  // displacing what the caches hold for reuse (5.24 -> 5.40 TB/s at the config-5 batch), issued
  // as buffer loads on a per-(page, kv head) descriptor (SGPR base, 32-bit lane offsets within
  // the 4 KB block: 215.9 -> 212.4 us against global loads)
  // live == false (no such page): a zero-size descriptor, so the loads read zeros and touch no
  // memory.  Loads are issued unconditionally this way because a branch around them makes the
  // compiler wait for them where the branch joins: the next page's loads behind an `if` had every
  // iteration wait for them before its last output MFMA.
  auto load_k = [&](int p, bool live) __attribute__((always_inline)) {
    const long pg = page_of(p);
    const bool ok = live && page_ok(pg);
    const __amdgpu_buffer_rsrc_t rk = kv_rsrc(a.k_cache + ((ok ? pg : 0) * a.Hkv + g) * kv_head_stride, ok);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      kr[kk] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, (lr * kHD + 32 * kk + 8 * lg) * 2, 0,
                                                                                 kCachePolicyNT));
  };
  auto load_v = [&](int p, bool live) __attribute__((always_inline)) {
    const long pg = page_of(p);
    const bool ok = live && page_ok(pg);
    const __amdgpu_buffer_rsrc_t rv = kv_rsrc(a.v_cache + ((ok ? pg : 0) * a.Hkv + g) * kv_head_stride, ok);
#pragma unroll
    for (int n = 0; n < 8; ++n)
      vr[n] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rv, ((16 * n + lr) * kPage + 4 * lg) * 2, 0,
                                                                                kCachePolicyNT));
  };

  int p = p_begin + wave;
  load_k(p, p < p_end);
  load_v(p, p < p_end);
  for (; p < p_end; p += kAttnWaves) {
    const bool more = p + kAttnWaves < p_end;
    // scores S^T: lane holds keys 4 lg + i of head lr
    v4f s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
      s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, kr[kk]), qop[kk], s, 0, 0, 0);
    load_k(p + kAttnWaves, more);
    const int key0 = p * kPage + 4 * lg;
    const int key_end = page_ok(page_of(p)) ? ctx : 0;  // an empty page has no live keys
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // the reference's rounding: bf16 matmul output, then a bf16 multiply by the scale
      const float x = bf16_round(bf16_round(s[i]) * a.scale);
      sv[i] = key0 + i < key_end ? x : -INFINITY;
    }
    float pm = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    pm = rows_max(pm);
    const float m_new = fmaxf(m_run, pm);  // -inf only while every page so far was empty
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;
    const float corr = __builtin_amdgcn_exp2f((m_run - m_ref) * 1.4426950408889634f);  // 0 on the first page
    float pv[4], ps = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pv[i] = __builtin_amdgcn_exp2f((sv[i] - m_ref) * 1.4426950408889634f);
      ps += pv[i];
    }
    ps = rows_sum(ps);
    l_run = l_run * corr + ps;
    m_run = m_new;
    // P^T as the B operand (keys 4 lg + i of head lr)
    v4s pb;
#pragma unroll
    for (int i = 0; i < 4; ++i) pb[i] = (short)f32_to_bf16(pv[i]);
    // keys past the end of the sequence (last page) have P = 0; their V slots may hold
    // anything (the pool is not cleared), so they are zeroed rather than multiplied by 0:
    // keys 4 lg + j with j < live_keys are valid (j = 0, 1 in v.x, j = 2, 3 in v.y)
    const int live_keys = key_end - key0;
    const uint32_t mask_x = live_keys >= 2 ? 0xffffffffu : (live_keys == 1 ? 0xffffu : 0u);
    const uint32_t mask_y = live_keys >= 4 ? 0xffffffffu : (live_keys == 3 ? 0xffffu : 0u);
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const uint32_t vx = vr[n].x & mask_x, vy = vr[n].y & mask_y;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[n][i] *= corr;
      v4s va;  // V^T rows: dim 16 n + lr, keys 4 lg .. 4 lg + 3
      va[0] = (short)(vx & 0xffffu);
      va[1] = (short)(vx >> 16);
      va[2] = (short)(vy & 0xffffu);
      va[3] = (short)(vy >> 16);
      o[n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, pb, o[n], 0, 0, 0);
    }
    load_v(p + kAttnWaves, more);
  }

  // merge the 4 waves: per head max, sum and O rows (head lr, dims 16 n + 4 lg + i)
  __shared__ float s_m[kAttnWaves][16], s_l[kAttnWaves][16];
  __shared__ __attribute__((aligned(16))) float s_o[kAttnWaves][16][kHD + 4];
  if (lg == 0) {
    s_m[wave][lr] = m_run;
    s_l[wave][lr] = l_run;
  }
#pragma unroll
  for (int n = 0; n < 8; ++n) *(v4f*)&s_o[wave][lr][16 * n + 4 * lg] = o[n];
  __syncthreads();
  // 256 threads: head hh = tid / 16 (< G used), dims 8 (tid % 16) .. +8
  const int hh = threadIdx.x >> 4, d0 = (threadIdx.x & 15) * 8;
  if (hh < G) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, s_m[w][hh]);
    float wgt[kAttnWaves], L = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      // a wave with no pages in this split has m = -inf and contributes nothing
      wgt[w] = s_m[w][hh] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((s_m[w][hh] - M) * 1.4426950408889634f);
      L += s_l[w][hh] * wgt[w];
    }
    const long base = (((long)b * a.Hkv + g) * a.max_splits + split) * G + hh;
    float* dst = a.part_o + base * kHD + d0;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) acc += s_o[w][hh][d0 + d] * wgt[w];
      dst[d] = acc;
    }
    if ((threadIdx.x & 15) == 0) {
      a.part_ml[base * 2] = M;
      a.part_ml[base * 2 + 1] = L;
    }
  }
}

// out[b, h, :] = bf16( sum_s w_s O_s / sum_s w_s l_s ), w_s = exp(m_s - max m), the sums in
// split order.  One workgroup per (sequence, kv head); a thread owns 4 dims of one head of the
// group.  The partials of the first kMergeUnroll splits are loaded at split indices clamped to
// the workspace's max_splits (in bounds whatever the context length), in the same round trip
// as the context length; splits past the sequence's count are masked.  Longer sequences (more
// splits, small batches) continue in batches of kMergeUnroll.
constexpr int kMergeUnroll = 8;
__global__ __launch_bounds__(256) void paged_attn_merge_kernel(AttnArgs a, uint16_t* __restrict__ out) {
  const int g = blockIdx.x, b = blockIdx.y;
  const int G = a.Hq / a.Hkv;
  const int ctx = a.context_lens[b];
  for (int i = threadIdx.x; i < G * (kHD / 4); i += blockDim.x) {
    const int hh = i / (kHD / 4), d0 = 4 * (i % (kHD / 4));
    const long base0 = ((long)b * a.Hkv + g) * a.max_splits * G + hh;  // split s: base0 + s G
    float2 ml[kMergeUnroll];
    float4 ov[kMergeUnroll];
    auto load = [&](int s0, int last) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < kMergeUnroll; ++u) {
        const long base = base0 + (long)min(s0 + u, last) * G;
        ml[u] = *(const float2*)(a.part_ml + base * 2);
        ov[u] = *(const float4*)(a.part_o + base * kHD + d0);
      }
    };
    load(0, a.max_splits - 1);
    uint16_t* dst = out + ((long)b * a.Hq + g * G + hh) * kHD + d0;
    const int ns = (attn_pages(ctx, a.max_pages) + a.pps - 1) / a.pps;
    if (ns == 0) {  // an empty context attends to nothing
      *(uint2*)dst = make_uint2(0u, 0u);
      continue;
    }
    float M = -INFINITY;
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) M = u < ns ? fmaxf(M, ml[u].x) : M;
    for (int s0 = kMergeUnroll; s0 < ns; s0 += kMergeUnroll) {
#pragma unroll
      for (int u = 0; u < kMergeUnroll; ++u)  // clamped repeats change no max
        M = fmaxf(M, a.part_ml[(base0 + (long)min(s0 + u, ns - 1) * G) * 2]);
    }
    float L = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < ns; s0 += kMergeUnroll) {
      if (s0 > 0) load(s0, ns - 1);
#pragma unroll
      for (int u = 0; u < kMergeUnroll; ++u) {
        if (s0 + u >= ns) break;
        // a split of empty pages only has m = -inf and adds nothing
        const float w = ml[u].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((ml[u].x - M) * 1.4426950408889634f);
        L += ml[u].y * w;
        acc[0] += ov[u].x * w;
        acc[1] += ov[u].y * w;
        acc[2] += ov[u].z * w;
        acc[3] += ov[u].w * w;
      }
    }
    if (L == 0.f) {  // every page of the context empty: as an empty context
      *(uint2*)dst = make_uint2(0u, 0u);
      continue;
    }
    *(uint2*)dst = make_uint2((uint32_t)f32_to_bf16(acc[0] / L) | ((uint32_t)f32_to_bf16(acc[1] / L) << 16),
                              (uint32_t)f32_to_bf16(acc[2] / L) | ((uint32_t)f32_to_bf16(acc[3] / L) << 16));
  }
}

// Writes the new token's k (row layout) and v (transposed layout) of every kv head at
// position positions[b] of sequence b.
__global__ __launch_bounds__(256) void kv_append_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                        uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
                                                        const int32_t* __restrict__ block_tables,
                                                        const int32_t* __restrict__ positions, int Hkv, int max_pages,
                                                        int num_pages) {
  const int b = blockIdx.x;
  const int pos = positions[b];
  if (pos < 0 || pos >= kPage * max_pages) return;  // outside the block table: nothing to write
  const long pg = block_tables[(long)b * max_pages + pos / kPage];
  if (pg < 0 || pg >= num_pages) return;  // a table entry outside the pools: nothing to write
  const int slot = pos % kPage;
  for (int i = threadIdx.x; i < Hkv * kHD; i += blockDim.x) {
    const int g = i / kHD, d = i % kHD;
    const long head = (pg * Hkv + g) * (long)(kHD * kPage);
    k_cache[head + slot * kHD + d] = k[(long)b * Hkv * kHD + i];
    v_cache[head + d * kPage + slot] = v[(long)b * Hkv * kHD + i];
  }
}

int attn_max_splits(int max_pages, int pps) { return (max_pages + pps - 1) / pps; }

// pages per split: enough workgroups to fill the chip for the batch, at least 8 pages each
int attn_pps(int B, int Hkv, int max_pages) {
  int pps = 64;  // <= 4 waves x 64 lanes: a wave's page ids fit one register
  while (pps > 8 && (long)B * Hkv * attn_max_splits(max_pages, pps) < 1024) pps /= 2;
  return pps;
}

// the decode grid (one workgroup per possible (sequence, kv head, split) item) and the items'
// int indices must stay below 2^31
bool attn_grid_ok(int B, int Hkv, int max_pages) {
  return (long)B * Hkv * attn_max_splits(max_pages, attn_pps(B, Hkv, max_pages)) < (1L << 31);
}

bool attn_args_ok(int B, int Hq, int Hkv, int head_dim, int page_size, int max_pages, int num_pages) {
  return B > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0 && Hq / Hkv <= 16 && head_dim == kHD &&
         page_size == kPage && max_pages > 0 && num_pages >= 0 && attn_grid_ok(B, Hkv, max_pages);
}

}  // namespace

extern "C" size_t moe_mi355x_paged_attn_workspace_bytes(int B, int Hq, int Hkv, int max_pages) {
  if (B <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv || max_pages <= 0 || !attn_grid_ok(B, Hkv, max_pages)) return 0;
  const int pps = attn_pps(B, Hkv, max_pages);
  const long parts = (long)B * Hq * attn_max_splits(max_pages, pps);
  return moe_align_up((size_t)parts * kHD * sizeof(float), 256) + moe_align_up((size_t)parts * 2 * sizeof(float), 256);
}

extern "C" int moe_mi355x_paged_attn_decode(const void* q, const void* k_cache, const void* v_cache,
                                            const int32_t* block_tables, const int32_t* context_lens, int B,
                                            int Hq, int Hkv, int head_dim, int page_size, int max_pages,
                                            int num_pages, float scale, void* out, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  MOE_RETURN_IF(!attn_args_ok(B, Hq, Hkv, head_dim, page_size, max_pages, num_pages), MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!q || !k_cache || !v_cache || !block_tables || !context_lens || !out, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!moe_aligned16(q) || !moe_aligned16(k_cache) || !moe_aligned16(v_cache) || !moe_aligned16(out),
                MOE_ERR_ALIGNMENT);
  MOE_RETURN_IF(!workspace || workspace_bytes < moe_mi355x_paged_attn_workspace_bytes(B, Hq, Hkv, max_pages),
                MOE_ERR_WORKSPACE);
  const int pps = attn_pps(B, Hkv, max_pages);
  const int ms = attn_max_splits(max_pages, pps);
  WsCarver c(workspace);
  const long parts = (long)B * Hq * ms;
  float* part_o = c.take<float>((size_t)parts * kHD);
  float* part_ml = c.take<float>((size_t)parts * 2);
  AttnArgs a{(const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache, block_tables, context_lens,
             part_o, part_ml, B, Hq, Hkv, max_pages, ms, pps, num_pages, scale};
  hipStream_t s = (hipStream_t)stream;
  // an upper bound of the (b, g, split) items; the kernel maps workgroups to the live ones
  hipLaunchKernelGGL(paged_attn_decode_kernel, dim3((unsigned)((long)B * Hkv * ms)), dim3(256), 0, s, a);
  MOE_CHECK_LAUNCH();
  hipLaunchKernelGGL(paged_attn_merge_kernel, dim3(Hkv, B), dim3(256), 0, s, a, (uint16_t*)out);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}

extern "C" int moe_mi355x_kv_append(const void* k, const void* v, void* k_cache, void* v_cache,
                                    const int32_t* block_tables, const int32_t* positions, int B, int Hkv,
                                    int head_dim, int page_size, int max_pages, int num_pages, void* stream) {
  MOE_RETURN_IF(B <= 0 || Hkv <= 0 || head_dim != kHD || page_size != kPage || max_pages <= 0 || num_pages < 0,
                MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!k || !v || !k_cache || !v_cache || !block_tables || !positions, MOE_ERR_INVALID_ARG);
  hipLaunchKernelGGL(kv_append_kernel, dim3(B), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)k,
                     (const uint16_t*)v, (uint16_t*)k_cache, (uint16_t*)v_cache, block_tables, positions, Hkv,
                     max_pages, num_pages);
  MOE_CHECK_LAUNCH();
  return MOE_OK;
}
