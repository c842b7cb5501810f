// bf16 linear layer without bias, y [M, N] = bf16(x [M, K] @ w [N, K]^T): the q/k/v and o_proj
// projections of a decode step (TF/models/qwen3_moe/modeling_qwen3_moe.py:162-164, :189), batches of
// up to a few hundred rows against weights of tens of MB.
//
// The weights are the stream (21 MB for the Qwen3-30B-A3B q/k/v at K = 2048), so they are spread
// over all CUs with a split of K across workgroups, and each workgroup reads its activation rows
// once per K block, into LDS, for all of its columns:
//   grid (N / 64 column blocks, ceil(M / 128) row blocks, ks K chunks); workgroup = 4 waves, wave w
//   owns 16 weight rows (columns of y) and all of the block's rows (up to 128 = 8 MFMA row tiles).
//   Per 128-deep K block the workgroup stages x [rows, 128] in LDS (double-buffered, one barrier
//   per block); each wave streams its 16 weight rows straight into VGPRs, PF blocks ahead, and the
//   activation rows for LDS are likewise loaded PF blocks ahead into VGPRs.
//   v_mfma_f32_16x16x32_bf16 with the weight fragment as A and the activation fragment as B:
//   lane l holds columns 4 (l / 16) + q of row l % 16.
// With ks > 1 each workgroup writes its fp32 partial block and linear_reduce_kernel sums the ks
// partials of every output in chunk order (deterministic) and rounds once to bf16.
//
// Measured on MI355X with weights cold in HBM and graph-launched calls: 10-10.7 us for the q/k/v and
// o_proj shapes at 1 to 16 rows (hipBLASLt: 12-14 us), 16 / 13.5 us at 64 rows (12.7 / 13.3 us);
// at 128 rows 20 / 18 us against hipBLASLt's 15 / 12 us, 4-5 us of which is the partial-sum pass.
#include "common.h"

namespace {

constexpr int LBM = 128;  // rows per workgroup
constexpr int LBN = 64;   // N granule: the columns of a 4-wave workgroup
constexpr int LBK = 128;  // K block

struct LinearArgs {
  const uint16_t* x;  // [M, K]
  const uint16_t* w;  // [N, K]
  float* part;        // [ks, M, N] (ks > 1)
  uint16_t* y;        // [M, N] (ks == 1)
  int M, N, K, kchunk;
};

template <int WM, int NW, int PF>  // 16-row MFMA tiles per wave, waves per workgroup, blocks loaded ahead
__global__ __launch_bounds__(64 * NW) void linear_bf16_kernel(LinearArgs p) {
  constexpr int BM = 16 * WM, NT = 64 * NW;
  // x block [BM rows][16 chunks of 8 bf16]; chunk c of row r at c ^ (r & 15), so the 16 rows of an
  // MFMA fragment read (one chunk per 16 lanes) fall in distinct banks
  __shared__ uint4 s_x[2][BM * 16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * (16 * NW) + 16 * wave;
  const int m0 = blockIdx.y * BM;
  const int kbeg = blockIdx.z * p.kchunk;
  const int nkb = (min(p.K, kbeg + p.kchunk) - kbeg) / LBK;

  // this lane's weight row and K offset within a block: 8 bf16 at 8 lg + 32 u, u = 0..3
  const uint16_t* wrow = p.w + (long)(n0 + lr) * p.K + kbeg + 8 * lg;
  auto load_w = [&](int kb, uint4 (&f)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 4; ++u) f[u] = *(const uint4*)(wrow + (long)kb * LBK + 32 * u);
  };
  // x staging: BM rows x 16 chunks, XPT per thread
  constexpr int XPT = (BM * 16 + NT - 1) / NT;
  auto load_x = [&](int kb, uint4 (&f)[XPT]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int idx = tid + NT * i, r = idx >> 4, c = idx & 15;
      if (BM * 16 % NT == 0 || idx < BM * 16) {
        const int row = min(m0 + r, p.M - 1);  // rows past M repeat the last one (never stored)
        f[i] = *(const uint4*)(p.x + (long)row * p.K + kbeg + (long)kb * LBK + 8 * c);
      }
    }
  };
  auto store_x = [&](int buf, const uint4 (&f)[XPT]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int idx = tid + NT * i, r = idx >> 4, c = idx & 15;
      if (BM * 16 % NT == 0 || idx < BM * 16) s_x[buf][r * 16 + (c ^ (r & 15))] = f[i];
    }
  };

  v4f acc[WM];
#pragma unroll
  for (int mi = 0; mi < WM; ++mi) acc[mi] = (v4f){0.f, 0.f, 0.f, 0.f};
  // rings: w[j] holds block kb + j, x[j] block kb + 1 + j (x of block kb is in LDS)
  uint4 wr[PF + 1][4], xr[PF][XPT];
#pragma unroll
  for (int j = 0; j <= PF; ++j)
    if (j < nkb) load_w(j, wr[j]);
  {
    uint4 x0[XPT];
    load_x(0, x0);
#pragma unroll
    for (int j = 0; j < PF; ++j)
      if (j + 1 < nkb) load_x(j + 1, xr[j]);
    store_x(0, x0);
  }
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int buf = kb & 1;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const v8bf a = __builtin_bit_cast(v8bf, wr[0][u]);
      const int ch = 4 * u + lg;  // chunk of the lane's 8 K values within the block
#pragma unroll
      for (int mi = 0; mi < WM; ++mi) {
        const int r = mi * 16 + lr;
        const v8bf b = __builtin_bit_cast(v8bf, s_x[buf][r * 16 + (ch ^ (r & 15))]);
        acc[mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[mi], 0, 0, 0);
      }
    }
    // advance the rings by one block and issue the loads PF + 1 (w) and PF + 1 (x) blocks ahead
#pragma unroll
    for (int j = 0; j < PF; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) wr[j][u] = wr[j + 1][u];
    if (kb + 1 + PF < nkb) load_w(kb + 1 + PF, wr[PF]);
    if (kb + 1 < nkb) {
      store_x(buf ^ 1, xr[0]);  // the other buffer was last read a block ago, before the last barrier
#pragma unroll
      for (int j = 0; j + 1 < PF; ++j)
#pragma unroll
        for (int i = 0; i < XPT; ++i) xr[j][i] = xr[j + 1][i];
      if (kb + 1 + PF < nkb) load_x(kb + 1 + PF, xr[PF - 1]);
    }
    __syncthreads();
  }

  // lane holds y[m0 + 16 mi + lr][n0 + 4 lg + q]
#pragma unroll
  for (int mi = 0; mi < WM; ++mi) {
    const int m = m0 + 16 * mi + lr;
    if (m >= p.M) continue;
    const int n = n0 + 4 * lg;
    if (p.part != nullptr) {
      *(float4*)(p.part + ((long)blockIdx.z * p.M + m) * p.N + n) =
          make_float4(acc[mi][0], acc[mi][1], acc[mi][2], acc[mi][3]);
    } else {
      uint2 v;
      v.x = (uint32_t)f32_to_bf16(acc[mi][0]) | ((uint32_t)f32_to_bf16(acc[mi][1]) << 16);
      v.y = (uint32_t)f32_to_bf16(acc[mi][2]) | ((uint32_t)f32_to_bf16(acc[mi][3]) << 16);
      *(uint2*)(p.y + (long)m * p.N + n) = v;
    }
  }
}

// y = bf16(sum over the ks partials in chunk order), 4 outputs per thread
__global__ __launch_bounds__(256) void linear_reduce_kernel(const float* __restrict__ part, int ks, long MN,
                                                            uint16_t* __restrict__ y) {
  const long i = 4 * ((long)blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= MN) return;
  float4 s = *(const float4*)(part + i);
  for (int z = 1; z < ks; ++z) {
    const float4 v = *(const float4*)(part + (long)z * MN + i);
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  uint2 o;
  o.x = (uint32_t)f32_to_bf16(s.x) | ((uint32_t)f32_to_bf16(s.y) << 16);
  o.y = (uint32_t)f32_to_bf16(s.z) | ((uint32_t)f32_to_bf16(s.w) << 16);
  *(uint2*)(y + i) = o;
}

// Configuration of one call: waves per workgroup (16 columns each), blocks loaded ahead and the
// number of K chunks.
struct LinearCfg {
  int nw, pf, ks;
};

int k_blocks_divisor(int nkb, int ks) {  // largest divisor of nkb not above ks (equal chunks)
  if (ks < 1) ks = 1;
  while (ks > 1 && nkb % ks != 0) --ks;
  return ks;
}

// Measured on MI355X (q/k/v 5120 x 2048 and o_proj 2048 x 4096 weights, batches 1 to 128): 4-wave
// workgroups; one block loaded ahead up to 16 rows, two above; K chunks of 4 blocks (512), fewer
// chunks where the fp32 partials (ks M N 4 bytes, written and read back once) would exceed half
// the weight bytes.
LinearCfg linear_cfg(int M, int N, int K) {
  LinearCfg c{4, M > 16 ? 2 : 1, 1};
  int ks = K / 512 > 0 ? K / 512 : 1;
  if (M > 0 && K / (4 * M) < ks) ks = K / (4 * M) > 0 ? K / (4 * M) : 1;
  c.ks = k_blocks_divisor(K / LBK, ks);
  return c;
}

bool linear_args_ok(int M, int N, int K) {
  return M >= 0 && N > 0 && K > 0 && N % LBN == 0 && K % LBK == 0 && (long)N * K < (1L << 31) &&
         (long)M * K < (1L << 31) && (long)M * N < (1L << 29);
}

size_t linear_ws_bytes(int M, int N, int ks) {
  return ks > 1 ? moe_align_up((size_t)ks * M * N * sizeof(float), 256) : 0;
}

template <int NW, int PF>
void launch_linear_kernel(const LinearArgs& a, int ks, hipStream_t s) {
  const int M = a.M;
  dim3 g(a.N / (16 * NW), M > 64 ? (M + LBM - 1) / LBM : 1, ks);
  // row blocks of 128 (8 row tiles per wave), or of the batch rounded up to 16, 32 or 64 rows
  if (M > 64)
    MOE_LAUNCH(MOE_PROF_LINEAR, s, (linear_bf16_kernel<8, NW, PF>), g, dim3(64 * NW), 0, s, a);
  else if (M > 32)
    MOE_LAUNCH(MOE_PROF_LINEAR, s, (linear_bf16_kernel<4, NW, PF>), g, dim3(64 * NW), 0, s, a);
  else if (M > 16)
    MOE_LAUNCH(MOE_PROF_LINEAR, s, (linear_bf16_kernel<2, NW, PF>), g, dim3(64 * NW), 0, s, a);
  else
    MOE_LAUNCH(MOE_PROF_LINEAR, s, (linear_bf16_kernel<1, NW, PF>), g, dim3(64 * NW), 0, s, a);
}

int run_linear(const void* x, const void* w, int M, int N, int K, void* y, void* workspace, size_t workspace_bytes,
               LinearCfg c, hipStream_t s) {
  MOE_RETURN_IF(!linear_args_ok(M, N, K) || N % (16 * c.nw) != 0, MOE_ERR_INVALID_ARG);
  if (M == 0) return MOE_OK;
  MOE_RETURN_IF(!x || !w || !y, MOE_ERR_INVALID_ARG);
  MOE_RETURN_IF(!moe_aligned16(x) || !moe_aligned16(w) || !moe_aligned16(y), MOE_ERR_ALIGNMENT);
  const size_t need = linear_ws_bytes(M, N, c.ks);
  MOE_RETURN_IF(need > 0 && (!workspace || workspace_bytes < need), MOE_ERR_WORKSPACE);
  MOE_RETURN_IF(need > 0 && !moe_aligned16(workspace), MOE_ERR_ALIGNMENT);
  LinearArgs a{(const uint16_t*)x, (const uint16_t*)w, c.ks > 1 ? (float*)workspace : nullptr, (uint16_t*)y, M, N, K,
               K / c.ks};
  if (c.nw == 4 && c.pf == 2)
    launch_linear_kernel<4, 2>(a, c.ks, s);
  else if (c.nw == 4 && c.pf == 1)
    launch_linear_kernel<4, 1>(a, c.ks, s);
#ifdef MOE_LINEAR_SWEEP
  else if (c.nw == 5 && c.pf == 2)
    launch_linear_kernel<5, 2>(a, c.ks, s);
  else if (c.nw == 10 && c.pf == 2)
    launch_linear_kernel<10, 2>(a, c.ks, s);
  else if (c.nw == 5 && c.pf == 1)
    launch_linear_kernel<5, 1>(a, c.ks, s);
  else if (c.nw == 10 && c.pf == 1)
    launch_linear_kernel<10, 1>(a, c.ks, s);
  else if (c.nw == 8 && c.pf == 2)
    launch_linear_kernel<8, 2>(a, c.ks, s);
  else if (c.nw == 8 && c.pf == 1)
    launch_linear_kernel<8, 1>(a, c.ks, s);
#endif
  else
    return MOE_ERR_INVALID_ARG;
  MOE_CHECK_LAUNCH();
  if (c.ks > 1) {
    const long MN = (long)M * N;
    MOE_LAUNCH(MOE_PROF_LINEAR, s, linear_reduce_kernel, dim3((unsigned)((MN / 4 + 255) / 256)), dim3(256), 0, s,
               (const float*)workspace, c.ks, MN, (uint16_t*)y);
    MOE_CHECK_LAUNCH();
  }
  return MOE_OK;
}

}  // namespace

extern "C" size_t moe_mi355x_linear_bf16_workspace_bytes(int M, int N, int K) {
  if (!linear_args_ok(M, N, K) || M == 0) return 0;
  return linear_ws_bytes(M, N, linear_cfg(M, N, K).ks);
}

extern "C" int moe_mi355x_linear_bf16(const void* x, const void* w, int M, int N, int K, void* y, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  MOE_RETURN_IF(!linear_args_ok(M, N, K), MOE_ERR_INVALID_ARG);
  return run_linear(x, w, M, N, K, y, workspace, workspace_bytes, linear_cfg(M, N, K), (hipStream_t)stream);
}

#ifdef MOE_LINEAR_SWEEP
// Tuning entry (built only with -DMOE_LINEAR_SWEEP): one call at a given configuration.
extern "C" int moe_linear_sweep(const void* x, const void* w, int M, int N, int K, void* y, void* workspace,
                                size_t workspace_bytes, int nw, int pf, int ks, void* stream) {
  MOE_RETURN_IF(K % LBK != 0, MOE_ERR_INVALID_ARG);
  return run_linear(x, w, M, N, K, y, workspace, workspace_bytes, LinearCfg{nw, pf, k_blocks_divisor(K / LBK, ks)},
                    (hipStream_t)stream);
}
#endif
