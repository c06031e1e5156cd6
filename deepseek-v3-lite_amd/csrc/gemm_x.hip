// Backward grouped GEMMs: every operand layout of the MoE backward pass.
//
//   dh  = dY W2        A rows (tokens gathered), B weights N-contiguous (NN),
//                      epilogue: SwiGLU backward with the saved g, u
//   dx  = [dg|du][W1;W3]  A rows, B weights N-contiguous, two K segments
//   dW13 = [dg|du]^T X, dW2 = (w dY)^T H
//                      A and B both K-major (K = the rows routed to an
//                      expert, a ragged range per group), per-expert outputs
//
// Restates the backward of models/moe.py:127-131 (autograd through the
// per-expert matmuls) and models/moe_triton.py:138-374 (dx and dW kernels);
// each output tile is produced by one block that walks its K range in
// ascending order, so dW accumulation is deterministic with no atomics.
//
// xgemm_simt_kernel: fp32 FMA tiles for every mode (fp32 path and fallback).
#include "gemm_tile.h"

namespace dsmoe {

constexpr int XS_BM = 64;
constexpr int XS_BN = 64;
constexpr int XS_BK = 16;

template <typename T>
__device__ __forceinline__ float xa_load(const XGemm& g, int grp, int row0, int m, int k) {
  const T* A = static_cast<const T*>(g.A);
  if (g.a_mode == XA_ROWS) {
    const int r = row0 + m;
    const int64_t ar = g.a_map ? g.a_map[r] : r;
    return to_f<T>(A[ar * g.lda + k]);
  }
  const int64_t ar = g.a_map ? g.a_map[k] : k;
  const float s = g.a_kscale ? g.a_kscale[k] : 1.0f;
  return to_f<T>(A[ar * g.lda + (int64_t)grp * g.a_col + row0 + m]) * s;
}

template <typename T>
__device__ __forceinline__ float xb_load(const XGemm& g, int grp, int n, int k) {
  if (g.b_mode == XB_ACT_KMAJOR) {
    const int64_t br = g.b_map ? g.b_map[k] : k;
    return to_f<T>(static_cast<const T*>(g.Bact)[br * g.ldb + (int64_t)grp * g.b_col + n]);
  }
  const int seg = k / g.kseg;
  const int kin = k - seg * g.kseg;
  const T* base = static_cast<const T*>(g.Btab[(int64_t)grp * g.nseg + seg]);
  if (g.b_mode == XB_W_NT) return to_f<T>(base[(int64_t)n * g.ldb + kin]);
  return to_f<T>(base[(int64_t)kin * g.ldb + n]);
}

// Shared epilogue for one output element (row m of the tile, column n).
template <typename T, int EPI>
__device__ __forceinline__ void x_store(const XGemm& g, int grp, int row0, int m, int n, float acc) {
  if (EPI == XE_WGRAD) {
    const int mm = row0 + m;
    void* base = mm < g.msplit ? g.Ctab0[grp] : g.Ctab1[grp];
    const int64_t o = (int64_t)(mm < g.msplit ? mm : mm - g.msplit) * g.ldc + n;
    if (g.c_f32)
      static_cast<float*>(base)[o] = acc;
    else
      static_cast<T*>(base)[o] = from_f<T>(acc);
    return;
  }
  const int r = row0 + m;
  const int64_t crow = g.c_map ? g.c_map[r] : r;
  T* C = static_cast<T*>(g.C);
  const int64_t o = crow * g.ldc + (int64_t)grp * g.c_group_col + n;
  if (EPI == XE_STORE) {
    C[o] = from_f<T>(acc);
    return;
  }
  // SwiGLU backward: h = silu(gv) * uv, dh = w * acc
  const int64_t ogu = (int64_t)r * g.ld_gu + (int64_t)grp * g.gu_group_col + n;
  const float gv = to_f<T>(static_cast<const T*>(g.Gs)[ogu]);
  const float uv = to_f<T>(static_cast<const T*>(g.Us)[ogu]);
  const float dh = (g.row_w ? g.row_w[r] : 1.0f) * acc;
  const float sg = sigmoid_f(gv);
  C[o] = from_f<T>(dh * uv * sg * (1.0f + gv * (1.0f - sg)));
  C[o + g.du_off] = from_f<T>(dh * gv * sg);
}

template <typename T, int EPI>
__global__ __launch_bounds__(256) void xgemm_simt_kernel(const XGemm g) {
  __shared__ float As[XS_BK][XS_BM + 4];
  __shared__ float Bs[XS_BK][XS_BN + 4];
  int grp, row0, rows, n_tile, kbeg, kend, split;
  if (!xtile<XS_BM, XS_BN>(g, grp, row0, rows, n_tile, kbeg, kend, split)) return;
  const int n0 = n_tile * XS_BN;
  const int tid = threadIdx.x;
  const int ty = tid >> 4, tx = tid & 15;
  float acc[4][4] = {};
  for (int k0 = kbeg; k0 < kend; k0 += XS_BK) {
    for (int i = tid; i < XS_BM * XS_BK; i += 256) {
      // K-major A: consecutive threads walk m (contiguous); row-major A: walk k
      int m, kk;
      if (g.a_mode == XA_KMAJOR) {
        kk = i / XS_BM;
        m = i - kk * XS_BM;
      } else {
        m = i / XS_BK;
        kk = i - m * XS_BK;
      }
      float v = 0.0f;
      if (m < rows && k0 + kk < kend) v = xa_load<T>(g, grp, row0, m, k0 + kk);
      As[kk][m] = v;
    }
    for (int i = tid; i < XS_BN * XS_BK; i += 256) {
      int n, kk;
      if (g.b_mode == XB_W_NT) {
        n = i / XS_BK;
        kk = i - n * XS_BK;
      } else {
        kk = i / XS_BN;
        n = i - kk * XS_BN;
      }
      float v = 0.0f;
      if (n0 + n < g.N && k0 + kk < kend) v = xb_load<T>(g, grp, n0 + n, k0 + kk);
      Bs[kk][n] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < XS_BK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = ty * 4 + i;
    if (m >= rows) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n < g.N) x_store<T, EPI>(g, grp, row0, m, n, acc[i][j]);
    }
  }
}

static int64_t xgrid(const XGemm& g, int bm, int bn) {
  int64_t m_bound;
  if (g.sched_mode == XS_ROUTED)
    m_bound = (int64_t)g.m_tiles_bound * (g.bm / bm);
  else if (g.sched_mode == XS_DENSE)
    m_bound = cdiv(g.dense_rows, bm) * g.groups;
  else
    m_bound = cdiv(g.M, bm) * g.groups;
  return 8 * cdiv(m_bound * cdiv(g.N, bn), 8);
}

template <typename T>
static int launch_xsimt(const XGemm& g, int epi, hipStream_t st) {
  const int64_t grid = xgrid(g, XS_BM, XS_BN);
  if (grid == 0) return DSMOE_OK;
  if (epi == XE_STORE)
    hipLaunchKernelGGL((xgemm_simt_kernel<T, XE_STORE>), dim3((unsigned)grid), dim3(256), 0, st, g);
  else if (epi == XE_SWIGLU_BWD)
    hipLaunchKernelGGL((xgemm_simt_kernel<T, XE_SWIGLU_BWD>), dim3((unsigned)grid), dim3(256), 0, st, g);
  else
    hipLaunchKernelGGL((xgemm_simt_kernel<T, XE_WGRAD>), dim3((unsigned)grid), dim3(256), 0, st, g);
  return check_launch("xgemm_simt");
}

int launch_xgemm(const XGemm& g, int epi, int dtype, bool allow_mfma, hipStream_t st) {
  if (g.N <= 0 || (g.sched_mode == XS_WGRAD ? g.M <= 0 : false)) return DSMOE_OK;
  if (dtype == DSMOE_BF16 && allow_mfma && xgemm_q_ok(g, epi)) return launch_xgemm_q(g, epi, st);
  if (dtype == DSMOE_BF16 && allow_mfma && xgemm_mfma_ok(g, epi)) return launch_xgemm_mfma(g, epi, st);
  if (g.ksplit > 1) {  // the FMA tiles store directly
    XGemm g1 = g;
    g1.ksplit = 1;
    return launch_xgemm(g1, epi, dtype, false, st);
  }
  if (g.sched_mode == XS_ROUTED && g.bm % XS_BM != 0)
    return fail(DSMOE_ERR_INVALID, "xgemm: schedule height must be a multiple of 64");
  if (dtype == DSMOE_BF16) return launch_xsimt<bf16_t>(g, epi, st);
  return launch_xsimt<float>(g, epi, st);
}

}  // namespace dsmoe
