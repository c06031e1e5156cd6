// (c) Grouped expert GEMMs over expert-sorted rows.
//
// C[cmap(r)][n] = epilogue( sum_k A[amap(r)][k] * B_g[n][k] ), both operands
// K-contiguous ("NT"), as nn.Linear stores x and W.  Restates the per-expert
// GEMMs of models/moe.py:127-131 (gate/up fused with silu*mul, then down) and
// the grouped operator of models/moe_triton.py:28-51,57-135.
//
// Work split: a launch enumerates (M tile, N tile) pairs, N fastest.  M tiles
// come from the device-side schedule the permute scan writes (one entry per
// BM-row tile inside each expert, so skewed loads simply produce more tiles
// for the hot experts) or are dense (shared experts: every group covers all
// rows).  Block b runs on XCD b % 8; each XCD takes one contiguous eighth of
// the tile list so the weight tiles of an expert stay in that XCD's L2.  The
// grid is sized from a host bound; blocks past the device count exit.
//
// Kernels (the default bf16 path is the persistent gemm_qp_kernel of
// gemm_qp.hip; this file holds the register-staged MFMA kernel for the shapes
// that one does not take, the fp32 fallback and the dispatcher):
//   gemm_mfma_kernel  bf16 on gfx950 v_mfma_f32_32x32x16_bf16.  Block =
//                     WM x WN waves, each owning TM x TN 32x32 output tiles
//                     (x2 for SwiGLU: the W1 and W3 tiles of the same columns
//                     sit in the same lane, so silu(g)*u is a register op).
//                     K slabs of 64 go global -> registers -> LDS (double
//                     buffered, XOR-swizzled 16-byte chunks) one slab ahead.
//                     Rows past a tile's end are clamped to a valid row: their
//                     results are discarded, so no load is predicated.
//   gemm_simt_kernel  fp32 FMA fallback for fp32 and for shapes the MFMA
//                     kernel does not take (any N, K, strides).
#include <cstdlib>
#include <cstring>

#include "gemm_tile.h"
#include "mfma.h"

namespace dsmoe {

// =============================================================== MFMA kernel
template <int EPI, int WM, int WN, int TM, int TN>
struct MfCfg {
  static constexpr int NB = (EPI == EPI_SWIGLU) ? 2 : 1;
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int BM = WM * TM * 32;
  static constexpr int BN = WN * TN * 32;
  static constexpr int A_EL = BM * MF_K;
  static constexpr int B_EL = BN * MF_K;
  static constexpr int STAGE = A_EL + NB * B_EL;
  static constexpr int RSTEP = THREADS / 8;       // rows covered by one pass of the block
  static constexpr int A_LD = BM / RSTEP;         // 16-byte chunks per thread per stage (A)
  static constexpr int B_LD = BN / RSTEP;         // per B operand
  static constexpr size_t LDS_BYTES = 2ull * STAGE * sizeof(bf16_t);
  static_assert(BM % RSTEP == 0 && BN % RSTEP == 0, "tile rows must be a multiple of threads/8");
};

template <int N>
__device__ __forceinline__ void load_rows(const bf16_t* __restrict__ base, const int64_t (&off)[N], int k0,
                                          u32x4_t (&r)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) r[i] = ldg16(base + off[i] + k0);
}

template <int N, int RSTEP>
__device__ __forceinline__ void store_rows(bf16_t* __restrict__ s, int lr, int lc, const u32x4_t (&r)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) *reinterpret_cast<u32x4_t*>(s + swz(lr + i * RSTEP, lc)) = r[i];
}

template <int EPI, int WM, int WN, int TM, int TN>
__global__ __launch_bounds__(64 * WM * WN) void gemm_mfma_kernel(const GemmDesc g, const float* __restrict__ row_scale) {
  using CF = MfCfg<EPI, WM, WN, TM, TN>;
  constexpr int NB = CF::NB, BM = CF::BM, BN = CF::BN, RSTEP = CF::RSTEP;
  constexpr int A_LD = CF::A_LD, B_LD = CF::B_LD;
  extern __shared__ __attribute__((aligned(16))) bf16_t smem_mf[];

  const int n_tiles = (int)cdiv(g.N, BN);
  int grp, row0, rows, n_tile;
  if (!tile_for_block<BM>(g, n_tiles, grp, row0, rows, n_tile)) return;
  const int n0 = n_tile * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int lc = tid & 7;
  const int lr = tid >> 3;

  // Source offsets of this thread's 16-byte chunks (row-clamped).
  const bf16_t* __restrict__ A = static_cast<const bf16_t*>(g.A);
  int64_t a_off[A_LD];
#pragma unroll
  for (int i = 0; i < A_LD; ++i) {
    const int r = min(lr + i * RSTEP, rows - 1);
    const int64_t arow = g.a_map ? (int64_t)g.a_map[row0 + r] : (int64_t)(row0 + r);
    a_off[i] = arow * g.lda + lc * 8;
  }
  int64_t b_off[B_LD];
#pragma unroll
  for (int i = 0; i < B_LD; ++i) b_off[i] = (int64_t)min(n0 + lr + i * RSTEP, g.N - 1) * g.ldb + lc * 8;

  u32x4_t ra[A_LD];
  u32x4_t rb0[B_LD];
  u32x4_t rb1[B_LD];

  f32x16_t acc[NB][TM][TN];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int mi = 0; mi < TM; ++mi)
#pragma unroll
      for (int ni = 0; ni < TN; ++ni)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[b][mi][ni][r] = 0.0f;

  const int nk = g.K / MF_K;
  const void* const* __restrict__ tab0 = g.B0 + (int64_t)grp * g.nseg;
  const void* const* __restrict__ tab1 = (NB == 2) ? g.B1 + (int64_t)grp * g.nseg : nullptr;

  // ---- prologue: slab 0 -> LDS stage 0
  {
    load_rows(A, a_off, 0, ra);
    load_rows(static_cast<const bf16_t*>(tab0[0]), b_off, 0, rb0);
    if (NB == 2) load_rows(static_cast<const bf16_t*>(tab1[0]), b_off, 0, rb1);
    bf16_t* s = smem_mf;
    store_rows<A_LD, RSTEP>(s, lr, lc, ra);
    store_rows<B_LD, RSTEP>(s + CF::A_EL, lr, lc, rb0);
    if (NB == 2) store_rows<B_LD, RSTEP>(s + CF::A_EL + CF::B_EL, lr, lc, rb1);
  }
  __syncthreads();

  for (int kb = 0; kb < nk; ++kb) {
    const int cur = kb & 1;
    const bool more = kb + 1 < nk;
    if (more) {
      const int k0 = (kb + 1) * MF_K;
      const int seg = k0 / g.kseg;
      const int kin = k0 - seg * g.kseg;
      load_rows(A, a_off, k0, ra);
      load_rows(static_cast<const bf16_t*>(tab0[seg]), b_off, kin, rb0);
      if (NB == 2) load_rows(static_cast<const bf16_t*>(tab1[seg]), b_off, kin, rb1);
    }
    const bf16_t* sA = smem_mf + cur * CF::STAGE;
#pragma unroll
    for (int kk = 0; kk < MF_K / 16; ++kk) {
      const int c = kk * 2 + (lane >> 5);
      bf16x8_t af[TM];
#pragma unroll
      for (int mi = 0; mi < TM; ++mi) {
        const int r = (wm * TM + mi) * 32 + (lane & 31);
        af[mi] = *reinterpret_cast<const bf16x8_t*>(sA + swz(r, c));
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const bf16_t* sB = sA + CF::A_EL + b * CF::B_EL;
        bf16x8_t bfr[TN];
#pragma unroll
        for (int ni = 0; ni < TN; ++ni) {
          const int n = (wn * TN + ni) * 32 + (lane & 31);
          bfr[ni] = *reinterpret_cast<const bf16x8_t*>(sB + swz(n, c));
        }
#pragma unroll
        for (int mi = 0; mi < TM; ++mi)
#pragma unroll
          for (int ni = 0; ni < TN; ++ni)
            acc[b][mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[ni], af[mi], acc[b][mi][ni], 0, 0, 0);
      }
    }
    if (more) {
      bf16_t* s = smem_mf + (cur ^ 1) * CF::STAGE;
      store_rows<A_LD, RSTEP>(s, lr, lc, ra);
      store_rows<B_LD, RSTEP>(s + CF::A_EL, lr, lc, rb0);
      if (NB == 2) store_rows<B_LD, RSTEP>(s + CF::A_EL + CF::B_EL, lr, lc, rb1);
    }
    __syncthreads();
  }

  // ---- epilogue.  Lane holds row m = .. + (lane & 31) and, per q, columns
  // n = .. + 8q + 4*(lane >> 5) + {0..3} (acc registers 4q..4q+3).
  bf16_t* C = static_cast<bf16_t*>(g.C);
  const int64_t ccol = (int64_t)grp * g.c_group_col;
#pragma unroll
  for (int mi = 0; mi < TM; ++mi) {
    const int m = (wm * TM + mi) * 32 + (lane & 31);
    if (m >= rows) continue;
    const int64_t crow = g.c_map ? (int64_t)g.c_map[row0 + m] : (int64_t)(row0 + m);
    float scale = 1.0f;
    if (EPI == EPI_STORE && row_scale) scale = row_scale[row0 + m];
#pragma unroll
    for (int ni = 0; ni < TN; ++ni) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + (wn * TN + ni) * 32 + q * 8 + (lane >> 5) * 4;
        if (n >= g.N) continue;
        const int64_t o = crow * g.ldc + ccol + n;
        uint32_t packed[2];
        if (EPI == EPI_SWIGLU) {
          uint32_t pg[2], pu[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float g0 = acc[0][mi][ni][q * 4 + 2 * h], g1 = acc[0][mi][ni][q * 4 + 2 * h + 1];
            const float u0 = acc[NB - 1][mi][ni][q * 4 + 2 * h], u1 = acc[NB - 1][mi][ni][q * 4 + 2 * h + 1];
            packed[h] = (uint32_t)f2bf(silu_f(g0) * u0) | ((uint32_t)f2bf(silu_f(g1) * u1) << 16);
            pg[h] = (uint32_t)f2bf(g0) | ((uint32_t)f2bf(g1) << 16);
            pu[h] = (uint32_t)f2bf(u0) | ((uint32_t)f2bf(u1) << 16);
          }
          if (g.Gs) *reinterpret_cast<uint2*>(static_cast<bf16_t*>(g.Gs) + o) = make_uint2(pg[0], pg[1]);
          if (g.Us) *reinterpret_cast<uint2*>(static_cast<bf16_t*>(g.Us) + o) = make_uint2(pu[0], pu[1]);
        } else {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float v0 = acc[0][mi][ni][q * 4 + 2 * h] * scale, v1 = acc[0][mi][ni][q * 4 + 2 * h + 1] * scale;
            packed[h] = (uint32_t)f2bf(v0) | ((uint32_t)f2bf(v1) << 16);
          }
        }
        *reinterpret_cast<uint2*>(C + o) = make_uint2(packed[0], packed[1]);
      }
    }
  }
}

// =============================================================== SIMT kernel
constexpr int SM_N = 64;
constexpr int SM_K = 16;

template <typename T, int EPI>
__global__ __launch_bounds__(256) void gemm_simt_kernel(const GemmDesc g, const float* __restrict__ row_scale) {
  constexpr int NB = (EPI == EPI_SWIGLU) ? 2 : 1;
  __shared__ float As[SM_K][TILE_M + 4];
  __shared__ float Bs[NB][SM_K][SM_N + 4];
  const int n_tiles = (int)cdiv(g.N, SM_N);
  int grp, row0, rows, n_tile;
  if (!tile_for_block<TILE_M>(g, n_tiles, grp, row0, rows, n_tile)) return;
  const int n0 = n_tile * SM_N;
  const int tid = threadIdx.x;
  const int ty = tid >> 4, tx = tid & 15;  // rows ty*8.., cols tx*4..
  const T* A = static_cast<const T*>(g.A);
  float acc[NB][8][4];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[b][i][j] = 0.0f;

  for (int k0 = 0; k0 < g.K; k0 += SM_K) {
    for (int i = tid; i < TILE_M * SM_K; i += 256) {
      const int r = i / SM_K, kk = i % SM_K;
      float v = 0.0f;
      if (r < rows && k0 + kk < g.K) {
        const int64_t arow = g.a_map ? g.a_map[row0 + r] : (row0 + r);
        v = to_f<T>(A[arow * g.lda + k0 + kk]);
      }
      As[kk][r] = v;
    }
    for (int i = tid; i < SM_N * SM_K; i += 256) {
      const int n = i / SM_K, kk = i % SM_K;
      const int k = k0 + kk;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float v = 0.0f;
        if (n0 + n < g.N && k < g.K) {
          const int seg = k / g.kseg;
          const T* base = static_cast<const T*>((b == 0 ? g.B0 : g.B1)[grp * g.nseg + seg]);
          v = to_f<T>(base[(int64_t)(n0 + n) * g.ldb + (k - seg * g.kseg)]);
        }
        Bs[b][kk][n] = v;
      }
    }
    __syncthreads();
#pragma unroll 4
    for (int kk = 0; kk < SM_K; ++kk) {
      float a[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = As[kk][ty * 8 + i];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float bv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) bv[j] = Bs[b][kk][tx * 4 + j];
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[b][i][j] = fmaf(a[i], bv[j], acc[b][i][j]);
      }
    }
    __syncthreads();
  }
  T* C = static_cast<T*>(g.C);
  const int64_t ccol = (int64_t)grp * g.c_group_col;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int m = ty * 8 + i;
    if (m >= rows) continue;
    const int64_t crow = g.c_map ? g.c_map[row0 + m] : (row0 + m);
    const float scale = (EPI == EPI_STORE && row_scale) ? row_scale[row0 + m] : 1.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n >= g.N) continue;
      const int64_t o = crow * g.ldc + ccol + n;
      if (EPI == EPI_SWIGLU) {
        const float gv = acc[0][i][j], uv = acc[NB - 1][i][j];
        C[o] = from_f<T>(silu_f(gv) * uv);
        if (g.Gs) static_cast<T*>(g.Gs)[o] = from_f<T>(gv);
        if (g.Us) static_cast<T*>(g.Us)[o] = from_f<T>(uv);
      } else {
        C[o] = from_f<T>(acc[0][i][j] * scale);
      }
    }
  }
}

// =============================================================== host launch
static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// MFMA kernels use 256-row M tiles (the routed schedule height): the
// persistent eight-wave kernel of gemm_qp.hip (K slabs of 64 streamed by
// direct loads) wherever its constraints hold, else gemm_mfma_kernel with 8
// waves (4 x 2), per wave 2 x 2 tiles (SwiGLU: x2) or 2 x 4 (store).
constexpr int MF_BM = 256;

// The MFMA kernel needs bf16, 16-byte aligned operands and strides, K and the
// K segment multiples of 64, N a multiple of 4 and 8-byte aligned output rows.
static bool mfma_ok(const GemmDesc& g) {
  return g.K % MF_K == 0 && g.kseg % MF_K == 0 && g.lda % 8 == 0 && g.ldb % 8 == 0 && g.N % 4 == 0 &&
         g.ldc % 4 == 0 && g.c_group_col % 4 == 0 && aligned16(g.A) && ((reinterpret_cast<uintptr_t>(g.C) & 7) == 0);
}

bool gemm_mfma_eligible(const GemmDesc& g, int dtype, bool allow_mfma) {
  return dtype == DSMOE_BF16 && allow_mfma && mfma_ok(g);
}

int gemm_tile_m(bool mfma) { return mfma ? MF_BM : TILE_M; }

static int64_t grid_for(const GemmDesc& g, int bm, int tile_n) {
  const int64_t m_bound = g.sched ? g.m_tiles_bound : cdiv(g.dense_rows, bm) * g.groups;
  const int64_t total = m_bound * cdiv(g.N, tile_n);
  return 8 * cdiv(total, 8);
}

template <int EPI, int WM, int WN, int TM, int TN>
static int launch_mfma_t(const GemmDesc& g, const float* row_scale, hipStream_t st) {
  using CF = MfCfg<EPI, WM, WN, TM, TN>;
  static_assert(CF::BM == MF_BM, "schedule height");
  const int64_t grid = grid_for(g, CF::BM, CF::BN);
  if (grid == 0) return DSMOE_OK;
  auto kern = gemm_mfma_kernel<EPI, WM, WN, TM, TN>;
  static const hipError_t attr =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)CF::LDS_BYTES);
  if (attr != hipSuccess) return fail(DSMOE_ERR_HIP, "gemm: cannot raise LDS limit");
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(CF::THREADS), CF::LDS_BYTES, st, g, row_scale);
  return check_launch("gemm_mfma");
}

int launch_grouped_gemm(const GemmDesc& g_in, int epi, int dtype, const float* row_scale, bool allow_mfma,
                        hipStream_t st) {
  const GemmDesc& g = g_in;
  if (g.N <= 0 || g.K <= 0) return DSMOE_OK;
  if (gemm_mfma_eligible(g, dtype, allow_mfma)) {
    if (g.bm != MF_BM) return fail(DSMOE_ERR_INVALID, "gemm: schedule tile height does not match the MFMA kernel");
    if (gemm_qp_ok(g)) return launch_gemm_qp(g, epi, row_scale, st);
    // shapes the persistent kernel does not take (N % 8 == 4, more than two K
    // segments, 8-byte aligned output): the register-staged 8-wave kernel
    if (epi == EPI_SWIGLU) return launch_mfma_t<EPI_SWIGLU, 4, 2, 2, 2>(g, row_scale, st);
    return launch_mfma_t<EPI_STORE, 4, 2, 2, 4>(g, row_scale, st);
  }
  if (g.bm != TILE_M) return fail(DSMOE_ERR_INVALID, "gemm: schedule tile height does not match the SIMT kernel");
  const int64_t grid = grid_for(g, TILE_M, SM_N);
  if (grid == 0) return DSMOE_OK;
  if (dtype == DSMOE_BF16) {
    if (epi == EPI_SWIGLU)
      hipLaunchKernelGGL((gemm_simt_kernel<bf16_t, EPI_SWIGLU>), dim3((unsigned)grid), dim3(256), 0, st, g, row_scale);
    else
      hipLaunchKernelGGL((gemm_simt_kernel<bf16_t, EPI_STORE>), dim3((unsigned)grid), dim3(256), 0, st, g, row_scale);
  } else {
    if (epi == EPI_SWIGLU)
      hipLaunchKernelGGL((gemm_simt_kernel<float, EPI_SWIGLU>), dim3((unsigned)grid), dim3(256), 0, st, g, row_scale);
    else
      hipLaunchKernelGGL((gemm_simt_kernel<float, EPI_STORE>), dim3((unsigned)grid), dim3(256), 0, st, g, row_scale);
  }
  return check_launch("gemm_simt");
}

int launch_grouped_gemm_pair(const GemmDesc& gr_in, const GemmDesc& gd_in, int epi, int dtype, const float* row_scale,
                             bool allow_mfma_r, bool allow_mfma_d, hipStream_t st) {
  const GemmDesc &gr = gr_in, &gd = gd_in;
  const bool one = gd.sched == nullptr && gr.N > 0 && gr.K > 0 && gd.N > 0 &&
                   gd.K > 0 && gemm_mfma_eligible(gr, dtype, allow_mfma_r) && gemm_mfma_eligible(gd, dtype, allow_mfma_d) &&
                   gemm_qp_ok(gr) && gemm_qp_ok(gd);
  if (one) return launch_gemm_qp_pair(gr, gd, epi, row_scale, st);
  const int rc = launch_grouped_gemm(gr_in, epi, dtype, row_scale, allow_mfma_r, st);
  if (rc) return rc;
  return launch_grouped_gemm(gd_in, epi, dtype, nullptr, allow_mfma_d, st);
}

}  // namespace dsmoe
