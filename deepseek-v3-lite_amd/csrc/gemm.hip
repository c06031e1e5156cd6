// (c) Grouped expert GEMMs over expert-sorted rows.
//
// C[cmap(r)][n] = epilogue( sum_k A[amap(r)][k] * B_g[n][k] ), both operands
// K-contiguous ("NT"), as nn.Linear stores x and W.  Restates the per-expert
// GEMMs of models/moe.py:127-131 (gate/up fused with silu*mul, then down) and
// the grouped operator of models/moe_triton.py:28-51,57-135.
//
// Work split: a launch enumerates (M tile, N tile) pairs, N fastest.  M tiles
// come from the device-side schedule the permute scan writes (one entry per
// 128-row tile inside each expert, so skewed loads simply produce more tiles
// for the hot experts) or are dense (shared experts: every group covers all
// rows).  Block b runs on XCD b % 8; each XCD takes one contiguous eighth of
// the tile list so the weight tiles of an expert stay in that XCD's L2.  The
// grid is sized from a host bound; blocks past the device count exit.
//
// Kernels:
//   gemm_mfma_kernel  bf16, gfx950 v_mfma_f32_32x32x16_bf16, 128x128x64
//                     block tile (x2 B operands for SwiGLU), 4 waves (2x2,
//                     64x64 each), LDS double buffer with XOR-swizzled 16-byte
//                     chunks, global prefetch of the next K slab in registers.
//   gemm_simt_kernel  fp32 FMA fallback for fp32 and for shapes the MFMA
//                     kernel does not take (any N, K, strides).
#include "common.h"

namespace dsmoe {

// ----------------------------------------------------------------- tile lookup
__device__ __forceinline__ bool tile_for_block(const GemmDesc& g, int n_tiles, int& grp, int& row0, int& rows,
                                               int& n_tile) {
  int64_t m_total;
  int tpg = 0;
  if (g.sched) {
    m_total = *g.sched_count;
  } else {
    tpg = (int)cdiv(g.dense_rows, TILE_M);
    m_total = (int64_t)tpg * g.groups;
  }
  const int64_t total = m_total * n_tiles;
  const int64_t per_xcd = cdiv(total, 8);
  const int64_t j = blockIdx.x >> 3;
  if (j >= per_xcd) return false;
  const int64_t lin = (int64_t)(blockIdx.x & 7) * per_xcd + j;
  if (lin >= total) return false;
  const int64_t m_tile = lin / n_tiles;
  n_tile = (int)(lin - m_tile * n_tiles);
  if (g.sched) {
    const MTile t = g.sched[m_tile];
    grp = t.group;
    row0 = t.row0;
    rows = t.rows;
  } else {
    grp = (int)(m_tile / tpg);
    const int mt = (int)(m_tile - (int64_t)grp * tpg);
    row0 = mt * TILE_M;
    rows = min(TILE_M, g.dense_rows - row0);
  }
  return true;
}

// =============================================================== MFMA kernel
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

constexpr int MF_N = 128;
constexpr int MF_K = 64;
constexpr int MF_THREADS = 256;

__device__ __forceinline__ int swz(int row, int chunk) { return row * MF_K + ((chunk ^ (row & 7)) << 3); }

template <int EPI>
__global__ __launch_bounds__(MF_THREADS) void gemm_mfma_kernel(const GemmDesc g, const float* __restrict__ row_scale) {
  constexpr int NB = (EPI == EPI_SWIGLU) ? 2 : 1;
  constexpr int A_EL = TILE_M * MF_K;
  constexpr int B_EL = MF_N * MF_K;
  constexpr int STAGE = A_EL + NB * B_EL;
  extern __shared__ __attribute__((aligned(16))) bf16_t smem_mf[];

  const int n_tiles = (int)cdiv(g.N, MF_N);
  int grp, row0, rows, n_tile;
  if (!tile_for_block(g, n_tiles, grp, row0, rows, n_tile)) return;
  const int n0 = n_tile * MF_N;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // ---- global -> register assignment: chunk lc (16 bytes) of rows lr + 32*i
  const int lc = tid & 7;
  const int lr = tid >> 3;
  const bf16_t* A = static_cast<const bf16_t*>(g.A);
  const bf16_t* a_src[4];
  bool a_ok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = lr + 32 * i;
    a_ok[i] = r < rows;
    int64_t arow = 0;
    if (a_ok[i]) arow = g.a_map ? g.a_map[row0 + r] : (row0 + r);
    a_src[i] = A + arow * g.lda + lc * 8;
  }
  bool b_ok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) b_ok[i] = (n0 + lr + 32 * i) < g.N;

  uint4 ra[4];
  uint4 rb[NB][4];
  const uint4 z4 = make_uint4(0, 0, 0, 0);

  auto gload = [&](int kb) {
    const int k0 = kb * MF_K;
    const int seg = k0 / g.kseg;
    const int kin = k0 - seg * g.kseg;
#pragma unroll
    for (int i = 0; i < 4; ++i) ra[i] = a_ok[i] ? *reinterpret_cast<const uint4*>(a_src[i] + k0) : z4;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const bf16_t* base = static_cast<const bf16_t*>((b == 0 ? g.B0 : g.B1)[grp * g.nseg + seg]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        rb[b][i] = b_ok[i] ? *reinterpret_cast<const uint4*>(base + (int64_t)(n0 + lr + 32 * i) * g.ldb + kin + lc * 8)
                           : z4;
    }
  };
  auto lstore = [&](int stage) {
    bf16_t* sA = smem_mf + stage * STAGE;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(sA + swz(lr + 32 * i, lc)) = ra[i];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      bf16_t* sB = sA + A_EL + b * B_EL;
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(sB + swz(lr + 32 * i, lc)) = rb[b][i];
    }
  };

  f32x16_t acc[NB][2][2];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[b][mi][ni][r] = 0.0f;

  const int nk = g.K / MF_K;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int kb = 0; kb < nk; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nk) gload(kb + 1);
    const bf16_t* sA = smem_mf + cur * STAGE;
#pragma unroll
    for (int kk = 0; kk < MF_K / 16; ++kk) {
      const int c = kk * 2 + (lane >> 5);
      bf16x8_t af[2];
#pragma unroll
      for (int mi = 0; mi < 2; ++mi) {
        const int r = wm * 64 + mi * 32 + (lane & 31);
        af[mi] = *reinterpret_cast<const bf16x8_t*>(sA + swz(r, c));
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const bf16_t* sB = sA + A_EL + b * B_EL;
        bf16x8_t bfr[2];
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
          const int n = wn * 64 + ni * 32 + (lane & 31);
          bfr[ni] = *reinterpret_cast<const bf16x8_t*>(sB + swz(n, c));
        }
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int ni = 0; ni < 2; ++ni)
            acc[b][mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[ni], af[mi], acc[b][mi][ni], 0, 0, 0);
      }
    }
    if (kb + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue.  Lane holds row m = .. + (lane & 31) and, per q, columns
  // n = .. + 8q + 4*(lane >> 5) + {0..3} (acc registers 4q..4q+3).
  bf16_t* C = static_cast<bf16_t*>(g.C);
  const int64_t ccol = (int64_t)grp * g.c_group_col;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
    const int m = wm * 64 + mi * 32 + (lane & 31);
    if (m >= rows) continue;
    const int64_t crow = g.c_map ? g.c_map[row0 + m] : (row0 + m);
    float scale = 1.0f;
    if (EPI == EPI_STORE && row_scale) scale = row_scale[row0 + m];
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0 + wn * 64 + ni * 32 + q * 8 + (lane >> 5) * 4;
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
  if (!tile_for_block(g, n_tiles, grp, row0, rows, n_tile)) return;
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

// The MFMA kernel needs bf16, 16-byte aligned operands and strides, K and the
// K segment multiples of 64, N a multiple of 4 and 8-byte aligned output rows.
static bool mfma_ok(const GemmDesc& g) {
  return g.K % MF_K == 0 && g.kseg % MF_K == 0 && g.N % 4 == 0 && g.lda % 8 == 0 && g.ldb % 8 == 0 &&
         g.ldc % 4 == 0 && g.c_group_col % 4 == 0 && aligned16(g.A) && ((reinterpret_cast<uintptr_t>(g.C) & 7) == 0);
}

static int64_t grid_for(const GemmDesc& g, int tile_n) {
  const int64_t m_bound = g.sched ? g.m_tiles_bound : cdiv(g.dense_rows, TILE_M) * g.groups;
  const int64_t total = m_bound * cdiv(g.N, tile_n);
  return 8 * cdiv(total, 8);
}

int launch_grouped_gemm(const GemmDesc& g, int epi, int dtype, const float* row_scale, bool allow_mfma,
                        hipStream_t st) {
  if (g.N <= 0 || g.K <= 0) return DSMOE_OK;
  if (dtype == DSMOE_BF16 && allow_mfma && mfma_ok(g)) {
    const int64_t grid = grid_for(g, MF_N);
    if (grid == 0) return DSMOE_OK;
    if (epi == EPI_SWIGLU) {
      const size_t lds = 2 * sizeof(bf16_t) * (TILE_M * MF_K + 2 * MF_N * MF_K);
      static bool attr = false;
      if (!attr) {
        if (hipFuncSetAttribute((const void*)gemm_mfma_kernel<EPI_SWIGLU>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess)
          return fail(DSMOE_ERR_HIP, "gemm: cannot raise LDS limit");
        attr = true;
      }
      hipLaunchKernelGGL(gemm_mfma_kernel<EPI_SWIGLU>, dim3((unsigned)grid), dim3(MF_THREADS), lds, st, g, row_scale);
    } else {
      const size_t lds = 2 * sizeof(bf16_t) * (TILE_M * MF_K + MF_N * MF_K);
      hipLaunchKernelGGL(gemm_mfma_kernel<EPI_STORE>, dim3((unsigned)grid), dim3(MF_THREADS), lds, st, g, row_scale);
    }
    return check_launch("gemm_mfma");
  }
  const int64_t grid = grid_for(g, SM_N);
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

}  // namespace dsmoe
