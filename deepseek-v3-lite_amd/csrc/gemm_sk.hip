// (c) Grouped NT GEMM for few rows per group: the decode shape (C3 at 64
// tokens: ~6 routed rows per expert, 64 shared rows).  There the layer is a
// weight stream (every expert's W1, W3 and W2 is read once, 1.14 GB at C3)
// and the bound is HBM bandwidth, not MFMA rate.
//
// A block owns one row tile (at most SK_BM = 64 rows of one group) and BN
// output columns (SwiGLU: 32 columns of h, i.e. 32 rows each of W1 and W3;
// store: 64 rows of W).  Its four waves split K into quarters, so every
// weight element is loaded exactly once, straight into registers (no LDS
// staging: each element feeds one MFMA per 16-row tile of the block).  A wave
// keeps SK_PD K steps of 32 in flight (4 x 16-byte loads per lane and step for
// the weights, plus one per 16-row tile for the activation rows, which are
// L2 hits).  MFMA v_mfma_f32_16x16x32_bf16 with the activation rows as the
// 16-row operand: lane l holds row l & 15 (A) / weight row l & 15 (B) and K
// elements 8 (l >> 4) .. + 7 of the step.  The four K-quarter partial sums
// meet in LDS and are added in wave order (w0 + w1) + w2 + w3, then the
// epilogue (SwiGLU or store, optional row scale, output row map) writes
// 16-byte chunks.
//
// Tile enumeration (gemm_tile.h) and GemmDesc contract as in gemm.hip, with row tiles of
// SK_BM rows (the routed schedule must be built with bm = SK_BM).
#include "gemm_tile.h"
#include "mfma.h"

namespace dsmoe {

constexpr int SK_KSTEP = 32;
constexpr int SK_PD = 4;       // K steps in flight per wave
constexpr int SK_CG = 4;       // 16-column groups per wave (SwiGLU: W1 x 2, W3 x 2)
constexpr int SK_MT_MAX = SK_BM / 16;

template <int EPI>
struct SKCfg {
  static constexpr int BN = (EPI == EPI_SWIGLU) ? 32 : 64;  // output columns per block
};

typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

// LDS: partial sums red[wave][cg][mt][lane][4] (64 KB at MT = 4).
constexpr size_t SK_LDS = (size_t)4 * SK_CG * SK_MT_MAX * 64 * 4 * sizeof(float);

__device__ __forceinline__ float sk_red(const float* red, int mt_n, int w, int cg, int mt, int r, int c) {
  // element (row r, col c) of a 16 x 16 MFMA tile: lane c + 16 (r >> 2), register r & 3
  return red[(((w * SK_CG + cg) * mt_n + mt) * 64 + c + 16 * (r >> 2)) * 4 + (r & 3)];
}

template <int EPI, int MT>
__device__ __forceinline__ void sk_tile(const GemmDesc& g, const float* __restrict__ row_scale, int grp, int row0,
                                        int rows, int n_tile) {
  constexpr int BN = SKCfg<EPI>::BN;
  extern __shared__ __attribute__((aligned(16))) float sk_smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n0 = n_tile * BN;

  // weight rows of this lane, per column group and K segment
  const bf16_t* bp[SK_CG][2];
#pragma unroll
  for (int cg = 0; cg < SK_CG; ++cg) {
    const bool w3 = (EPI == EPI_SWIGLU) && cg >= 2;
    const int col = (EPI == EPI_SWIGLU) ? n0 + 16 * (cg & 1) + (lane & 15) : n0 + 16 * cg + (lane & 15);
    const int64_t roff = (int64_t)min(col, g.N - 1) * g.ldb + (lane >> 4) * 8;
    const void* const* tab = (w3 ? g.B1 : g.B0) + (int64_t)grp * g.nseg;
    bp[cg][0] = static_cast<const bf16_t*>(tab[0]) + roff;
    bp[cg][1] = static_cast<const bf16_t*>(tab[g.nseg - 1]) + roff;
  }
  const int kseg = g.nseg > 1 ? g.kseg : 0x7fffffff;
  // activation rows of this lane, per 16-row tile (rows past the tile repeat its last row)
  const bf16_t* ap[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int r = min(16 * mt + (lane & 15), rows - 1);
    const int64_t arow = g.a_map ? (int64_t)g.a_map[row0 + r] : (int64_t)(row0 + r);
    ap[mt] = static_cast<const bf16_t*>(g.A) + arow * g.lda + (lane >> 4) * 8;
  }

  const int per = g.K / (4 * SK_KSTEP);   // K steps of this wave
  const int kb = wave * per;
  u32x4_t wbuf[SK_PD][SK_CG], abuf[SK_PD][MT];
  f32x4_t acc[SK_CG][MT];
#pragma unroll
  for (int cg = 0; cg < SK_CG; ++cg)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[cg][mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  auto load = [&](int buf, int s) {
    const int k0 = (kb + s) * SK_KSTEP;
    const bool hi = k0 >= kseg;
    const int kin = hi ? k0 - kseg : k0;
#pragma unroll
    for (int cg = 0; cg < SK_CG; ++cg) wbuf[buf][cg] = ldg16((hi ? bp[cg][1] : bp[cg][0]) + kin);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) abuf[buf][mt] = ldg16(ap[mt] + k0);
  };
#pragma unroll
  for (int p = 0; p < SK_PD; ++p)
    if (p < per) load(p, p);
  for (int s0 = 0; s0 < per; s0 += SK_PD) {
#pragma unroll
    for (int p = 0; p < SK_PD; ++p) {
      const int s = s0 + p;
      if (s < per) {
#pragma unroll
        for (int cg = 0; cg < SK_CG; ++cg)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[cg][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, abuf[p][mt]),
                                                                  __builtin_bit_cast(bf16x8_t, wbuf[p][cg]),
                                                                  acc[cg][mt], 0, 0, 0);
        if (s + SK_PD < per) load(p, s + SK_PD);
      }
    }
  }

  // K-quarter partial sums -> LDS
  float* red = sk_smem;
#pragma unroll
  for (int cg = 0; cg < SK_CG; ++cg)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      *reinterpret_cast<f32x4_t*>(red + (((wave * SK_CG + cg) * MT + mt) * 64 + lane) * 4) = acc[cg][mt];
  __syncthreads();

  // epilogue: thread -> (row, 8 consecutive columns)
  constexpr int TPR = BN / 8;              // threads per row
  constexpr int RPP = 256 / TPR;           // rows per pass
  const int c8 = 8 * (tid % TPR);
  const int64_t ccol = (int64_t)grp * g.c_group_col;
  bf16_t* C = static_cast<bf16_t*>(g.C);
  for (int r = tid / TPR; r < rows; r += RPP) {
    const int mt = r >> 4, rl = r & 15;
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = c8 + i;
      const int cg = c >> 4, cl = c & 15;
      float a0 = sk_red(red, MT, 0, cg, mt, rl, cl);
      a0 += sk_red(red, MT, 1, cg, mt, rl, cl);
      a0 += sk_red(red, MT, 2, cg, mt, rl, cl);
      a0 += sk_red(red, MT, 3, cg, mt, rl, cl);
      if (EPI == EPI_SWIGLU) {
        float a1 = sk_red(red, MT, 0, cg + 2, mt, rl, cl);
        a1 += sk_red(red, MT, 1, cg + 2, mt, rl, cl);
        a1 += sk_red(red, MT, 2, cg + 2, mt, rl, cl);
        a1 += sk_red(red, MT, 3, cg + 2, mt, rl, cl);
        v[i] = a0 * __builtin_amdgcn_rcpf(1.0f + __expf(-a0)) * a1;
      } else {
        v[i] = a0;
      }
    }
    if (EPI == EPI_STORE && row_scale) {
      const float sc = row_scale[row0 + r];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] *= sc;
    }
    const int n = n0 + c8;
    if (n < g.N) {
      const int64_t crow = g.c_map ? (int64_t)g.c_map[row0 + r] : (int64_t)(row0 + r);
      u32x4_t o;
      o.x = pack_bf16x2(v[0], v[1]);
      o.y = pack_bf16x2(v[2], v[3]);
      o.z = pack_bf16x2(v[4], v[5]);
      o.w = pack_bf16x2(v[6], v[7]);
      *reinterpret_cast<u32x4_t*>(C + crow * g.ldc + ccol + n) = o;
    }
  }
}

// One launch computes g0 alone (pair = 0), or g0 and the dense problem g1
// side by side (pair = 1); row_scale applies to g0's rows only.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_sk_kernel(const GemmDesc g0, const GemmDesc g1, const int pair,
                                                      const float* __restrict__ row_scale_0) {
  constexpr int BN = SKCfg<EPI>::BN;
  int which = 0, grp, row0, rows, n_tile;
  if (pair) {
    if (!tile_for_block_pair<SK_BM>(g0, g1, BN, which, grp, row0, rows, n_tile)) return;
  } else {
    if (!tile_for_block<SK_BM>(g0, (int)cdiv(g0.N, BN), grp, row0, rows, n_tile)) return;
  }
  which = __builtin_amdgcn_readfirstlane(which);
  grp = __builtin_amdgcn_readfirstlane(grp);
  row0 = __builtin_amdgcn_readfirstlane(row0);
  rows = __builtin_amdgcn_readfirstlane(rows);
  n_tile = __builtin_amdgcn_readfirstlane(n_tile);
  if (rows <= 0) return;
  const GemmDesc& g = which ? g1 : g0;
  const float* row_scale = which ? nullptr : row_scale_0;
  switch ((rows + 15) >> 4) {
    case 1: sk_tile<EPI, 1>(g, row_scale, grp, row0, rows, n_tile); break;
    case 2: sk_tile<EPI, 2>(g, row_scale, grp, row0, rows, n_tile); break;
    case 3: sk_tile<EPI, 3>(g, row_scale, grp, row0, rows, n_tile); break;
    default: sk_tile<EPI, 4>(g, row_scale, grp, row0, rows, n_tile); break;
  }
}

// ---------------------------------------------------------------- host side
bool gemm_sk_ok(const GemmDesc& g) {
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool rows_ok = g.sched ? g.bm == SK_BM : g.dense_rows >= 0;
  return rows_ok && g.nseg >= 1 && g.nseg <= 2 && g.K > 0 && g.K % (4 * SK_KSTEP) == 0 && g.kseg % SK_KSTEP == 0 &&
         g.N > 0 && g.N % 8 == 0 && g.lda % 8 == 0 && g.ldb % 8 == 0 && g.ldc % 8 == 0 && g.c_group_col % 8 == 0 &&
         a16(g.A) && a16(g.C) && g.Gs == nullptr && g.Us == nullptr;
}

static int64_t sk_mtiles(const GemmDesc& g) {
  return g.sched ? g.m_tiles_bound : cdiv(g.dense_rows, SK_BM) * g.groups;
}

template <int EPI>
static int sk_launch(const GemmDesc& g0, const GemmDesc& g1, int pair, const float* row_scale, int64_t grid,
                     hipStream_t st) {
  if (grid == 0) return DSMOE_OK;
  static_assert(SK_LDS <= 64 * 1024, "default LDS limit");
  hipLaunchKernelGGL(gemm_sk_kernel<EPI>, dim3((unsigned)grid), dim3(256), SK_LDS, st, g0, g1, pair, row_scale);
  return check_launch("gemm_sk");
}

int launch_gemm_sk(const GemmDesc& g, int epi, const float* row_scale, hipStream_t st) {
  const int bn = (epi == EPI_SWIGLU) ? SKCfg<EPI_SWIGLU>::BN : SKCfg<EPI_STORE>::BN;
  const int64_t grid = 8 * cdiv(sk_mtiles(g) * cdiv(g.N, bn), 8);
  return epi == EPI_SWIGLU ? sk_launch<EPI_SWIGLU>(g, g, 0, row_scale, grid, st)
                           : sk_launch<EPI_STORE>(g, g, 0, row_scale, grid, st);
}

int launch_gemm_sk_pair(const GemmDesc& gr, const GemmDesc& gd, int epi, const float* row_scale, hipStream_t st) {
  const int bn = (epi == EPI_SWIGLU) ? SKCfg<EPI_SWIGLU>::BN : SKCfg<EPI_STORE>::BN;
  const int64_t td = sk_mtiles(gd) * cdiv(gd.N, bn), tr = sk_mtiles(gr) * cdiv(gr.N, bn);
  const int64_t grid = 8 * (cdiv(td, 8) + cdiv(tr, 8));
  return epi == EPI_SWIGLU ? sk_launch<EPI_SWIGLU>(gr, gd, 1, row_scale, grid, st)
                           : sk_launch<EPI_STORE>(gr, gd, 1, row_scale, grid, st);
}

}  // namespace dsmoe
