// LDS slab layout, MFMA fragment reads and the MFMA step of the eight-wave
// ping-pong grouped GEMM for gfx950 (gemm_qp.hip).  A slab is 64 K of 256 A
// rows and 256 B rows, 128 bytes per LDS row (one cache line) with the
// 16-byte chunk index c of row r stored at c ^ ((r >> 1) & 7), so the 16 rows
// read at one logical chunk by a fragment load (16 lanes per LDS cycle) land
// on 16 distinct bank groups.  Each wave owns a 128 x 64 block of the
// 256 x 256 tile (row group wm, column group cg) as 4 x 2 tiles of
// v_mfma_f32_32x32x16_bf16, with the weights as the A operand (a lane holds one
// output row and four consecutive columns per 32-column tile), and holds a
// whole slab of fragments (96 registers) so it can run a slab's 32 MFMAs back
// to back.
#pragma once

#include "gemm_tile.h"
#include "mfma.h"

namespace dsmoe {

constexpr int QW_BM = 256;
constexpr int QW_BK = 64;                             // K per slab
constexpr int QW_ROWB = QW_BK * 2;                    // bytes per LDS row (one cache line)
constexpr int QW_REG = 256 * QW_ROWB;                 // one operand of a slab (32 KB)
constexpr int QW_ASLOTS = 2;                          // A ring (activations: L2 / MALL hits)
constexpr int QW_BSLOTS = 3;                          // B ring (weights: streamed from HBM)
constexpr int QW_BOFF = QW_ASLOTS * QW_REG;           // B ring after the A ring
constexpr size_t QW_LDS = (size_t)(QW_ASLOTS + QW_BSLOTS) * QW_REG;  // 160 KB (the epilogue reuses it)
constexpr int QW_LD = 8;                              // 1 KB direct loads per loading wave and slab
constexpr int QW_THREADS = 512;
constexpr int QW_MAX_SEG = 2;                         // K segments of B (shared experts summed in one GEMM)

__device__ __forceinline__ int qw_swz(int r, int c) { return r * QW_ROWB + ((c ^ ((r >> 1) & 7)) << 4); }

template <int EPI>
struct QWCfg {
  static constexpr int NB = (EPI == EPI_SWIGLU) ? 2 : 1;      // B operands (W1, W3)
  static constexpr int TN = (EPI == EPI_SWIGLU) ? 1 : 2;      // 32-column tiles per wave and operand
  static constexpr int BN = (EPI == EPI_SWIGLU) ? 128 : 256;  // output columns per tile
};

// A wave's fragments of one slab: per K step, A sub-tiles j (rows
// (2j + wm) * 32 ..) and its B tiles (column group cg).
template <int EPI>
struct QWFrag {
  bf16x8_t fa[4][4];
  bf16x8_t fb[4][QWCfg<EPI>::NB][QWCfg<EPI>::TN];
};

template <int EPI, int NMI>
__device__ __forceinline__ void qw_read(QWFrag<EPI>& F, int kb, int wm, int cg, int lane) {
  using CF = QWCfg<EPI>;
  extern __shared__ __attribute__((aligned(16))) char qw_smem[];
  if (NMI == 0) return;
  const char* sA = qw_smem + (kb & 1) * QW_REG;
  const char* sB = qw_smem + QW_BOFF + (kb % QW_BSLOTS) * QW_REG;
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const int c = st * 2 + (lane >> 5);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      F.fa[st][j] = j < NMI ? *reinterpret_cast<const bf16x8_t*>(sA + qw_swz((2 * j + wm) * 32 + (lane & 31), c))
                            : __builtin_nondeterministic_value(F.fa[st][j]);  // unused: not kept live
#pragma unroll
    for (int b = 0; b < CF::NB; ++b)
#pragma unroll
      for (int ni = 0; ni < CF::TN; ++ni) {
        // SwiGLU: W1 rows 0..127, the same W3 rows at 128..255
        const int r = (CF::NB == 2 ? b * 128 + cg * 32 : cg * 64 + ni * 32) + (lane & 31);
        F.fb[st][b][ni] = *reinterpret_cast<const bf16x8_t*>(sB + qw_swz(r, c));
      }
  }
}

template <int EPI, int NMI>
__device__ __forceinline__ void qw_mma(const QWFrag<EPI>& F, f32x16_t (&acc)[QWCfg<EPI>::NB][4][QWCfg<EPI>::TN]) {
  using CF = QWCfg<EPI>;
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int j = 0; j < NMI; ++j)
#pragma unroll
      for (int b = 0; b < CF::NB; ++b)
#pragma unroll
        for (int ni = 0; ni < CF::TN; ++ni)
          acc[b][j][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F.fb[st][b][ni], F.fa[st][j], acc[b][j][ni], 0, 0, 0);
}

__device__ __forceinline__ void qw_sync() {
  __builtin_amdgcn_sched_barrier(0);
  lds_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// The same fragment reads with the number of active A sub-tiles given at run
// time (the first slab of the next tile, read at a tile boundary).
template <int EPI>
__device__ __forceinline__ void qw_read_rt(QWFrag<EPI>& F, int kb, int nmi, int wm, int cg, int lane) {
  using CF = QWCfg<EPI>;
  extern __shared__ __attribute__((aligned(16))) char qw_smem[];
  if (nmi == 0) return;
  const char* sA = qw_smem + (kb & 1) * QW_REG;
  const char* sB = qw_smem + QW_BOFF + (kb % QW_BSLOTS) * QW_REG;
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const int c = st * 2 + (lane >> 5);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      F.fa[st][j] = j < nmi ? *reinterpret_cast<const bf16x8_t*>(sA + qw_swz((2 * j + wm) * 32 + (lane & 31), c))
                            : __builtin_nondeterministic_value(F.fa[st][j]);
#pragma unroll
    for (int b = 0; b < CF::NB; ++b)
#pragma unroll
      for (int ni = 0; ni < CF::TN; ++ni) {
        const int r = (CF::NB == 2 ? b * 128 + cg * 32 : cg * 64 + ni * 32) + (lane & 31);
        F.fb[st][b][ni] = *reinterpret_cast<const bf16x8_t*>(sB + qw_swz(r, c));
      }
  }
}

// qw_mma for a tile's first slab: the accumulators start from zero.
template <int EPI, int NMI>
__device__ __forceinline__ void qw_mma_first(const QWFrag<EPI>& F,
                                             f32x16_t (&acc)[QWCfg<EPI>::NB][4][QWCfg<EPI>::TN]) {
  using CF = QWCfg<EPI>;
  const f32x16_t zero = {};
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int j = 0; j < NMI; ++j)
#pragma unroll
      for (int b = 0; b < CF::NB; ++b)
#pragma unroll
        for (int ni = 0; ni < CF::TN; ++ni)
          acc[b][j][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F.fb[st][b][ni], F.fa[st][j],
                                                                  st == 0 ? zero : acc[b][j][ni], 0, 0, 0);
}

// Active 32-row A sub-tiles of a wave in row group wm: j with (2j + wm) * 32 < rows.
__device__ __forceinline__ int qw_nmi(int rows, int wm) {
  const int nsub = (rows + 31) >> 5;
  return max(0, min(4, (nsub - wm + 1) >> 1));
}

}  // namespace dsmoe
