// (c) Grouped NT GEMM for gfx950: four waves, one per SIMD, each owning a
// 128 x 128 block of the 256 x 256 output tile, fed from LDS slabs that
// stream in with direct global->LDS loads.
//
// Same contract and tile enumeration as gemm_mfma_kernel (gemm.hip).  The
// shape follows from gfx950 limits measured on MI355X:
//  * 512 VGPRs per lane: a 128 x 128 wave tile (256 accumulator registers)
//    is the largest a wave can hold, and it reads the fewest LDS bytes per
//    MFMA (8 fragments per 16 MFMAs).  It leaves room for one wave per SIMD.
//  * L2 -> LDS direct loads move whole 128-byte rows best, so K advances in
//    slabs of 64 bf16 (one cache line per row and operand).
//  * 160 KB of LDS: a slab is 32 KB per operand (256 rows of 128 bytes).  A
//    (activation rows, mostly L2 / MALL hits) cycles through a ring of two
//    slots, B (weights, streamed from HBM) through a ring of three.
//
// Per slab kb a wave runs four 16-wide K steps.  Fragments are read two steps
// ahead of their MFMAs through three register sets, so LDS latency hides
// behind MFMAs.  After the MFMAs of step 1 each wave waits for its LDS reads
// of slab kb and its own direct loads of slab kb + 1; the workgroup barrier
// then makes slab kb + 1 visible and frees slab kb's slots.  The refills of
// slab kb + 2 are spread over the whole slab: B(kb + 2) during steps 0 and 1
// (into slab kb - 1's slot, freed by the previous barrier), A(kb + 2) during
// steps 2 and 3, four loads per step, one after every fourth MFMA.  Loads are
// addressed as a wave-uniform base in SGPRs plus 32-bit per-lane offsets.
// Loads past the last slab re-read the last slab into the free slot (never
// read), so the loop body has no branches and the wait counts stay exact;
// they are drained before the epilogue.
//
// Ragged tiles: the wave in row group wm owns the 32-row sub-tiles wm,
// wm + 2, wm + 4 and wm + 6 of the block, so the valid rows of a partly
// filled tile are spread over all four SIMDs; a wave skips the MFMAs and A
// fragment reads of its sub-tiles past the valid rows (the main loop is
// instantiated for 0..4 active sub-tiles to stay branch-free).
//
// LDS rows are 128 bytes (8 chunks of 16 bytes); chunk c of row r is stored
// at chunk c ^ ((r >> 1) & 7), so the 16 rows read at one logical chunk by a
// fragment load (16 lanes per LDS cycle) land on 16 distinct bank groups.  A
// direct load writes 64 consecutive 16-byte chunks (lane i to chunk i) = 8
// rows, so each lane fetches the global chunk that belongs at its position.
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
constexpr int QW_LD = QW_REG / 1024 / 4;              // direct loads per wave, operand and slab (8)
constexpr int QW_MAX_SEG = 2;                         // K segments of B (shared experts summed in one GEMM)

__device__ __forceinline__ int qw_swz(int r, int c) { return r * QW_ROWB + ((c ^ ((r >> 1) & 7)) << 4); }

template <int EPI>
struct QWCfg {
  static constexpr int NB = (EPI == EPI_SWIGLU) ? 2 : 1;      // B operands
  static constexpr int TN = (EPI == EPI_SWIGLU) ? 2 : 4;      // 32-column tiles per wave and B operand
  static constexpr int BN = (EPI == EPI_SWIGLU) ? 128 : 256;  // output columns per block
};

// Direct-load sources of one wave (wave-uniform bases, per-lane byte
// offsets).  Wave w fills rows 64 w .. 64 w + 63 of both operand regions of
// a slab.
struct QWLoad {
  const char* a;           // A
  const char* b0;          // this wave's B table entry, K segment 0
  const char* b1;          // last K segment
  uint32_t offa[QW_LD];    // per-lane byte offsets of the 8 A loads
  uint32_t offb[QW_LD];    // and of the 8 B loads
  int kseg;                // K at which b1 takes over (0x7fffffff: one segment)
  int lds_off;             // byte offset of this wave's 8 KB inside an operand region
  int nk;                  // number of slabs
};

// Direct load i (0 .. 7) of this wave for A of slab ka (ring slot ka % 2) /
// for B of slab kb (slot kb % 3).  Past the last slab the last slab is
// reloaded into the (free) slot instead, so the loop body has no branches and
// the wait counts stay exact.
__device__ __forceinline__ void qw_load_a(const QWLoad& L, int ka, int i) {
  extern __shared__ __attribute__((aligned(16))) char qw_smem[];
  const uint32_t da = lds_addr(qw_smem) + L.lds_off + (ka & 1) * QW_REG;
  const int k0 = min(ka, L.nk - 1) * QW_BK;
  dma16s(L.a + 2 * k0, L.offa[i], da + i * 1024);
}

__device__ __forceinline__ void qw_load_b(const QWLoad& L, int kb, int i) {
  extern __shared__ __attribute__((aligned(16))) char qw_smem[];
  const uint32_t db = lds_addr(qw_smem) + L.lds_off + QW_BOFF + (kb % QW_BSLOTS) * QW_REG;
  const int k0 = min(kb, L.nk - 1) * QW_BK;
  const bool hi = k0 >= L.kseg;
  const char* src = hi ? L.b1 : L.b0;
  const int kin = hi ? k0 - L.kseg : k0;
  dma16s(src + 2 * kin, L.offb[i], db + i * 1024);
}

// Fragments of K step s (0..3) of slab kb: A sub-tiles j < NMI (rows
// (2j + wm) * 32 ..), B tiles of this wave's columns.
template <int EPI, int NMI>
__device__ __forceinline__ void qw_read(int kb, int s, int wm, int wn, int lane, bf16x8_t (&fa)[4],
                                        bf16x8_t (&fb)[QWCfg<EPI>::NB][QWCfg<EPI>::TN]) {
  using CF = QWCfg<EPI>;
  extern __shared__ __attribute__((aligned(16))) char qw_smem[];
  const char* sA = qw_smem + (kb & 1) * QW_REG;
  const char* sB = qw_smem + QW_BOFF + (kb % QW_BSLOTS) * QW_REG;
  const int c = s * 2 + (lane >> 5);
#pragma unroll
  for (int j = 0; j < NMI; ++j)
    fa[j] = *reinterpret_cast<const bf16x8_t*>(sA + qw_swz((2 * j + wm) * 32 + (lane & 31), c));
  if (NMI > 0) {
#pragma unroll
    for (int b = 0; b < CF::NB; ++b)
#pragma unroll
      for (int ni = 0; ni < CF::TN; ++ni) {
        const int r = (CF::NB == 2 ? b * 128 + wn * 64 : wn * 128) + ni * 32 + (lane & 31);
        fb[b][ni] = *reinterpret_cast<const bf16x8_t*>(sB + qw_swz(r, c));
      }
  }
}

// MFMAs T0 .. T1-1 of one K step (MMAS per step, in the order
// t = (j * NB + b) * TN + ni).  With NL > 0, load i of the step's NL direct
// loads (index LI0 + i of A (LK 0) or B (LK 1) of slab kl) follows MFMA
// floor(i * MMAS / NL), so the loads are spread evenly over the step.
template <int EPI, int NMI, int T0, int T1, int NL, int LK, int LI0>
__device__ __forceinline__ void qw_mma(const bf16x8_t (&fa)[4], const bf16x8_t (&fb)[QWCfg<EPI>::NB][QWCfg<EPI>::TN],
                                       f32x16_t (&acc)[QWCfg<EPI>::NB][4][QWCfg<EPI>::TN], const QWLoad& L, int kl) {
  using CF = QWCfg<EPI>;
  constexpr int MMAS = NMI * CF::NB * CF::TN;
#pragma unroll
  for (int t = T0; t < T1; ++t) {
    const int j = t / (CF::NB * CF::TN), b = (t / CF::TN) % CF::NB, ni = t % CF::TN;
    acc[b][j][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[b][ni], fa[j], acc[b][j][ni], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      if ((i * MMAS / (NL > 0 ? NL : 1)) == t) {
        __builtin_amdgcn_sched_barrier(0);
        if (LK == 0) qw_load_a(L, kl, LI0 + i); else qw_load_b(L, kl, LI0 + i);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

__device__ __forceinline__ void qw_sync() {
  __builtin_amdgcn_sched_barrier(0);
  lds_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// Fragment reads run two K steps ahead of their MFMAs through three register
// sets (step t of the kernel uses set t % 3; the four steps of a slab rotate
// through the sets, so the roles shift by one set per slab and the loop body
// covers three slabs).
template <int EPI, int NMI>
struct QWPipe {
  using CF = QWCfg<EPI>;
  bf16x8_t fa[3][4];
  bf16x8_t fb[3][CF::NB][CF::TN];
};

template <int EPI, int NMI, int SET>
__device__ __forceinline__ void qw_read_set(QWPipe<EPI, NMI>& P, int kb, int s, int wm, int wn, int lane) {
  qw_read<EPI, NMI>(kb, s, wm, wn, lane, P.fa[SET], P.fb[SET]);
}

// One slab; its step 0 uses register set S0 (steps use S0, S0+1, S0+2, S0
// mod 3).  On entry slab kb is visible to every wave and this wave's loads of
// A(kb + 1) and B(kb + 1) are in flight (older ones complete).
//
// The refill loads of slab kb + 2 are spread over the whole slab, four after
// every quarter of a K step's MFMAs: B(kb + 2) during steps 0 and 1 (its slot,
// that of slab kb - 1, was freed by the previous barrier) and A(kb + 2) during
// steps 2 and 3 (its slot is slab kb's, freed by this slab's barrier).  Load
// bursts stall the issuing wave while the L2 -> LDS path drains, and with one
// wave per SIMD a stalled wave idles its MFMA pipe; spread over all four steps
// the path runs at half the rate of a two-step spread.
//
// The barrier sits after step 1: by then every read of slab kb has been
// issued (steps 2 and 3 are read during steps 0 and 1); the wave waits for
// them and for its own loads of slab kb + 1 (only the 8 B(kb + 2) loads are
// younger), and after the barrier slab kb + 1 is visible and slab kb's slots
// are free.
template <int EPI, int NMI, int S0>
__device__ __forceinline__ void qw_slab(QWPipe<EPI, NMI>& P, const QWLoad& L, int kb, int wm, int wn, int lane,
                                        f32x16_t (&acc)[QWCfg<EPI>::NB][4][QWCfg<EPI>::TN]) {
  using CF = QWCfg<EPI>;
  constexpr int MMAS = NMI * CF::NB * CF::TN;  // MFMAs per K step
  constexpr int A0 = S0 % 3, A1 = (S0 + 1) % 3, A2 = (S0 + 2) % 3;
  constexpr int NL = QW_LD / 2;                // direct loads per K step
  // step 0: read step 2, B(kb + 2) loads 0-3
  __builtin_amdgcn_sched_barrier(0);
  qw_read_set<EPI, NMI, A2>(P, kb, 2, wm, wn, lane);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (MMAS > 0) {
    qw_mma<EPI, NMI, 0, MMAS, NL, 1, 0>(P.fa[A0], P.fb[A0], acc, L, kb + 2);
  } else {
#pragma unroll
    for (int i = 0; i < NL; ++i) qw_load_b(L, kb + 2, i);
  }
  // step 1: read step 3 (into the set step 0 just used), B(kb + 2) loads 4-7
  __builtin_amdgcn_sched_barrier(0);
  qw_read_set<EPI, NMI, A0>(P, kb, 3, wm, wn, lane);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (MMAS > 0) {
    qw_mma<EPI, NMI, 0, MMAS, NL, 1, NL>(P.fa[A1], P.fb[A1], acc, L, kb + 2);
  } else {
#pragma unroll
    for (int i = 0; i < NL; ++i) qw_load_b(L, kb + 2, NL + i);
  }
  __builtin_amdgcn_sched_barrier(0);
  wait_lgkm0();
  wait_vm<QW_LD>();
  qw_sync();
  // steps 2 and 3: A(kb + 2) loads; step 0 of slab kb + 1 is read after the
  // first four MFMAs of step 2 (into the set step 1 used), step 1 of kb + 1
  // before step 3 (into the set step 2 used)
  if constexpr (MMAS > 0) {
    constexpr int H = MMAS < 4 ? MMAS : 4;
    qw_mma<EPI, NMI, 0, H, NL, 0, 0>(P.fa[A2], P.fb[A2], acc, L, kb + 2);
    __builtin_amdgcn_sched_barrier(0);
    qw_read_set<EPI, NMI, A1>(P, kb + 1, 0, wm, wn, lane);
    __builtin_amdgcn_sched_barrier(0);
    qw_mma<EPI, NMI, H, MMAS, NL, 0, 0>(P.fa[A2], P.fb[A2], acc, L, kb + 2);
    __builtin_amdgcn_sched_barrier(0);
    qw_read_set<EPI, NMI, A2>(P, kb + 1, 1, wm, wn, lane);
    __builtin_amdgcn_sched_barrier(0);
    qw_mma<EPI, NMI, 0, MMAS, NL, 0, NL>(P.fa[A0], P.fb[A0], acc, L, kb + 2);
  } else {
#pragma unroll
    for (int i = 0; i < QW_LD; ++i) qw_load_a(L, kb + 2, i);
  }
}

// Main loop for a wave with NMI active row sub-tiles.  On entry slab 0 is
// visible to every wave and A(1), B(1) are in flight.  No scalar load may be
// in flight at the loop head: scalar loads return out of order, and a pending
// one would turn every LDS wait in the loop into a full drain.
template <int EPI, int NMI>
__device__ __forceinline__ void qw_loop(const QWLoad& L, int wm, int wn, int lane,
                                        f32x16_t (&acc)[QWCfg<EPI>::NB][4][QWCfg<EPI>::TN]) {
  // slab kb's step 0 uses set (4 kb) % 3 = kb % 3
  QWPipe<EPI, NMI> P;
  qw_read_set<EPI, NMI, 0>(P, 0, 0, wm, wn, lane);
  qw_read_set<EPI, NMI, 1>(P, 0, 1, wm, wn, lane);
  wait_lgkm0();
  int kb = 0;
  for (; kb + 3 <= L.nk; kb += 3) {
    qw_slab<EPI, NMI, 0>(P, L, kb, wm, wn, lane, acc);
    qw_slab<EPI, NMI, 1>(P, L, kb + 1, wm, wn, lane, acc);
    qw_slab<EPI, NMI, 2>(P, L, kb + 2, wm, wn, lane, acc);
  }
  if (kb < L.nk) qw_slab<EPI, NMI, 0>(P, L, kb, wm, wn, lane, acc);
  if (kb + 1 < L.nk) qw_slab<EPI, NMI, 1>(P, L, kb + 1, wm, wn, lane, acc);
  __builtin_amdgcn_sched_barrier(0);
  wait_vm<0>();
}

// One launch computes g0 alone (pair = 0), or g0 and the dense problem g1
// side by side (pair = 1, tiles enumerated by tile_for_block_pair); row_scale
// applies to g0's rows only.
template <int EPI>
__global__ __launch_bounds__(256) void gemm_qw_kernel(const GemmDesc g0, const GemmDesc g1, const int pair,
                                                      const float* __restrict__ row_scale_0) {
  using CF = QWCfg<EPI>;
  constexpr int NB = CF::NB, TN = CF::TN, BN = CF::BN;

  int which = 0, grp, row0, rows, n_tile;
  if (pair) {
    if (!tile_for_block_pair<QW_BM>(g0, g1, BN, which, grp, row0, rows, n_tile)) return;
  } else {
    if (!tile_for_block<QW_BM>(g0, (int)cdiv(g0.N, BN), grp, row0, rows, n_tile)) return;
  }
  which = __builtin_amdgcn_readfirstlane(which);
  const GemmDesc& g = which ? g1 : g0;
  const float* row_scale = which ? nullptr : row_scale_0;
  grp = __builtin_amdgcn_readfirstlane(grp);
  row0 = __builtin_amdgcn_readfirstlane(row0);
  rows = __builtin_amdgcn_readfirstlane(rows);
  n_tile = __builtin_amdgcn_readfirstlane(n_tile);
  const int n0 = n_tile * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // ---- direct-load sources.  Load i of wave w fills 1 KB block 8 w + i of
  // an operand region, rows r = 8 (8 w + i) + (l >> 3); lane l writes
  // physical chunk l & 7, i.e. logical chunk (l & 7) ^ ((r >> 1) & 7).
  // SwiGLU: B rows 0..127 are W1 rows n0.., rows 128..255 the same W3 rows
  // (waves 0-1 load the first half, waves 2-3 the second).
  QWLoad L;
  L.nk = g.K / QW_BK;
  L.lds_off = wave * QW_LD * 1024;
  L.a = static_cast<const char*>(g.A);
  {
    const void* const* tab = ((NB == 2 && wave >= 2) ? g.B1 : g.B0) + (int64_t)grp * g.nseg;
    L.b0 = static_cast<const char*>(tab[0]);
    L.b1 = static_cast<const char*>(tab[g.nseg - 1]);
    L.kseg = g.nseg > 1 ? g.kseg : 0x7fffffff;
  }
#pragma unroll
  for (int i = 0; i < QW_LD; ++i) {
    const int r = (wave * QW_LD + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int ra = min(r, rows - 1);
    const int64_t arow = g.a_map ? (int64_t)g.a_map[row0 + ra] : (int64_t)(row0 + ra);
    L.offa[i] = (uint32_t)(2 * (arow * g.lda + c * 8));
    const int bn = (NB == 2) ? n0 + (r & 127) : n0 + r;
    L.offb[i] = (uint32_t)(2 * ((int64_t)min(bn, g.N - 1) * g.ldb + c * 8));
  }

  f32x16_t acc[NB][4][TN];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int ni = 0; ni < TN; ++ni)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[b][j][ni][r] = 0.0f;

  // ---- prologue: A(0), B(0) and A(1), B(1) in flight together (slab 1 is
  // the last slab reloaded when there is only one); slab 0 visible to all
  // waves
#pragma unroll
  for (int i = 0; i < QW_LD; ++i) qw_load_a(L, 0, i);
#pragma unroll
  for (int i = 0; i < QW_LD; ++i) qw_load_b(L, 0, i);
#pragma unroll
  for (int i = 0; i < QW_LD; ++i) qw_load_a(L, 1, i);
#pragma unroll
  for (int i = 0; i < QW_LD; ++i) qw_load_b(L, 1, i);
  wait_vm<2 * QW_LD>();
  qw_sync();

  // active sub-tiles of this wave: j with (2j + wm) * 32 < rows
  const int nsub = (int)cdiv(rows, 32);
  const int nmi = max(0, min(4, (nsub - wm + 1) >> 1));
  switch (nmi) {
    case 4: qw_loop<EPI, 4>(L, wm, wn, lane, acc); break;
    case 3: qw_loop<EPI, 3>(L, wm, wn, lane, acc); break;
    case 2: qw_loop<EPI, 2>(L, wm, wn, lane, acc); break;
    case 1: qw_loop<EPI, 1>(L, wm, wn, lane, acc); break;
    default: qw_loop<EPI, 0>(L, wm, wn, lane, acc); break;
  }

  // ---- epilogue.  Lane holds row m = (2j + wm) * 32 + (lane & 31) and, per
  // q, columns .. + 8q + 4 (lane >> 5) + {0..3} (registers 4q..4q+3).  Each
  // output (h, then g and u when saved; or the down projection) is rounded to
  // bf16, staged in LDS as the block's row-major 256 x BN tile and written
  // back one 16-byte chunk per lane, so every row leaves as whole cache lines
  // (direct 8-byte stores from the MFMA layout would split each line over
  // eight store instructions).  Staging: 8-byte unit u of row m sits at unit
  // u ^ (m & 31), which keeps both the 32-row register writes and the 16-lane
  // row reads free of bank conflicts.
  __builtin_amdgcn_sched_barrier(0);
  wait_lgkm0();
  qw_sync();  // every wave is done with the slab buffers
  extern __shared__ __attribute__((aligned(16))) char qw_smem[];
  constexpr int ROWB = BN * 2;       // staged row bytes
  constexpr int LPR = ROWB / 16;     // lanes per row in the write-back
  constexpr int RPP = 256 / LPR;     // rows per write-back pass
  // Passes: the output (h or the down projection), then, when training
  // saves the pre-activations, g and u together (two staged tiles of 64 KB).
  const bool gu2 = EPI == EPI_SWIGLU && g.Gs && g.Us;
  const int npass = (EPI == EPI_SWIGLU) ? (gu2 ? 2 : 1 + (g.Gs ? 1 : 0) + (g.Us ? 1 : 0)) : 1;
  const int64_t ccol = (int64_t)grp * g.c_group_col;
  const int rr = tid / LPR, cc = tid % LPR;
  // Output rows of the tile: the c_map entries are fetched once, ahead of the
  // staging writes, and kept in LDS past the staged tiles (a map lookup per
  // write-back pass would wait on global memory every pass).
  static_assert(2 * 256 * QWCfg<EPI_SWIGLU>::BN * 2 <= 128 * 1024 && 256 * QWCfg<EPI_STORE>::BN * 2 <= 128 * 1024,
                "staged tiles below the row table");
  int32_t* crow_tab = reinterpret_cast<int32_t*>(qw_smem + 128 * 1024);
  char* stage_u = qw_smem + 256 * ROWB;   // second staged tile (u in the g|u pass)
  const int32_t my_crow = (g.c_map && tid < rows) ? g.c_map[row0 + tid] : row0 + tid;
  for (int pass = 0; pass < npass; ++pass) {
    // registers -> LDS
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = (2 * j + wm) * 32 + (lane & 31);
      float scale = 1.0f;
      if (EPI == EPI_STORE && row_scale) scale = (m < rows) ? row_scale[row0 + m] : 0.0f;
#pragma unroll
      for (int ni = 0; ni < TN; ++ni)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int u = (wn * (BN / 2) + ni * 32 + q * 8 + (lane >> 5) * 4) >> 2;
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a0 = acc[0][j][ni][q * 4 + e];
            if (EPI == EPI_SWIGLU) {
              const float a1 = acc[NB - 1][j][ni][q * 4 + e];
              v[e] = pass == 0 ? a0 * __builtin_amdgcn_rcpf(1.0f + __expf(-a0)) * a1
                               : ((pass == 1 && g.Gs) ? a0 : a1);
            } else {
              v[e] = a0 * scale;
            }
          }
          uint2 w;
          w.x = pack_bf16x2(v[0], v[1]);
          w.y = pack_bf16x2(v[2], v[3]);
          *reinterpret_cast<uint2*>(qw_smem + m * ROWB + ((u ^ (m & 31)) << 3)) = w;
          if (EPI == EPI_SWIGLU && gu2 && pass == 1) {
            // u beside g
            uint2 wu;
            wu.x = pack_bf16x2(acc[NB - 1][j][ni][q * 4 + 0], acc[NB - 1][j][ni][q * 4 + 1]);
            wu.y = pack_bf16x2(acc[NB - 1][j][ni][q * 4 + 2], acc[NB - 1][j][ni][q * 4 + 3]);
            *reinterpret_cast<uint2*>(stage_u + m * ROWB + ((u ^ (m & 31)) << 3)) = wu;
          }
        }
    }
    if (pass == 0) crow_tab[tid] = my_crow;
    qw_sync();
    // LDS -> global: lane cc of a row group stores 16-byte chunk cc of its row
    bf16_t* C = static_cast<bf16_t*>(pass == 0 ? g.C : ((pass == 1 && g.Gs) ? g.Gs : g.Us));
    const int n = n0 + cc * 8;
    // unrolled so that the LDS reads of several rows are in flight together
#pragma unroll 4
    for (int r = rr; r < rows; r += RPP) {
      const int pu = (2 * cc) ^ (r & 31);
      u32x4_t v = *reinterpret_cast<const u32x4_t*>(qw_smem + r * ROWB + ((pu >> 1) << 4));
      if (r & 1) v = u32x4_t{v.z, v.w, v.x, v.y};
      if (n < g.N) {
        *reinterpret_cast<u32x4_t*>(C + (int64_t)crow_tab[r] * g.ldc + ccol + n) = v;
      }
    }
    if (EPI == EPI_SWIGLU && gu2 && pass == 1) {
      bf16_t* U = static_cast<bf16_t*>(g.Us);
#pragma unroll 4
      for (int r = rr; r < rows; r += RPP) {
        const int pu = (2 * cc) ^ (r & 31);
        u32x4_t v = *reinterpret_cast<const u32x4_t*>(stage_u + r * ROWB + ((pu >> 1) << 4));
        if (r & 1) v = u32x4_t{v.z, v.w, v.x, v.y};
        if (n < g.N) *reinterpret_cast<u32x4_t*>(U + (int64_t)crow_tab[r] * g.ldc + ccol + n) = v;
      }
    }
    if (pass + 1 < npass) qw_sync();
  }
}

// Requirements beyond mfma_ok (gemm.hip): at most QW_MAX_SEG K segments, K
// and the segment length multiples of 64, and 32-bit element offsets into A
// and into every B block.
bool gemm_qw_ok(const GemmDesc& g) {
  const int64_t lim = int64_t(1) << 31;
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return g.nseg >= 1 && g.nseg <= QW_MAX_SEG && g.K % QW_BK == 0 && g.kseg % QW_BK == 0 && g.a_rows * g.lda < lim &&
         (int64_t)g.N * g.ldb < lim && g.bm == QW_BM && g.N % 8 == 0 && g.ldc % 8 == 0 && g.c_group_col % 8 == 0 &&
         a16(g.C) && a16(g.Gs) && a16(g.Us);
}

template <int EPI>
static int qw_launch(const GemmDesc& g0, const GemmDesc& g1, int pair, const float* row_scale, int64_t grid,
                     hipStream_t st) {
  if (grid == 0) return DSMOE_OK;
  // once per instantiation; the initialisation of a local static is thread-safe
  // (autograd runs the backward on its own thread)
  static const hipError_t attr = hipFuncSetAttribute((const void*)gemm_qw_kernel<EPI>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)QW_LDS);
  if (attr != hipSuccess) return fail(DSMOE_ERR_HIP, "gemm_qw: cannot raise LDS limit");
  hipLaunchKernelGGL(gemm_qw_kernel<EPI>, dim3((unsigned)grid), dim3(256), QW_LDS, st, g0, g1, pair, row_scale);
  return check_launch("gemm_qw");
}

int launch_gemm_qw(const GemmDesc& g, int epi, const float* row_scale, hipStream_t st) {
  const int bn = (epi == EPI_SWIGLU) ? QWCfg<EPI_SWIGLU>::BN : QWCfg<EPI_STORE>::BN;
  const int64_t m_bound = g.sched ? g.m_tiles_bound : cdiv(g.dense_rows, QW_BM) * g.groups;
  const int64_t grid = 8 * cdiv(m_bound * cdiv(g.N, bn), 8);
  return epi == EPI_SWIGLU ? qw_launch<EPI_SWIGLU>(g, g, 0, row_scale, grid, st)
                           : qw_launch<EPI_STORE>(g, g, 0, row_scale, grid, st);
}

// gr (routed schedule or dense) and the dense gd in one launch; the grid
// covers gd's tiles exactly and gr's up to its host bound (tile_for_block_pair).
int launch_gemm_qw_pair(const GemmDesc& gr, const GemmDesc& gd, int epi, const float* row_scale, hipStream_t st) {
  const int bn = (epi == EPI_SWIGLU) ? QWCfg<EPI_SWIGLU>::BN : QWCfg<EPI_STORE>::BN;
  const int64_t mr = gr.sched ? gr.m_tiles_bound : cdiv(gr.dense_rows, QW_BM) * gr.groups;
  const int64_t md = cdiv(gd.dense_rows, QW_BM) * gd.groups;
  const int64_t grid = 8 * (cdiv(md * cdiv(gd.N, bn), 8) + cdiv(mr * cdiv(gr.N, bn), 8));
  return epi == EPI_SWIGLU ? qw_launch<EPI_SWIGLU>(gr, gd, 1, row_scale, grid, st)
                           : qw_launch<EPI_STORE>(gr, gd, 1, row_scale, grid, st);
}

}  // namespace dsmoe
