// (c) Grouped NT GEMM for gfx950: a 256 x 256 output tile per workgroup of
// eight waves in two groups of four (one wave of each group per SIMD) that
// take turns at the matrix cores, fed from LDS slabs that stream in with
// direct global->LDS loads.
//
// Same contract and tile enumeration as gemm_mfma_kernel (gemm.hip).  The
// shape follows from gfx950 limits measured on MI355X:
//  * 512 VGPRs per SIMD lane for two waves: each wave owns a 128 x 64 block
//    of the tile (8 accumulator tiles, 128 registers) and holds a whole K
//    slab of fragments (96 registers), so a wave can run a slab's 32 MFMAs
//    back to back from registers.
//  * L2 -> LDS direct loads move whole 128-byte rows best, so K advances in
//    slabs of 64 bf16 (one cache line per row and operand).
//  * 160 KB of LDS: a slab is 32 KB per operand (256 rows of 128 bytes).  A
//    (activation rows, mostly L2 / MALL hits) cycles through a ring of two
//    slots, B (weights, streamed from HBM) through a ring of three.
//
// Ping-pong.  Barrier phases alternate: in phase 2k group 0 runs the MFMAs of
// slab k from registers while group 1 issues the direct loads of B(k + 2)
// and reads its fragments of slab k from LDS; in phase 2k + 1 group 1 runs
// slab k's MFMAs while group 0 issues A(k + 2) and reads slab k + 1.  So one
// wave per SIMD feeds the matrix core while the other issues loads and LDS
// reads, and neither waits on the other's memory traffic.  Each group waits
// for its own direct loads of a slab before the barrier that publishes it:
// group 0 for A(k + 1) at the end of phase 2k, group 1 for B(k + 1) in phase
// 2k.  A(k + 2) goes into slab k's A slot (read by group 1 in phase 2k and by
// group 0 before it), B(k + 2) into slab k - 1's B slot.  Both groups pass
// 1 + 2 nk barriers.  The eight-wave epilogue stages and writes the tile with
// twice the threads of a four-wave one.
//
// Ragged tiles: the waves in row group wm own the 32-row sub-tiles wm,
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
// Group 0's waves load the A rows 64 s .. 64 s + 63 (s = wave in group),
// group 1's the same B rows; loads are addressed as a wave-uniform base in
// SGPRs plus 32-bit per-lane offsets.
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

// Direct-load sources of one wave: group 0 loads A, group 1 B (two K segments
// at most: the segment that holds slab k0 starts at K = 0 or at kseg).
struct QWLoad {
  const char* base0;
  const char* base1;
  uint32_t off[QW_LD];    // byte offset of load i's row chunk
  int kseg;               // K at which base1 takes over (0x7fffffff: one segment)
  int lds_off;            // byte offset of this wave's 8 KB inside an operand region
  int nk;
};

__device__ __forceinline__ void qw_load_a(const QWLoad& L, int ka) {
  extern __shared__ __attribute__((aligned(16))) char qw_smem[];
  const uint32_t d = lds_addr(qw_smem) + L.lds_off + (ka & 1) * QW_REG;
  const int k0 = ka * QW_BK;
#pragma unroll
  for (int i = 0; i < QW_LD; ++i) dma16s(L.base0 + 2 * k0, L.off[i], d + i * 1024);
}

__device__ __forceinline__ void qw_load_b(const QWLoad& L, int kb) {
  extern __shared__ __attribute__((aligned(16))) char qw_smem[];
  const uint32_t d = lds_addr(qw_smem) + L.lds_off + QW_BOFF + (kb % QW_BSLOTS) * QW_REG;
  const int k0 = kb * QW_BK;
  const bool hi = k0 >= L.kseg;
  const char* src = hi ? L.base1 : L.base0;
  const int kin = hi ? k0 - L.kseg : k0;
#pragma unroll
  for (int i = 0; i < QW_LD; ++i) dma16s(src + 2 * kin, L.off[i], d + i * 1024);
}

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
    for (int j = 0; j < NMI; ++j)
      F.fa[st][j] = *reinterpret_cast<const bf16x8_t*>(sA + qw_swz((2 * j + wm) * 32 + (lane & 31), c));
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

// Group 0: computes slab k in phase 2k; in phase 2k + 1 issues A(k + 2) and
// reads slab k + 1.
template <int EPI, int NMI>
__device__ __forceinline__ void qw_loop0(const QWLoad& L, int wm, int cg, int lane,
                                         f32x16_t (&acc)[QWCfg<EPI>::NB][4][QWCfg<EPI>::TN]) {
  QWFrag<EPI> F;
  qw_read<EPI, NMI>(F, 0, wm, cg, lane);
  wait_lgkm0();
  qw_sync();
  for (int k = 0; k < L.nk; ++k) {
    __builtin_amdgcn_sched_barrier(0);
    qw_mma<EPI, NMI>(F, acc);
    __builtin_amdgcn_sched_barrier(0);
    wait_vm<0>();  // this wave's part of A(k + 1) has landed
    qw_sync();
    if (k + 2 < L.nk) qw_load_a(L, k + 2);
    __builtin_amdgcn_sched_barrier(0);
    if (k + 1 < L.nk) qw_read<EPI, NMI>(F, k + 1, wm, cg, lane);
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm0();
    qw_sync();
  }
}

// Group 1: in phase 2k issues B(k + 2) and reads slab k; computes it in phase
// 2k + 1.
template <int EPI, int NMI>
__device__ __forceinline__ void qw_loop1(const QWLoad& L, int wm, int cg, int lane,
                                         f32x16_t (&acc)[QWCfg<EPI>::NB][4][QWCfg<EPI>::TN]) {
  QWFrag<EPI> F;
  qw_sync();
  for (int k = 0; k < L.nk; ++k) {
    if (k + 2 < L.nk) qw_load_b(L, k + 2);
    __builtin_amdgcn_sched_barrier(0);
    qw_read<EPI, NMI>(F, k, wm, cg, lane);
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm0();
    if (k + 2 < L.nk)
      wait_vm<QW_LD>();  // B(k + 1) has landed; B(k + 2) may still be in flight
    else
      wait_vm<0>();
    qw_sync();
    __builtin_amdgcn_sched_barrier(0);
    qw_mma<EPI, NMI>(F, acc);
    __builtin_amdgcn_sched_barrier(0);
    qw_sync();
  }
}

// Registers -> LDS staging of output pass `pass` (0: h or the down
// projection; 1: g, with u beside it when both are saved; 2: u) as the
// block's row-major 256 x BN bf16 tile: 8-byte unit u of row m at unit
// u ^ (m & 31), which keeps both the 32-row register writes and the 16-lane
// row reads free of bank conflicts.
template <int EPI>
__device__ __forceinline__ void qw_stage(const f32x16_t (&acc)[QWCfg<EPI>::NB][4][QWCfg<EPI>::TN], const GemmDesc& g,
                                         const float* __restrict__ row_scale, int pass, int rows, int row0, int wm,
                                         int cg, int lane) {
  using CF = QWCfg<EPI>;
  constexpr int NB = CF::NB, TN = CF::TN, ROWB = CF::BN * 2;
  extern __shared__ __attribute__((aligned(16))) char qw_smem[];
  const bool gu2 = EPI == EPI_SWIGLU && g.Gs && g.Us;
  char* stage_u = qw_smem + 256 * ROWB;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = (2 * j + wm) * 32 + (lane & 31);
    float scale = 1.0f;
    if (EPI == EPI_STORE && row_scale) scale = (m < rows) ? row_scale[row0 + m] : 0.0f;
#pragma unroll
    for (int ni = 0; ni < TN; ++ni)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int colb = (EPI == EPI_SWIGLU ? cg * 32 : cg * 64 + ni * 32);
        const int u = (colb + q * 8 + (lane >> 5) * 4) >> 2;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a0 = acc[0][j][ni][q * 4 + e];
          if (EPI == EPI_SWIGLU) {
            const float a1 = acc[NB - 1][j][ni][q * 4 + e];
            v[e] = pass == 0 ? a0 * __builtin_amdgcn_rcpf(1.0f + __expf(-a0)) * a1 : ((pass == 1 && g.Gs) ? a0 : a1);
          } else {
            v[e] = a0 * scale;
          }
        }
        uint2 w;
        w.x = pack_bf16x2(v[0], v[1]);
        w.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2*>(qw_smem + m * ROWB + ((u ^ (m & 31)) << 3)) = w;
        if (EPI == EPI_SWIGLU && gu2 && pass == 1) {
          uint2 wu;
          wu.x = pack_bf16x2(acc[NB - 1][j][ni][q * 4 + 0], acc[NB - 1][j][ni][q * 4 + 1]);
          wu.y = pack_bf16x2(acc[NB - 1][j][ni][q * 4 + 2], acc[NB - 1][j][ni][q * 4 + 3]);
          *reinterpret_cast<uint2*>(stage_u + m * ROWB + ((u ^ (m & 31)) << 3)) = wu;
        }
      }
  }
}

// One launch computes g0 alone (pair = 0), or g0 and the dense problem g1
// side by side (pair = 1, tiles enumerated by tile_for_block_pair); row_scale
// applies to g0's rows only.
template <int EPI>
__global__ __launch_bounds__(QW_THREADS) void gemm_qw_kernel(const GemmDesc g0, const GemmDesc g1, const int pair,
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
  const int G = wave >> 2, s = wave & 3;        // group, wave in group
  const int wm = s >> 1, cg = (s & 1) * 2 + G;  // row group, column group

  // ---- direct-load sources.  Load i of wave s of a group fills 1 KB block
  // 8 s + i of its operand region, rows r = 8 (8 s + i) + (l >> 3); lane l
  // writes physical chunk l & 7, i.e. logical chunk (l & 7) ^ ((r >> 1) & 7).
  // SwiGLU: B rows 0..127 are W1 rows n0.., rows 128..255 the same W3 rows.
  QWLoad L;
  L.nk = g.K / QW_BK;
  L.lds_off = s * QW_LD * 1024;
  L.kseg = 0x7fffffff;
  if (G == 0) {
    L.base0 = L.base1 = static_cast<const char*>(g.A);
  } else {
    const void* const* tab = ((NB == 2 && s >= 2) ? g.B1 : g.B0) + (int64_t)grp * g.nseg;
    L.base0 = static_cast<const char*>(tab[0]);
    L.base1 = static_cast<const char*>(tab[g.nseg - 1]);
    L.kseg = g.nseg > 1 ? g.kseg : 0x7fffffff;
  }
#pragma unroll
  for (int i = 0; i < QW_LD; ++i) {
    const int r = (s * QW_LD + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    if (G == 0) {
      const int ra = min(r, rows - 1);
      const int64_t arow = g.a_map ? (int64_t)g.a_map[row0 + ra] : (int64_t)(row0 + ra);
      L.off[i] = (uint32_t)(2 * (arow * g.lda + c * 8));
    } else {
      const int bn = (NB == 2) ? n0 + (r & 127) : n0 + r;
      L.off[i] = (uint32_t)(2 * ((int64_t)min(bn, g.N - 1) * g.ldb + c * 8));
    }
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

  // ---- prologue: slabs 0 and 1 in flight; slab 0 visible to all waves
  if (G == 0) {
    qw_load_a(L, 0);
    if (L.nk > 1) qw_load_a(L, 1);
  } else {
    qw_load_b(L, 0);
    if (L.nk > 1) qw_load_b(L, 1);
  }
  if (L.nk > 1)
    wait_vm<QW_LD>();
  else
    wait_vm<0>();
  qw_sync();

  // active sub-tiles of this wave: j with (2j + wm) * 32 < rows
  const int nsub = (int)cdiv(rows, 32);
  const int nmi = max(0, min(4, (nsub - wm + 1) >> 1));
  if (G == 0) {
    switch (nmi) {
      case 4: qw_loop0<EPI, 4>(L, wm, cg, lane, acc); break;
      case 3: qw_loop0<EPI, 3>(L, wm, cg, lane, acc); break;
      case 2: qw_loop0<EPI, 2>(L, wm, cg, lane, acc); break;
      case 1: qw_loop0<EPI, 1>(L, wm, cg, lane, acc); break;
      default: qw_loop0<EPI, 0>(L, wm, cg, lane, acc); break;
    }
  } else {
    switch (nmi) {
      case 4: qw_loop1<EPI, 4>(L, wm, cg, lane, acc); break;
      case 3: qw_loop1<EPI, 3>(L, wm, cg, lane, acc); break;
      case 2: qw_loop1<EPI, 2>(L, wm, cg, lane, acc); break;
      case 1: qw_loop1<EPI, 1>(L, wm, cg, lane, acc); break;
      default: qw_loop1<EPI, 0>(L, wm, cg, lane, acc); break;
    }
  }

  // ---- epilogue.  Each output (h, then g and u when saved; or the down
  // projection) is rounded to bf16, staged in LDS as the block's row-major
  // tile (qw_stage) and written back one 16-byte chunk per lane, so every row
  // leaves as whole cache lines (direct 8-byte stores from the MFMA layout
  // would split each line over eight store instructions).
  __builtin_amdgcn_sched_barrier(0);
  wait_vm<0>();
  wait_lgkm0();
  qw_sync();  // every wave is done with the slab buffers
  extern __shared__ __attribute__((aligned(16))) char qw_smem[];
  constexpr int ROWB = BN * 2;             // staged row bytes
  constexpr int LPR = ROWB / 16;           // lanes per row in the write-back
  constexpr int RPP = QW_THREADS / LPR;    // rows per write-back pass
  // Passes: the output (h or the down projection), then, when training
  // saves the pre-activations, g and u together (two staged tiles of 64 KB).
  const bool gu2 = EPI == EPI_SWIGLU && g.Gs && g.Us;
  const int npass = (EPI == EPI_SWIGLU) ? (gu2 ? 2 : 1 + (g.Gs ? 1 : 0) + (g.Us ? 1 : 0)) : 1;
  const int64_t ccol = (int64_t)grp * g.c_group_col;
  const int rr = tid / LPR, cc = tid % LPR;
  // Output rows of the tile: the c_map entries are fetched once and kept in
  // LDS past the staged tiles (a map lookup per write-back pass would wait on
  // global memory every pass).
  static_assert(2 * 256 * QWCfg<EPI_SWIGLU>::BN * 2 <= 128 * 1024 && 256 * QWCfg<EPI_STORE>::BN * 2 <= 128 * 1024,
                "staged tiles below the row table");
  int32_t* crow_tab = reinterpret_cast<int32_t*>(qw_smem + 128 * 1024);
  char* stage_u = qw_smem + 256 * ROWB;   // second staged tile (u in the g|u pass)
  if (tid < 256) crow_tab[tid] = (g.c_map && tid < rows) ? g.c_map[row0 + tid] : row0 + tid;
  for (int pass = 0; pass < npass; ++pass) {
    qw_stage<EPI>(acc, g, row_scale, pass, rows, row0, wm, cg, lane);
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
      if (n < g.N) *reinterpret_cast<u32x4_t*>(C + (int64_t)crow_tab[r] * g.ldc + ccol + n) = v;
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
  hipLaunchKernelGGL(gemm_qw_kernel<EPI>, dim3((unsigned)grid), dim3(QW_THREADS), QW_LDS, st, g0, g1, pair,
                     row_scale);
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
