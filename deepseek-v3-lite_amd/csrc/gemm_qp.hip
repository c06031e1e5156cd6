// (c) Grouped NT GEMM for gfx950, persistent: one workgroup per CU streams
// 64-wide K slabs through its LDS rings without a break between output tiles.
//
// Tiles are 256 x 256 outputs (the gate/up projection: 128 h columns, each
// from a W1 and a W3 row block); gemm_pp.h describes the slab layout and the
// waves' fragment and MFMA steps.  Eight waves in two groups of four (one
// wave of each group per SIMD) take turns at the matrix cores: in phase 2s
// group 0 runs the 32 MFMAs of slab s from registers while group 1 issues the
// direct loads of B(s + 2) and reads its fragments of slab s; in phase 2s + 1
// group 1 computes slab s while group 0 issues A(s + 2) and reads slab s + 1.
// A cycles through a ring of two 32 KB slots, B (weights, streamed from HBM)
// through a ring of three; each group waits for its own direct loads of a
// slab before the barrier that publishes it.
//
// s counts the slabs of all the tiles a workgroup owns, one after another
// (measured on MI355X: a workgroup per tile paid about 8 us of a 55 us tile
// at K = 2048 with idle matrix cores, for the tile lookup, the row map, the
// first slab's load latency and an epilogue behind two barriers):
//  * the loaders run two slabs ahead across tile boundaries, so the first
//    slabs of tile i + 1 load while tile i computes its last ones; a tile's
//    row map is fetched one slab before its first load;
//  * each group runs its epilogue in its own load phase, group 0 right after
//    its last MFMAs of a tile (while group 1 computes the tile's last slab),
//    group 1 in the next phase (while group 0 computes the next tile's first
//    slab).  A wave stages its outputs in a ring slot that no load fills and
//    no wave reads during that phase, reads them back as whole row pieces and
//    stores those; it issues the load that refills the slot only afterwards.
//
// Tiles: block b runs on XCD b % 8; each XCD takes a contiguous eighth of
// the dense problem's tiles (the shared experts, pair launches) and of the
// routed problem's tiles, and its workgroups take that list round robin.  The
// grid is one workgroup per CU (160 KB of LDS keeps it at one per CU).
#include "gemm_pp.h"

#include <atomic>

namespace dsmoe {

// Global-address-space access: pointers in the descriptor are generic to the
// compiler, and flat accesses also count against the LDS wait counter, so a
// wait for LDS fragments would wait for them too.
template <class T>
__device__ __forceinline__ T ldg_as1(const T* p) {
  typedef __attribute__((address_space(1))) const T gT;
  return *(gT*)(p);
}
typedef __attribute__((address_space(1))) u32x4_t gu32x4_st;
__device__ __forceinline__ void stg16(void* p, u32x4_t v) { *(gu32x4_st*)(p) = v; }
// Non-temporal: the g, u saves of a training forward are read only by the
// backward, so they should not displace the caches' operand tiles.
__device__ __forceinline__ void stg16_nt(void* p, u32x4_t v) { __builtin_nontemporal_store(v, (gu32x4_st*)(p)); }

// Kernel arguments, read through the kernarg segment pointer.  qp_args()
// hides the pointer's origin from the compiler, so each tile switch loads the
// descriptor fields it needs from the scalar cache again; otherwise the
// compiler hoists every field of both descriptors to the kernel entry and
// keeps them live through the persistent loop, which spills.
struct QPArgs {
  GemmDesc g[2];            // g[0]: routed (or the only) problem; g[1]: dense problem of a pair launch
  const float* row_scale;   // per-row output scale of g[0] (down projection), or null
  int pair;
};
typedef __attribute__((address_space(4))) const QPArgs QPArgsK;

__device__ __forceinline__ QPArgsK* qp_args() {
  QPArgsK* p = (QPArgsK*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return p;
}

// The lane index, recomputed (mbcnt) and hidden from the compiler in the same
// way: the per-lane address arithmetic of a tile switch is redone there
// instead of being hoisted out of the persistent loop and kept in registers.
__device__ __forceinline__ int qp_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Scalar (SMEM) load of a wave-uniform value that earlier launches wrote and
// this one only reads (tile schedule, its count, weight pointer tables): it
// lands in SGPRs and counts against the LDS/scalar counter, not the vector
// memory counter, so it never waits for the direct loads in flight.
template <class T>
__device__ __forceinline__ T ld_scalar(const T* p) {
  typedef __attribute__((address_space(4))) const T kT;
  return *(kT*)(p);
}

// A pointer made wave-uniform (SGPRs): the direct loads take their base
// address in SGPRs.
__device__ __forceinline__ const char* qp_uniform(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const char*>(((uint64_t)hi << 32) | lo);
}

struct QPTile {
  int which;  // 0: g0, 1: g1 (dense problem of a pair launch)
  int grp, row0, rows, n0, nk;
};

// This workgroup's share of its XCD's tile list: items j, j + nb, ...; items
// below d_cnt are dense tiles of g[1], the rest tiles of g[0].
struct QPList {
  int d_base, r_base, d_cnt, ntd, ntr, j, nb, ntiles;
};

__device__ __forceinline__ QPList qp_list(int bn) {
  QPArgsK* P = qp_args();
  QPList L;
  const int x = blockIdx.x & 7;
  L.j = blockIdx.x >> 3;
  L.nb = gridDim.x >> 3;
  const GemmDesc __attribute__((address_space(4)))& g0 = P->g[0];
  L.ntr = (int)cdiv(g0.N, bn);
  const int64_t mr = g0.sched ? (int64_t)ld_scalar(g0.sched_count) : cdiv(g0.dense_rows, QW_BM) * g0.groups;
  const int64_t tr = mr * L.ntr, per_r = cdiv(tr, 8);
  L.r_base = (int)(x * per_r);
  const int r_cnt = (int)max<int64_t>(0, min<int64_t>(per_r, tr - L.r_base));
  L.ntd = 1;
  L.d_base = 0;
  L.d_cnt = 0;
  if (P->pair) {
    const GemmDesc __attribute__((address_space(4)))& g1 = P->g[1];
    L.ntd = (int)cdiv(g1.N, bn);
    const int64_t td = cdiv(g1.dense_rows, QW_BM) * g1.groups * L.ntd, per_d = cdiv(td, 8);
    L.d_base = (int)(x * per_d);
    L.d_cnt = (int)max<int64_t>(0, min<int64_t>(per_d, td - L.d_base));
  }
  const int tot = L.d_cnt + r_cnt;
  L.ntiles = tot > L.j ? (int)cdiv(tot - L.j, L.nb) : 0;
  L.d_cnt = __builtin_amdgcn_readfirstlane(L.d_cnt);
  L.ntiles = __builtin_amdgcn_readfirstlane(L.ntiles);
  return L;
}

__device__ __forceinline__ QPTile qp_tile(const QPList& L, int bn, int i) {
  QPArgsK* P = qp_args();
  QPTile t;
  const int li = L.j + i * L.nb;
  int lin, nt;
  if (li < L.d_cnt) {
    t.which = 1;
    lin = L.d_base + li;
    nt = L.ntd;
  } else {
    t.which = 0;
    lin = L.r_base + (li - L.d_cnt);
    nt = L.ntr;
  }
  t.which = __builtin_amdgcn_readfirstlane(t.which);
  const GemmDesc __attribute__((address_space(4)))& g = P->g[t.which];
  int mt = (int)((uint32_t)lin / (uint32_t)nt);
  int nb_i = lin - mt * nt;
  if (g.sched) {
    static_assert(sizeof(MTile) == sizeof(u32x4_t), "MTile is four 32-bit fields");
    const u32x4_t* sch = reinterpret_cast<const u32x4_t*>(g.sched);
    u32x4_t m = ld_scalar(sch + mt);
    // Item order inside a group (expert) of n M tiles: every item reads 256
    // weight rows and 256 activation rows per slab, so with more N blocks
    // than M tiles (nt > n) the group's weights are the larger operand and
    // its items run N block by N block (item q = nb_i * n + i of the group's
    // range): the workgroups on consecutive items read the same weight rows
    // at about the same time, and each weight block comes from HBM about
    // once.  Otherwise M tile by M tile (the activation rows read once).
    const uint32_t n = m.w & 0xffffu;  // MTile::seq: tiles of the group
    if (n > 1 && (uint32_t)nt > n) {
      const int t0 = mt - (int)(m.w >> 16);
      const uint32_t q = (uint32_t)(lin - t0 * nt);
      const int mt2 = t0 + (int)(q % n);
      nb_i = (int)(q / n);
      if (mt2 != mt) m = ld_scalar(sch + mt2);
    }
    t.grp = (int)m.x;    // MTile::group
    t.row0 = (int)m.y;   // MTile::row0
    t.rows = (int)m.z;   // MTile::rows
  } else {
    const int tpg = (int)cdiv(g.dense_rows, QW_BM);
    t.grp = (int)((uint32_t)mt / (uint32_t)tpg);
    t.row0 = (mt - t.grp * tpg) * QW_BM;
    t.rows = min(QW_BM, g.dense_rows - t.row0);
  }
  t.n0 = nb_i * bn;
  t.nk = g.K / QW_BK;
  t.grp = __builtin_amdgcn_readfirstlane(t.grp);
  t.row0 = __builtin_amdgcn_readfirstlane(t.row0);
  t.rows = __builtin_amdgcn_readfirstlane(t.rows);
  t.n0 = __builtin_amdgcn_readfirstlane(t.n0);
  t.nk = __builtin_amdgcn_readfirstlane(t.nk);
  return t;
}

// ---- group 0's loader: A rows of the load tile (the tile whose slab is
// loaded next, up to two slabs ahead of the compute cursor).  Load i of wave
// s fills 1 KB block 8 s + i of the A slot: rows r = 8 (8 s + i) + (l >> 3),
// lane l writing physical chunk l & 7 = logical chunk (l & 7) ^ ((r >> 1) & 7).
struct QPA {
  const char* base;
  uint32_t lda2;         // bytes per A row
  uint32_t off[QW_LD];   // byte offsets; after a tile switch the A row indices until converted
  int lt, lk, nk, ls;    // load tile, its next slab, its slab count, global index of the next load
  int pend;              // off[] holds row indices
  int nld;               // loads of this wave that hold rows of the tile (the rest are skipped)
};

__device__ __forceinline__ void qpa_rows(QPA& A, const QPTile& t, int s, int lane_) {
  QPArgsK* P = qp_args();
  const int lane = qp_lane();
  const GemmDesc __attribute__((address_space(4)))& g = P->g[t.which];
  const int32_t* amap = g.a_map;
#pragma unroll
  for (int i = 0; i < QW_LD; ++i) {
    const int r = (s * QW_LD + i) * 8 + (lane >> 3);
    const int ra = t.row0 + min(r, t.rows - 1);
    A.off[i] = amap ? (uint32_t)ldg_as1(amap + ra) : (uint32_t)ra;
  }
  A.base = qp_uniform(g.A);
  A.lda2 = (uint32_t)(2 * g.lda);
  // Load i of wave s covers rows (s QW_LD + i) 8 .. + 7; loads wholly past
  // the tile's rows are skipped.  The LDS rows they would fill feed only
  // output rows that are never stored (an output row depends on its A row
  // alone), so a partial tile moves only the A bytes it uses (C3: the last
  // M tile of 30 of the 64 experts holds 3 to 94 rows).
  A.nld = __builtin_amdgcn_readfirstlane(min(QW_LD, max(0, (t.rows + 7) / 8 - s * QW_LD)));
  A.nk = t.nk;
  A.lk = 0;
  A.pend = 1;
}

__device__ __forceinline__ void qpa_step(QPA& A, const QPList& L, int bn, int s, int lane, uint32_t lds_a) {
  if (A.lt >= L.ntiles) return;
  if (A.pend) {
    lane = qp_lane();
#pragma unroll
    for (int i = 0; i < QW_LD; ++i) {
      const int r = (s * QW_LD + i) * 8 + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      A.off[i] = A.off[i] * A.lda2 + (uint32_t)(c * 16);
    }
    A.pend = 0;
  }
  const uint32_t d = lds_a + (A.ls & 1) * QW_REG;
  const char* src = A.base + A.lk * (QW_BK * 2);
  if (A.nld == QW_LD) {
#pragma unroll
    for (int i = 0; i < QW_LD; ++i) dma16s(src, A.off[i], d + i * 1024);
  } else {
#pragma unroll
    for (int i = 0; i < QW_LD; ++i)
      if (i < A.nld) dma16s(src, A.off[i], d + i * 1024);
  }
  ++A.ls;
  if (++A.lk == A.nk) {
    if (++A.lt < L.ntiles) qpa_rows(A, qp_tile(L, bn, A.lt), s, lane);
  }
}

// ---- group 1's loader: B rows n0 .. of the load tile's weight block(s) (two
// K segments at most: base1 takes over at K = kseg).  SwiGLU: waves 0, 1 load
// W1 rows n0 .. n0 + 127, waves 2, 3 the same W3 rows.
struct QPB {
  const char* base0;
  const char* base1;
  int kseg;
  uint32_t off[QW_LD];
  int lt, lk, nk, ls;
};

template <int NB>
__device__ __forceinline__ void qpb_set(QPB& B, const QPTile& t, int s, int lane_) {
  QPArgsK* P = qp_args();
  const int lane = qp_lane();
  const GemmDesc __attribute__((address_space(4)))& g = P->g[t.which];
  const int nseg = g.nseg, N = g.N;
  const int64_t ldb = g.ldb;
  const void* const* tab = ((NB == 2 && s >= 2) ? g.B1 : g.B0) + (int64_t)t.grp * nseg;
  B.base0 = qp_uniform(ld_scalar(tab));
  B.base1 = qp_uniform(ld_scalar(tab + nseg - 1));
  B.kseg = nseg > 1 ? g.kseg : 0x7fffffff;
#pragma unroll
  for (int i = 0; i < QW_LD; ++i) {
    const int r = (s * QW_LD + i) * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    const int bn = (NB == 2) ? t.n0 + (r & 127) : t.n0 + r;
    B.off[i] = (uint32_t)(2 * ((int64_t)min(bn, N - 1) * ldb + c * 8));
  }
  B.nk = t.nk;
  B.lk = 0;
}

// Issues the next B slab; false when the block's tiles are all loaded.
template <int NB>
__device__ __forceinline__ bool qpb_step(QPB& B, const QPList& L, int bn, int s, int lane, uint32_t lds_b) {
  if (B.lt >= L.ntiles) return false;
  const uint32_t d = lds_b + (B.ls % QW_BSLOTS) * QW_REG;
  const int k0 = B.lk * QW_BK;
  const bool hi = k0 >= B.kseg;
  const char* src = (hi ? B.base1 : B.base0) + 2 * (hi ? k0 - B.kseg : k0);
#pragma unroll
  for (int i = 0; i < QW_LD; ++i) dma16s(src, B.off[i], d + i * 1024);
  ++B.ls;
  if (++B.lk == B.nk) {
    if (++B.lt < L.ntiles) qpb_set<NB>(B, qp_tile(L, bn, B.lt), s, lane);
  }
  return true;
}

// ---- epilogue of one wave's part of a tile.  Each wave stages its own
// outputs in LDS, in a region of a ring slot no load or read uses during the
// epilogue's phase, reads them back as whole row pieces (128 bytes per row
// for the down projection, 64 for gate/up) and stores those: a store
// instruction then writes 8 (or 16) rows of full pieces instead of 32 bytes
// of each of 32 rows from the MFMA layout.  No other wave reads the region,
// and LDS accesses of one wave complete in order, so no barrier is needed.
//
// Staged layout: local row r (sub-tile j - j0, MFMA lane row) of WB bytes
// (64 TN), 8-byte unit u = 8 ni + 2q + h (columns colb + 8q + 4h .. + 3) at
// unit u ^ swz(r): swz keeps unit pairs together (16-byte read-back) and
// spreads the 32 rows of an MFMA-layout write over all banks.
template <int EPI>
struct QPOut {
  static constexpr int TN = QWCfg<EPI>::TN;
  static constexpr int WB = 64 * TN;       // staged row bytes
  static constexpr int LPR = WB / 16;      // lanes per row in the read-back
  static constexpr int RPI = 64 / LPR;     // rows per read-back instruction
  __device__ static __forceinline__ int swz(int r) {
    return WB == 64 ? (((r >> 2) & 3) << 1) : (((r >> 1) & 7) << 1);
  }
};

// One pass: sub-tiles j0 .. j0 + NJ - 1 of output `kind` (0: C, 1: G, 2: U)
// staged at LDS byte address `region` and written back.
template <int EPI, int NMI, int J0, int NJ>
__device__ __forceinline__ void qp_out_pass(const f32x16_t (&acc)[QWCfg<EPI>::NB][4][QWCfg<EPI>::TN], int kind,
                                            char* __restrict__ out, const int (&crow)[4], const float (&scale)[4],
                                            int64_t ldc, int64_t ccol, int n0, int N, int rows, int row0,
                                            bool has_map, int wm, int cg, int lane, uint32_t region) {
  using O = QPOut<EPI>;
  constexpr int NB = QWCfg<EPI>::NB, TN = QWCfg<EPI>::TN;
  extern __shared__ __attribute__((aligned(16))) char qw_smem[];
  char* const base = qw_smem + (region - lds_addr(qw_smem));
  const int half = lane >> 5;
  // registers -> LDS
#pragma unroll
  for (int j = J0; j < J0 + NJ; ++j) {
    if (j >= NMI) break;
    const int r = (j - J0) * 32 + (lane & 31);
#pragma unroll
    for (int ni = 0; ni < TN; ++ni)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a0 = acc[0][j][ni][q * 4 + e];
          if (EPI == EPI_SWIGLU) {
            const float a1 = acc[NB - 1][j][ni][q * 4 + e];
            v[e] = kind == 0 ? a0 * __builtin_amdgcn_rcpf(1.0f + __expf(-a0)) * a1 : (kind == 1 ? a0 : a1);
          } else {
            v[e] = a0 * scale[j];
          }
        }
        const int u = ni * 8 + 2 * q + half;
        *reinterpret_cast<u32x2_t*>(base + r * O::WB + ((u ^ O::swz(r)) << 3)) =
            u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      }
  }
  // LDS -> global: lane L reads 16 bytes (chunk L % LPR) of local row
  // i * RPI + L / LPR
  const int c = lane % O::LPR;
  const int colb = (EPI == EPI_SWIGLU ? cg * 32 : cg * 64) + c * 8;
#pragma unroll
  for (int i = 0; i < NJ * 32 / O::RPI; ++i) {
    const int j = J0 + (i * O::RPI) / 32;
    if (j >= NMI) break;
    const int lr = (i * O::RPI) % 32 + lane / O::LPR;  // MFMA lane row that held this row
    const int r = i * O::RPI + lane / O::LPR;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(base + r * O::WB + (((2 * c) ^ O::swz(r)) << 3));
    const int m = (2 * j + wm) * 32 + lr;
    const int64_t row = has_map ? (int64_t)__builtin_amdgcn_ds_bpermute(lr << 2, crow[j]) : (int64_t)(row0 + m);
    if (m < rows && n0 + colb < N) {
      if (kind == 0)
        stg16(out + 2 * (row * ldc + ccol + colb), v);
      else
        stg16_nt(out + 2 * (row * ldc + ccol + colb), v);
    }
  }
}

// The epilogue of one wave.  Group 0 (BIG) has two 32 KB slots (ra, rb) free
// in its epilogue phase, group 1 one (ra).  Wave sw stages only in the 8 KB
// at sw * 8 KB of a slot: in the A slot that is the part its own next A load
// refills (each wave loads 8 KB of an operand slot), in the B slot the part
// its own next B load (group 1) refills, so no wave's load lands in another
// wave's staging.
template <int EPI, int NMI, bool BIG>
__device__ __forceinline__ void qp_epilogue(const f32x16_t (&acc)[QWCfg<EPI>::NB][4][QWCfg<EPI>::TN],
                                            const QPTile& t, const int (&crow)[4], int sw, int wm, int cg,
                                            uint32_t ra, uint32_t rb) {
  QPArgsK* P = qp_args();
  const int lane = qp_lane();
  const GemmDesc __attribute__((address_space(4)))& g = P->g[t.which];
  const int32_t* c_map = g.c_map;
  const float* row_scale = t.which ? nullptr : P->row_scale;
  const int64_t ldc = g.ldc;
  const int N = g.N;
  const int64_t ccol = (int64_t)t.grp * g.c_group_col + t.n0;
  // per-row scales of this lane's MFMA rows (the seam's fused routing weight)
  float scale[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  if (EPI == EPI_STORE && row_scale) {
#pragma unroll
    for (int j = 0; j < NMI; ++j) {
      const int m = (2 * j + wm) * 32 + (lane & 31);
      scale[j] = m < t.rows ? ldg_as1(row_scale + t.row0 + m) : 0.0f;
    }
  }
  const bool has_map = c_map != nullptr;
  char* const C = static_cast<char*>(g.C);
#define QP_PASS(KIND, OUT, J0, NJ, REG)                                                                          \
  qp_out_pass<EPI, NMI, J0, NJ>(acc, KIND, OUT, crow, scale, ldc, ccol, t.n0, N, t.rows, t.row0, has_map, wm, cg, \
                                lane, REG)
  if (EPI == EPI_SWIGLU) {
    // 8 KB per wave and output
    const uint32_t w = ra + sw * 8192;
    char* const Gs = static_cast<char*>(g.Gs);
    char* const Us = static_cast<char*>(g.Us);
    QP_PASS(0, C, 0, 4, w);
    if (Gs) QP_PASS(1, Gs, 0, 4, BIG ? rb + sw * 8192 : w);
    if (Us) QP_PASS(2, Us, 0, 4, w);
  } else if (BIG) {
    // sub-tiles 0, 1 in this wave's 8 KB of the A slot (the part its own
    // next A load refills, issued after this returns), 2, 3 in its 8 KB of
    // the B slot
    QP_PASS(0, C, 0, 2, ra + sw * 8192);
    QP_PASS(0, C, 2, 2, rb + sw * 8192);
  } else {
    const uint32_t w = ra + sw * 8192;
    QP_PASS(0, C, 0, 2, w);
    QP_PASS(0, C, 2, 2, w);
  }
#undef QP_PASS
  wait_lgkm0();  // the read-back is done before a direct load may refill the slot
}

// Output rows (row map) of this lane's MFMA rows, loaded one MFMA phase before
// the epilogue needs them (rows past the tile's end: 0, never stored).
template <int NMI>
__device__ __forceinline__ void qp_rowmap(const QPTile& t, int wm, int (&crow)[4]) {
  QPArgsK* P = qp_args();
  const int32_t* c_map = P->g[t.which].c_map;
  const int lane = qp_lane();
#pragma unroll
  for (int j = 0; j < 4; ++j) crow[j] = 0;
  if (c_map) {
#pragma unroll
    for (int j = 0; j < NMI; ++j) {
      const int m = (2 * j + wm) * 32 + (lane & 31);
      crow[j] = m < t.rows ? ldg_as1(c_map + t.row0 + m) : 0;
    }
  }
}

// ---- group 0: one tile, slabs s .. s + nk - 1, both phases of each.  The
// first even phase also reads the tile's first fragments (slab s is visible:
// its loads were waited for before the previous barrier); the odd phase of
// the last slab runs the epilogue while group 1 computes that slab.  The
// accumulators and fragments are local to the tile, so nothing but the
// loader state is live from one tile to the next.
template <int EPI, int NMI>
__device__ __forceinline__ void qp_tile0(const QPTile& t, QPA& A, const QPList& L, int s, int sw, int wm, int cg,
                                         int lane, uint32_t lds_a) {
  f32x16_t acc[QWCfg<EPI>::NB][4][QWCfg<EPI>::TN];
  QWFrag<EPI> F;
  int crow[4];
  qw_read<EPI, NMI>(F, s, wm, cg, lane);
  wait_lgkm0();
  for (int k = 0; k < t.nk; ++k) {
    // the row map for the epilogue, in flight during the last slab's MFMAs
    // (waited for with this phase's loads)
    if (k == t.nk - 1) qp_rowmap<NMI>(t, wm, crow);
    __builtin_amdgcn_sched_barrier(0);
    // the MFMA wave takes issue precedence over the loading wave on its SIMD
    // (measured on MI355X: about 1 % on both forward GEMMs at C3)
    __builtin_amdgcn_s_setprio(3);
    if (k == 0)
      qw_mma_first<EPI, NMI>(F, acc);
    else
      qw_mma<EPI, NMI>(F, acc);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    wait_vm<0>();  // this wave's part of A(s + k + 1) has landed
    qw_sync();
    if (k + 1 < t.nk) {
      qpa_step(A, L, QWCfg<EPI>::BN, sw, lane, lds_a);
      __builtin_amdgcn_sched_barrier(0);
      qw_read<EPI, NMI>(F, s + k + 1, wm, cg, lane);
      __builtin_amdgcn_sched_barrier(0);
      wait_lgkm0();
      qw_sync();
    }
  }
  // odd phase of the last slab S: epilogue staged in slab S's A and B slots
  // (group 1 read them in the even phase; nothing loads into them until the
  // A load below, A(S + 2) into slab S's A slot), then that load
  __builtin_amdgcn_sched_barrier(0);
  {
    const int S = s + t.nk - 1;
    const uint32_t base = lds_a - sw * QW_LD * 1024;
    qp_epilogue<EPI, NMI, true>(acc, t, crow, sw, wm, cg, base + (S & 1) * QW_REG,
                                base + QW_BOFF + (S % QW_BSLOTS) * QW_REG);
  }
  __builtin_amdgcn_sched_barrier(0);
  qpa_step(A, L, QWCfg<EPI>::BN, sw, lane, lds_a);
  __builtin_amdgcn_sched_barrier(0);
  wait_lgkm0();
  qw_sync();
}

// ---- group 1: one tile, slabs s .. s + nk - 1, both phases of each, then
// the epilogue, which opens the even phase of the next tile's first slab
// (group 0 computes that slab meanwhile; the caller continues the phase with
// the next tile's loads and fragment reads).
template <int EPI, int NMI>
__device__ __forceinline__ void qp_tile1(const QPTile& t, QPB& B, const QPList& L, int s, int sw, int wm, int cg,
                                         int lane, uint32_t lds_b) {
  f32x16_t acc[QWCfg<EPI>::NB][4][QWCfg<EPI>::TN];
  QWFrag<EPI> F;
  int crow[4];
  if (t.nk == 1) qp_rowmap<NMI>(t, wm, crow);
  for (int k = 0; k < t.nk; ++k) {
    const bool issued = qpb_step<QWCfg<EPI>::NB>(B, L, QWCfg<EPI>::BN, sw, lane, lds_b);
    __builtin_amdgcn_sched_barrier(0);
    qw_read<EPI, NMI>(F, s + k, wm, cg, lane);
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm0();
    if (issued)
      wait_vm<QW_LD>();  // B(s + k + 1) (and earlier stores) done; B(s + k + 2) may still be in flight
    else
      wait_vm<0>();
    qw_sync();
    // the row map for the epilogue, in flight from the odd phase of the
    // second-to-last slab (the next even phase's vmcnt wait covers it)
    if (k == t.nk - 2) qp_rowmap<NMI>(t, wm, crow);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(3);
    if (k == 0)
      qw_mma_first<EPI, NMI>(F, acc);
    else
      qw_mma<EPI, NMI>(F, acc);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    qw_sync();
  }
  // start of the even phase of slab S + 1 (S = the tile's last slab): the
  // epilogue staged in slab S's B slot (read by both groups already; B(S + 3)
  // goes there, issued by the caller's next tile after this returns)
  __builtin_amdgcn_sched_barrier(0);
  {
    const int S = s + t.nk - 1;
    const uint32_t base = lds_b - sw * QW_LD * 1024;  // start of the B ring
    qp_epilogue<EPI, NMI, false>(acc, t, crow, sw, wm, cg, base + (S % QW_BSLOTS) * QW_REG, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
}

template <int EPI>
__global__ __launch_bounds__(QW_THREADS) void gemm_qp_kernel(const QPArgs args) {
  (void)args;  // read through qp_args()
  using CF = QWCfg<EPI>;
  constexpr int NB = CF::NB, BN = CF::BN;
  extern __shared__ __attribute__((aligned(16))) char qw_smem[];

  const QPList L = qp_list(BN);
  if (L.ntiles == 0) return;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = wave >> 2, s = wave & 3;        // group, wave in group
  const int wm = s >> 1, cg = (s & 1) * 2 + G;  // row group, column group
  const uint32_t lds_w = lds_addr(qw_smem) + s * QW_LD * 1024;  // this wave's 8 KB of an operand slot

  if (G == 0) {
    // ---- group 0: A loads; computes in even phases
    QPA A;
    A.lt = 0;
    A.ls = 0;
    qpa_rows(A, qp_tile(L, BN, 0), s, lane);
    qpa_step(A, L, BN, s, lane, lds_w);
    qpa_step(A, L, BN, s, lane, lds_w);
    wait_vm<0>();
    qw_sync();  // slab 0 visible
    int sg = 0;  // global index of the tile's first slab
    for (int i = 0; i < L.ntiles; ++i) {
      const QPTile cur = qp_tile(L, BN, i);
      switch (qw_nmi(cur.rows, wm)) {
        case 4: qp_tile0<EPI, 4>(cur, A, L, sg, s, wm, cg, lane, lds_w); break;
        case 3: qp_tile0<EPI, 3>(cur, A, L, sg, s, wm, cg, lane, lds_w); break;
        case 2: qp_tile0<EPI, 2>(cur, A, L, sg, s, wm, cg, lane, lds_w); break;
        case 1: qp_tile0<EPI, 1>(cur, A, L, sg, s, wm, cg, lane, lds_w); break;
        default: qp_tile0<EPI, 0>(cur, A, L, sg, s, wm, cg, lane, lds_w); break;
      }
      sg += cur.nk;
    }
  } else {
    // ---- group 1: B loads; computes in odd phases
    QPB B;
    B.lt = 0;
    B.ls = 0;
    qpb_set<NB>(B, qp_tile(L, BN, 0), s, lane);
    qpb_step<NB>(B, L, BN, s, lane, lds_w + QW_BOFF);
    if (qpb_step<NB>(B, L, BN, s, lane, lds_w + QW_BOFF))
      wait_vm<QW_LD>();
    else
      wait_vm<0>();
    qw_sync();  // slab 0 visible
    int sg = 0;  // global index of the tile's first slab
    for (int i = 0; i < L.ntiles; ++i) {
      const QPTile cur = qp_tile(L, BN, i);
      switch (qw_nmi(cur.rows, wm)) {
        case 4: qp_tile1<EPI, 4>(cur, B, L, sg, s, wm, cg, lane, lds_w + QW_BOFF); break;
        case 3: qp_tile1<EPI, 3>(cur, B, L, sg, s, wm, cg, lane, lds_w + QW_BOFF); break;
        case 2: qp_tile1<EPI, 2>(cur, B, L, sg, s, wm, cg, lane, lds_w + QW_BOFF); break;
        case 1: qp_tile1<EPI, 1>(cur, B, L, sg, s, wm, cg, lane, lds_w + QW_BOFF); break;
        default: qp_tile1<EPI, 0>(cur, B, L, sg, s, wm, cg, lane, lds_w + QW_BOFF); break;
      }
      sg += cur.nk;
    }
  }
}

// Requirements beyond mfma_ok (gemm.hip): at most QW_MAX_SEG K segments, K
// and the segment length multiples of 64, 32-bit byte offsets into A and into
// every B block, and 16-byte aligned output rows and column groups.
bool gemm_qp_ok(const GemmDesc& g) {
  const int64_t lim = int64_t(1) << 31;
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  return g.nseg >= 1 && g.nseg <= QW_MAX_SEG && g.K % QW_BK == 0 && g.kseg % QW_BK == 0 && g.a_rows * g.lda < lim &&
         (int64_t)g.N * g.ldb < lim && g.bm == QW_BM && g.N % 8 == 0 && g.ldc % 8 == 0 && g.c_group_col % 8 == 0 &&
         a16(g.C) && a16(g.Gs) && a16(g.Us);
}

static int qp_grid() {
  static std::atomic<int> ncu{0};
  int n = ncu.load(std::memory_order_relaxed);
  if (n == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    ncu.store(n, std::memory_order_relaxed);
  }
  return (int)(8 * cdiv(n, 8));
}

template <int EPI>
static int qp_launch(const GemmDesc& g0, const GemmDesc& g1, int pair, const float* row_scale, hipStream_t st) {
  static const hipError_t attr = hipFuncSetAttribute((const void*)gemm_qp_kernel<EPI>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)QW_LDS);
  if (attr != hipSuccess) return fail(DSMOE_ERR_HIP, "gemm_qp: cannot raise LDS limit");
  QPArgs a;
  a.g[0] = g0;
  a.g[1] = g1;
  a.row_scale = row_scale;
  a.pair = pair;
  hipLaunchKernelGGL(gemm_qp_kernel<EPI>, dim3((unsigned)qp_grid()), dim3(QW_THREADS), QW_LDS, st, a);
  return check_launch("gemm_qp");
}

int launch_gemm_qp(const GemmDesc& g, int epi, const float* row_scale, hipStream_t st) {
  return epi == EPI_SWIGLU ? qp_launch<EPI_SWIGLU>(g, g, 0, row_scale, st)
                           : qp_launch<EPI_STORE>(g, g, 0, row_scale, st);
}

int launch_gemm_qp_pair(const GemmDesc& gr, const GemmDesc& gd, int epi, const float* row_scale, hipStream_t st) {
  return epi == EPI_SWIGLU ? qp_launch<EPI_SWIGLU>(gr, gd, 1, row_scale, st)
                           : qp_launch<EPI_STORE>(gr, gd, 1, row_scale, st);
}

}  // namespace dsmoe
