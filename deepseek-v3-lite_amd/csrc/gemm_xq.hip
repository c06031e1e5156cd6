// Backward grouped GEMMs on gfx950, quad-wave design (four waves, one per
// SIMD, each owning 128 x 128 of a 256 x 256 tile; K slabs of 64 streamed
// into separate A and B LDS rings by direct
// global -> LDS loads; fragment reads two K steps ahead of the MFMAs;
// LDS-staged, whole-row epilogues) extended to operands whose reduction
// index K is the ROW index of the stored matrix ("K-major", KM):
//   dh   = dY W2            A = dY rows (K contiguous)     B(n=i, k=d) = W2[d][i]
//   dx   = [dg|du][W1;W3]   A = [dg|du] rows               B(n=d, k=i) = W1[i][d] / W3[i][d]
//   dW13 = [dg|du]^T X      A(m=i, k=r) = dgdu[r][i]       B(n=d, k=r) = Xs[r][d]
//   dW2  = (w dY)^T H       A(m=d, k=r) = dYw[r][d]        B(n=i, k=r) = H[r][i]
// (models/moe.py:127-131 under autograd; models/moe_triton.py:142-374.)
// Every KM operand is read with identity rows: the layer materialises the
// routed rows of X in sorted order (forward) and w * dY in sorted order
// (backward preparation), so a KM slab is 64 consecutive rows of 512 bytes.
//
// KM slabs are stored untransposed, [64 k][256 columns], 512-byte rows, and
// gfx950's transposing LDS read (ds_read_b64_tr_b16) builds the MFMA
// fragment: within each 16-lane group, lane s supplies the 8-byte address of
// row k0 + (s >> 2), columns c0 + 4 (s & 3) .. +3, and lane i receives the
// column c0 + i of the four rows.  Two such reads (k0 and k0 + 4) give a
// lane its 8 consecutive k of one column, the v_mfma_f32_32x32x16_bf16
// operand layout.  8-byte unit u of k row r is stored at unit u ^ 8 (r & 3):
// the 32 lanes of a half-wave read 4 rows x 8 units that land on 32
// distinct bank pairs, and the 16-byte chunks a direct load writes stay
// contiguous (the XOR leaves unit bits 0-2 alone).
//
// Weight-gradient K ranges (an expert's rows) are ragged: A rows past the
// range are read from a zero block instead, so their products vanish.
//
// Determinism: one block owns each output tile and walks its K range in
// ascending order (fp32 accumulation, one rounding); split-K partials of the
// shared-expert weight gradients are added in ascending part order by
// wgrad_reduce_kernel.
#include <algorithm>
#include <atomic>

#include "gemm_tile.h"
#include "mfma.h"

namespace dsmoe {

constexpr int XQ_BM = 256, XQ_BN = 256;
constexpr int XQ_BK = 64;                             // K per slab
constexpr int XQ_REG = 32 * 1024;                     // one operand of a slab
constexpr int XQ_ASLOTS = 2, XQ_BSLOTS = 3;
constexpr int XQ_BOFF = XQ_ASLOTS * XQ_REG;
constexpr size_t XQ_LDS = (size_t)(XQ_ASLOTS + XQ_BSLOTS) * XQ_REG;  // 160 KB (the epilogue reuses it)
constexpr int XQ_LD = XQ_REG / 1024 / 4;              // direct loads per wave, operand and slab (8)

// A block of zeros: the source of weight-gradient A rows past the K range.
__device__ __attribute__((aligned(16))) uint4 g_xq_zero[4];
// 1.0: the row weight of an unweighted SwiGLU-backward epilogue.
__device__ float g_xq_one[1] = {1.0f};
// Where the SwiGLU-backward epilogue stores elements outside its tile (never
// read): 16 bytes per thread of 64 workgroup slots, so the out-of-tile stores
// of a ragged tile spread over 256 KB instead of meeting in one cache line.
constexpr int XQ_SINK_SLOTS = 64;
__device__ __attribute__((aligned(16))) uint4 g_xq_sink[XQ_SINK_SLOTS * 256];

typedef short xq_v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) u32x4_t xq_gv4u;  // a global-memory u32x4_t

// K-contiguous ("NT") slab: [256 rows][64 k], 128-byte rows, 16-byte chunk c
// of row r at chunk c ^ ((r >> 1) & 7).
__device__ __forceinline__ int xq_nt(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }
// K-major slab: [64 k][256 columns], 512-byte rows; 8-byte unit u of row k at
// unit u ^ 8 (k & 3).  Byte offset of the 8 bytes holding columns 4u .. 4u+3.
__device__ __forceinline__ int xq_km(int k, int u) { return k * 512 + ((u ^ ((k & 3) << 3)) << 3); }

__device__ __forceinline__ xq_v4s xq_tr(const char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) xq_v4s*)p);
}

// MFMA fragment of a KM slab region: 32 columns c0 .. c0+31 (lane l: column
// c0 + (l & 31)) at k0 + 8 (l >> 5) .. +7.
__device__ __forceinline__ bf16x8_t xq_km_frag(const char* reg, int k0, int c0, int lane) {
  const int gq = lane >> 4, s = lane & 15;
  const int k = k0 + 8 * (gq >> 1) + (s >> 2);
  const int u = (c0 >> 2) + 4 * (gq & 1) + (s & 3);
  const xq_v4s lo = xq_tr(reg + xq_km(k, u));
  const xq_v4s hi = xq_tr(reg + xq_km(k + 4, u));
  typedef short v8s __attribute__((ext_vector_type(8)));
  const v8s v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8_t, v);
}

// Direct-load sources of one wave.  Wave w fills rows 64 w .. 64 w + 63 of an
// NT region, or k rows 16 w .. 16 w + 15 of a KM region (load i: rows
// 16 w + 2 i + (l >> 5)).
struct XQLoad {
  const bf16_t* a;        // A base (KM: + group column offset)
  int64_t a_ld;           // KM: elements per k row
  const bf16_t* b0;       // B, K segment 0 (weights) or matrix base (+ group column offset)
  const bf16_t* b1;       // B, last K segment
  int64_t b_ld;
  uint32_t offa[XQ_LD];   // NT: row * lda + chunk (KM: unused)
  uint32_t kma[2];        // KM A: offset of load i = kma[i & 1] + 2 i lda  (= k_i * lda + column)
  uint32_t kmb[2];        // B: offset of load i = kmb[i & 1] + 2 i ldb  (= k_i * ldb + column)
  int kseg;               // K at which b1 takes over (0x7fffffff: one segment)
  int kbeg, kend, nk;
  int g0;                 // persistent loop: ring index of the tile's first slab (ring index - g0 = K slab)
  int lds_off;            // byte offset of this wave's 8 KB inside an operand region
  int krow0;              // KM: first k row of this wave's loads (16 w)
};

template <int AMODE, int I0, int I1>
__device__ __forceinline__ void xq_issue_a(const XQLoad& L, int ka, int lane) {
  extern __shared__ __attribute__((aligned(16))) char xq_smem[];
  const uint32_t da = lds_addr(xq_smem) + L.lds_off + (ka & 1) * XQ_REG;
  const int k0 = L.kbeg + min(ka, L.nk - 1) * XQ_BK;
#pragma unroll
  for (int i = I0; i < I1; ++i) {
    const bf16_t* src;
    if (AMODE == XA_ROWS) {
      src = L.a + L.offa[i] + k0;
    } else {
      // rows past the K range read zeros (weight-gradient tails)
      const int kr = k0 + L.krow0 + 2 * i + (lane >> 5);
      const uint32_t off = L.kma[i & 1] + (uint32_t)(2 * i) * (uint32_t)L.a_ld;
      src = kr < L.kend ? L.a + (int64_t)k0 * L.a_ld + off : reinterpret_cast<const bf16_t*>(g_xq_zero);
    }
    dma16(src, da + i * 1024);
  }
}

template <int BMODE, int I0, int I1>
__device__ __forceinline__ void xq_issue_b(const XQLoad& L, int kb, int lane) {
  extern __shared__ __attribute__((aligned(16))) char xq_smem[];
  const uint32_t db = lds_addr(xq_smem) + L.lds_off + XQ_BOFF + (kb % XQ_BSLOTS) * XQ_REG;
  const int k0 = L.kbeg + min(kb, L.nk - 1) * XQ_BK;
  const bool hi = k0 >= L.kseg;
  const bf16_t* src = (hi ? L.b1 : L.b0) + (int64_t)(hi ? k0 - L.kseg : k0) * L.b_ld;
#pragma unroll
  for (int i = I0; i < I1; ++i) {
    const bf16_t* p = src + (L.kmb[i & 1] + (uint32_t)(2 * i) * (uint32_t)L.b_ld);
    if (BMODE == XB_ACT_KMAJOR) {
      // activation rows past the K range (the last one may be the matrix's
      // last row) are not read: zeros instead
      const int kr = k0 + L.krow0 + 2 * i + (lane >> 5);
      if (kr >= L.kend) p = reinterpret_cast<const bf16_t*>(g_xq_zero);
    }
    dma16(p, db + i * 1024);
  }
}


template <int AMODE>
__device__ __forceinline__ void xq_issue_a_one(const XQLoad& L, int ka, int lane, int i) {
  extern __shared__ __attribute__((aligned(16))) char xq_smem[];
  const uint32_t da = lds_addr(xq_smem) + L.lds_off + (ka & 1) * XQ_REG;
  const int k0 = L.kbeg + min(ka, L.nk - 1) * XQ_BK;
  const bf16_t* src;
  if (AMODE == XA_ROWS) {
    src = L.a + L.offa[i] + k0;
  } else {
    const int kr = k0 + L.krow0 + 2 * i + (lane >> 5);
    const uint32_t off = L.kma[i & 1] + (uint32_t)(2 * i) * (uint32_t)L.a_ld;
    src = kr < L.kend ? L.a + (int64_t)k0 * L.a_ld + off : reinterpret_cast<const bf16_t*>(g_xq_zero);
  }
  dma16(src, da + i * 1024);
}

template <int BMODE>
__device__ __forceinline__ void xq_issue_b_one(const XQLoad& L, int kb, int lane, int i) {
  extern __shared__ __attribute__((aligned(16))) char xq_smem[];
  const uint32_t db = lds_addr(xq_smem) + L.lds_off + XQ_BOFF + (kb % XQ_BSLOTS) * XQ_REG;
  const int k0 = L.kbeg + min(kb, L.nk - 1) * XQ_BK;
  const bool hi = k0 >= L.kseg;
  const bf16_t* p = (hi ? L.b1 : L.b0) + (int64_t)(hi ? k0 - L.kseg : k0) * L.b_ld +
                    (L.kmb[i & 1] + (uint32_t)(2 * i) * (uint32_t)L.b_ld);
  if (BMODE == XB_ACT_KMAJOR) {
    const int kr = k0 + L.krow0 + 2 * i + (lane >> 5);
    if (kr >= L.kend) p = reinterpret_cast<const bf16_t*>(g_xq_zero);
  }
  dma16(p, db + i * 1024);
}

// Fragments of K step s (0..3) of slab kb: A sub-tiles j < NMI (rows
// (2j + wm) * 32 ..), B tiles ni (columns wn * 128 + 32 ni ..).
template <int AMODE, int NMI>
__device__ __forceinline__ void xq_read(int kb, int s, int wm, int wn, int lane, bf16x8_t (&fa)[4],
                                        bf16x8_t (&fb)[4]) {
  extern __shared__ __attribute__((aligned(16))) char xq_smem[];
  if (NMI == 0) return;
  const char* sA = xq_smem + (kb & 1) * XQ_REG;
  const char* sB = xq_smem + XQ_BOFF + (kb % XQ_BSLOTS) * XQ_REG;
#pragma unroll
  for (int j = 0; j < NMI; ++j) {
    if (AMODE == XA_ROWS)
      fa[j] = *reinterpret_cast<const bf16x8_t*>(sA + xq_nt((2 * j + wm) * 32 + (lane & 31), s * 2 + (lane >> 5)));
    else
      fa[j] = xq_km_frag(sA, s * 16, (2 * j + wm) * 32, lane);
  }
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) fb[ni] = xq_km_frag(sB, s * 16, wn * 128 + ni * 32, lane);
}

// MFMAs T0 .. T1-1 of one K step, t = j * 4 + ni.
template <int NMI, int T0 = 0, int T1 = NMI * 4>
__device__ __forceinline__ void xq_mma(const bf16x8_t (&fa)[4], const bf16x8_t (&fb)[4], f32x16_t (&acc)[4][4]) {
#pragma unroll
  for (int t = T0; t < T1; ++t)
    acc[t / 4][t % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[t % 4], fa[t / 4], acc[t / 4][t % 4], 0, 0, 0);
}

// MFMAs T0 .. T1-1 of one K step (MMAS per step, t = j * 4 + ni).  With
// NL > 0, load i of the step's NL direct loads (index LI0 + i of A (LK 0) or
// B (LK 1) of slab kl) follows MFMA floor(i * MMAS / NL).
template <int AMODE, int NMI, int T0, int T1, int NL, int LK, int LI0>
__device__ __forceinline__ void xq_mma_ld(const bf16x8_t (&fa)[4], const bf16x8_t (&fb)[4], f32x16_t (&acc)[4][4],
                                          const XQLoad& L, int kl, int lane) {
  constexpr int MMAS = NMI * 4;
  constexpr int BM = AMODE == XA_ROWS ? XB_W_NN : XB_ACT_KMAJOR;
#pragma unroll
  for (int t = T0; t < T1; ++t) {
    acc[t / 4][t % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[t % 4], fa[t / 4], acc[t / 4][t % 4], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      if ((i * MMAS / (NL > 0 ? NL : 1)) == t) {
        __builtin_amdgcn_sched_barrier(0);
        if (LK == 0) xq_issue_a_one<AMODE>(L, kl, lane, LI0 + i); else xq_issue_b_one<BM>(L, kl, lane, LI0 + i);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

__device__ __forceinline__ void xq_sync() {
  __builtin_amdgcn_sched_barrier(0);
  lds_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

struct XQPipe {
  bf16x8_t fa[3][4];
  bf16x8_t fb[3][4];
};

// One slab whose step 0 uses register set S0 (reads run two steps ahead; the barrier follows step 1; the
// refills of slab kb + 2 are spread over the slab, B(kb + 2) during steps 0
// and 1 into slab kb - 1's slot, A(kb + 2) during steps 2 and 3 into slab
// kb's).
template <int AMODE, int NMI, int S0>
__device__ __forceinline__ void xq_slab(XQPipe& P, const XQLoad& L, int kb, int wm, int wn, int lane,
                                        f32x16_t (&acc)[4][4]) {
  constexpr int MMAS = NMI * 4;
  constexpr int A0 = S0 % 3, A1 = (S0 + 1) % 3, A2 = (S0 + 2) % 3;
  constexpr int NL = XQ_LD / 2;
  constexpr int BM = AMODE == XA_ROWS ? XB_W_NN : XB_ACT_KMAJOR;
  __builtin_amdgcn_sched_barrier(0);
  xq_read<AMODE, NMI>(kb, 2, wm, wn, lane, P.fa[A2], P.fb[A2]);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (MMAS > 0) {
    xq_mma_ld<AMODE, NMI, 0, MMAS, NL, 1, 0>(P.fa[A0], P.fb[A0], acc, L, kb + 2, lane);
  } else {
#pragma unroll
    for (int i = 0; i < NL; ++i) xq_issue_b_one<BM>(L, kb + 2, lane, i);
  }
  __builtin_amdgcn_sched_barrier(0);
  xq_read<AMODE, NMI>(kb, 3, wm, wn, lane, P.fa[A0], P.fb[A0]);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (MMAS > 0) {
    xq_mma_ld<AMODE, NMI, 0, MMAS, NL, 1, NL>(P.fa[A1], P.fb[A1], acc, L, kb + 2, lane);
  } else {
#pragma unroll
    for (int i = 0; i < NL; ++i) xq_issue_b_one<BM>(L, kb + 2, lane, NL + i);
  }
  __builtin_amdgcn_sched_barrier(0);
  // all reads of slab kb issued: wait for them and for this wave's loads of
  // A(kb + 1) and B(kb + 1) (only the 8 B(kb + 2) loads are younger); then
  // slab kb + 1 is visible and slab kb's slots are free
  wait_lgkm0();
  wait_vm<XQ_LD>();
  xq_sync();
  if constexpr (MMAS > 0) {
    constexpr int H = MMAS < 4 ? MMAS : 4;
    xq_mma_ld<AMODE, NMI, 0, H, NL, 0, 0>(P.fa[A2], P.fb[A2], acc, L, kb + 2, lane);
    __builtin_amdgcn_sched_barrier(0);
    xq_read<AMODE, NMI>(kb + 1, 0, wm, wn, lane, P.fa[A1], P.fb[A1]);
    __builtin_amdgcn_sched_barrier(0);
    xq_mma_ld<AMODE, NMI, H, MMAS, NL, 0, 0>(P.fa[A2], P.fb[A2], acc, L, kb + 2, lane);
    __builtin_amdgcn_sched_barrier(0);
    xq_read<AMODE, NMI>(kb + 1, 1, wm, wn, lane, P.fa[A2], P.fb[A2]);
    __builtin_amdgcn_sched_barrier(0);
    xq_mma_ld<AMODE, NMI, 0, MMAS, NL, 0, NL>(P.fa[A0], P.fb[A0], acc, L, kb + 2, lane);
  } else {
    xq_issue_a<AMODE, 0, XQ_LD>(L, kb + 2, lane);
  }
}

template <int AMODE, int NMI>
__device__ __forceinline__ void xq_loop(const XQLoad& L, int wm, int wn, int lane, f32x16_t (&acc)[4][4]) {
  XQPipe P;
  xq_read<AMODE, NMI>(0, 0, wm, wn, lane, P.fa[0], P.fb[0]);
  xq_read<AMODE, NMI>(0, 1, wm, wn, lane, P.fa[1], P.fb[1]);
  wait_lgkm0();  // no scalar load in flight at the loop head (see qw_loop)
  int kb = 0;
  for (; kb + 3 <= L.nk; kb += 3) {
    xq_slab<AMODE, NMI, 0>(P, L, kb, wm, wn, lane, acc);
    xq_slab<AMODE, NMI, 1>(P, L, kb + 1, wm, wn, lane, acc);
    xq_slab<AMODE, NMI, 2>(P, L, kb + 2, wm, wn, lane, acc);
  }
  if (kb < L.nk) xq_slab<AMODE, NMI, 0>(P, L, kb, wm, wn, lane, acc);
  if (kb + 1 < L.nk) xq_slab<AMODE, NMI, 1>(P, L, kb + 1, wm, wn, lane, acc);
  __builtin_amdgcn_sched_barrier(0);
  wait_vm<0>();
}

template <int EPI, int AMODE>
__global__ __launch_bounds__(256) void xgemm_q_kernel(const XGemm g) {
  extern __shared__ __attribute__((aligned(16))) char xq_smem[];
  int grp, row0, rows, n_tile, kbeg, kend, split;
  if (!xtile<XQ_BM, XQ_BN>(g, grp, row0, rows, n_tile, kbeg, kend, split)) return;
  grp = __builtin_amdgcn_readfirstlane(grp);
  row0 = __builtin_amdgcn_readfirstlane(row0);
  rows = __builtin_amdgcn_readfirstlane(rows);
  n_tile = __builtin_amdgcn_readfirstlane(n_tile);
  kbeg = __builtin_amdgcn_readfirstlane(kbeg);
  kend = __builtin_amdgcn_readfirstlane(kend);
  split = __builtin_amdgcn_readfirstlane(split);
  const int n0 = n_tile * XQ_BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  XQLoad L;
  L.kbeg = kbeg;
  L.kend = kend;
  L.nk = (kend > kbeg) ? (int)cdiv(kend - kbeg, XQ_BK) : 0;
  L.lds_off = wave * XQ_LD * 1024;
  L.krow0 = wave * 16;
  constexpr int BM = AMODE == XA_ROWS ? XB_W_NN : XB_ACT_KMAJOR;  // B mode paired with the A mode
  // ---- A sources
  if (AMODE == XA_ROWS) {
    // wave w: rows 64 w + 8 i + (l >> 3), chunk (l & 7) of 128-byte rows
    L.a = static_cast<const bf16_t*>(g.A);
    L.a_ld = g.lda;
#pragma unroll
    for (int i = 0; i < XQ_LD; ++i) {
      const int r = (wave * XQ_LD + i) * 8 + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      const int ra = min(r, rows - 1);
      const int64_t arow = g.a_map ? (int64_t)g.a_map[row0 + ra] : (int64_t)(row0 + ra);
      L.offa[i] = (uint32_t)(arow * g.lda + c * 8);
    }
  } else {
    // KM: k rows 16 w + 2 i + (l >> 5), 16-byte chunk (l & 31) of 512-byte
    // rows; the chunk swizzle depends on k & 3, i.e. on the parity of i
    L.a = static_cast<const bf16_t*>(g.A) + (int64_t)grp * g.a_col;
    L.a_ld = g.lda;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      // load i reads k row k_i = 16 w + 2 i + (l >> 5), whose swizzle depends
      // on k_i & 3, i.e. on par = i & 1; the 2 i rows go into the per-load term
      const int kr = wave * 16 + (lane >> 5);
      const int c = (lane & 31) ^ (((kr + 2 * par) & 3) << 2);
      const int m = min(row0 + 8 * c, g.M - 8);  // output rows are columns of the stored A
      L.kma[par] = (uint32_t)((int64_t)kr * g.lda + m);
    }
  }
  // ---- B sources (always KM)
  if (BM == XB_W_NN) {
    const void* const* tab = g.Btab + (int64_t)grp * g.nseg;
    L.b0 = static_cast<const bf16_t*>(tab[0]);
    L.b1 = static_cast<const bf16_t*>(tab[g.nseg - 1]);
    L.kseg = g.nseg > 1 ? g.kseg : 0x7fffffff;
  } else {
    L.b0 = L.b1 = static_cast<const bf16_t*>(g.Bact) + (int64_t)grp * g.b_col;
    L.kseg = 0x7fffffff;
  }
  L.b_ld = g.ldb;
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int kr = wave * 16 + (lane >> 5);
    const int c = (lane & 31) ^ (((kr + 2 * par) & 3) << 2);
    const int n = min(n0 + 8 * c, g.N - 8);
    L.kmb[par] = (uint32_t)((int64_t)kr * g.ldb + n);
  }

  f32x16_t acc[4][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[j][ni][r] = 0.0f;

  if (L.nk > 0) {
    // ---- prologue: A(0), B(0) and A(1), B(1) in flight together; slab 0
    // visible to all waves
    xq_issue_a<AMODE, 0, XQ_LD>(L, 0, lane);
    xq_issue_b<BM, 0, XQ_LD>(L, 0, lane);
    xq_issue_a<AMODE, 0, XQ_LD>(L, 1, lane);
    xq_issue_b<BM, 0, XQ_LD>(L, 1, lane);
    wait_vm<2 * XQ_LD>();
    xq_sync();
    // active row sub-tiles of this wave; none when its 128 columns all lie
    // past N (the last column tile of N = 1408, for instance)
    const int nsub = (int)cdiv(rows, 32);
    const int nmi = (n0 + wn * 128 >= g.N) ? 0 : max(0, min(4, (nsub - wm + 1) >> 1));
    switch (nmi) {
      case 4: xq_loop<AMODE, 4>(L, wm, wn, lane, acc); break;
      case 3: xq_loop<AMODE, 3>(L, wm, wn, lane, acc); break;
      case 2: xq_loop<AMODE, 2>(L, wm, wn, lane, acc); break;
      case 1: xq_loop<AMODE, 1>(L, wm, wn, lane, acc); break;
      default: xq_loop<AMODE, 0>(L, wm, wn, lane, acc); break;
    }
  }

  // ---- epilogue.  Lane holds tile row m = (2j + wm) * 32 + (lane & 31) and,
  // per q, columns n = wn * 128 + 32 ni + 8 q + 4 (lane >> 5) + {0..3}
  // (registers 4q .. 4q+3).  Split-K partials, and fp32 weight gradients,
  // go straight out as fp32.
  if (EPI == XE_WGRAD && (g.ksplit > 1 || g.c_f32)) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = (2 * j + wm) * 32 + (lane & 31);
      if (m >= rows) continue;
      const int r = row0 + m;
      float* prow = g.ksplit > 1
                        ? g.part + (((int64_t)split * g.groups + grp) * g.M + r) * g.N
                        : static_cast<float*>(r < g.msplit ? g.Ctab0[grp] : g.Ctab1[grp]) +
                              (int64_t)(r < g.msplit ? r : r - g.msplit) * g.ldc;
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n0 + wn * 128 + ni * 32 + q * 8 + (lane >> 5) * 4;
          if (n < g.N)
            *reinterpret_cast<float4*>(prow + n) =
                make_float4(acc[j][ni][q * 4], acc[j][ni][q * 4 + 1], acc[j][ni][q * 4 + 2], acc[j][ni][q * 4 + 3]);
        }
    }
    return;
  }
  // Otherwise the tile goes through LDS and leaves as whole rows; output row
  // pointers are resolved once per row.
  __builtin_amdgcn_sched_barrier(0);
  wait_lgkm0();
  xq_sync();  // every wave is done with the slab buffers
  char* sm = xq_smem;
  int64_t* rowp = reinterpret_cast<int64_t*>(sm + 128 * 1024);  // past the staged tile (<= 128 KB)
  int64_t my_rowp;
  {
    const int r = row0 + min(tid, rows - 1);
    if (EPI == XE_WGRAD)
      my_rowp = reinterpret_cast<int64_t>(static_cast<bf16_t*>(r < g.msplit ? g.Ctab0[grp] : g.Ctab1[grp]) +
                                          (int64_t)(r < g.msplit ? r : r - g.msplit) * g.ldc);
    else
      my_rowp = reinterpret_cast<int64_t>(static_cast<bf16_t*>(g.C) + (int64_t)grp * g.c_group_col +
                                          (g.c_map ? (int64_t)g.c_map[r] : (int64_t)r) * g.ldc);
  }
  if (EPI != XE_SWIGLU_BWD) {
    // bf16 tile, 256 rows x 512 bytes; 8-byte unit u of row m at unit u ^ (m & 31)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = (2 * j + wm) * 32 + (lane & 31);
#pragma unroll
      for (int ni = 0; ni < 4; ++ni)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int u = (wn * 128 + ni * 32 + q * 8 + (lane >> 5) * 4) >> 2;
          u32x2_t w;
          w.x = pack_bf16x2(acc[j][ni][q * 4], acc[j][ni][q * 4 + 1]);
          w.y = pack_bf16x2(acc[j][ni][q * 4 + 2], acc[j][ni][q * 4 + 3]);
          *reinterpret_cast<u32x2_t*>(sm + m * 512 + ((u ^ (m & 31)) << 3)) = w;
        }
    }
    rowp[tid] = my_rowp;
    xq_sync();
    // 32 lanes per row, 16 bytes each; 8 rows per pass
    const int cc = tid & 31, n = n0 + cc * 8;
#pragma unroll 4
    for (int r = tid >> 5; r < rows; r += 8) {
      const int pu = (2 * cc) ^ (r & 31);
      u32x4_t v = *reinterpret_cast<const u32x4_t*>(sm + r * 512 + ((pu >> 1) << 4));
      if (r & 1) v = u32x4_t{v.z, v.w, v.x, v.y};
      if (n < g.N) *reinterpret_cast<u32x4_t*>(reinterpret_cast<bf16_t*>(rowp[r]) + n) = v;
    }
    return;
  }
  // SwiGLU backward: dh stays fp32 until dg and du are formed, so the tile is
  // staged as fp32 one column quarter (64 columns, owned by the waves with
  // wn == quarter / 2) at a time; 16-byte unit u of row m at unit u ^ (m & 15).
  // Thread tid serves rows (tid >> 3) + 32 i and columns n0 + 64 quarter +
  // 8 (tid & 7) + {0..7}.  The g and u of quarter q + 1 are loaded while
  // quarter q is staged, formed and stored, so only the first quarter waits
  // for its loads.  All four quarters run, and the body has no branches:
  // loads read a clamped row and column, and an element outside the tile is
  // stored to g_xq_sink.  The compiler then knows how many memory operations
  // follow each load and waits for that load alone (a load or store under a
  // lane guard makes it wait for all of them).
  const bf16_t* Gs = static_cast<const bf16_t*>(g.Gs);
  const bf16_t* Us = static_cast<const bf16_t*>(g.Us);
  const uint4* sink = g_xq_sink + (blockIdx.x % XQ_SINK_SLOTS) * 256 + tid;
  rowp[tid] = my_rowp;
  const int cc = tid & 7, rq = tid >> 3;
  // row weights, or a stride-0 read of 1.0 when there are none
  const float* rw_base = g.row_w ? g.row_w : g_xq_one;
  const int rw_step = g.row_w ? 1 : 0;
  float rwv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) rwv[i] = rw_base[(row0 + min(rq + 32 * i, rows - 1)) * rw_step];
  u32x4_t gp[2][8], up[2][8];
  int64_t rpv[8];  // output row addresses of the thread's rows
  auto issue = [&](int qt, u32x4_t (&gq)[8], u32x4_t (&uq)[8]) {
    const int nc = min(n0 + qt * 64 + cc * 8, g.N - 8);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = min(rq + 32 * i, rows - 1);
      const int64_t ogu = (int64_t)(row0 + r) * g.ld_gu + (int64_t)grp * g.gu_group_col + nc;
      gq[i] = *reinterpret_cast<const u32x4_t*>(Gs + ogu);
      uq[i] = *reinterpret_cast<const u32x4_t*>(Us + ogu);
    }
  };
  issue(0, gp[0], up[0]);
#pragma unroll
  for (int qt = 0; qt < 4; ++qt) {
    if (qt + 1 < 4) issue(qt + 1, gp[(qt + 1) & 1], up[(qt + 1) & 1]);
    if (qt) xq_sync();  // the previous quarter's reads are done
    if (wn == (qt >> 1)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = (2 * j + wm) * 32 + (lane & 31);
#pragma unroll
        for (int nl = 0; nl < 2; ++nl)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int ni = 2 * (qt & 1) + nl;
            const int u = nl * 8 + q * 2 + (lane >> 5);
            *reinterpret_cast<float4*>(sm + m * 256 + ((u ^ (m & 15)) << 4)) =
                make_float4(acc[j][ni][q * 4], acc[j][ni][q * 4 + 1], acc[j][ni][q * 4 + 2], acc[j][ni][q * 4 + 3]);
          }
      }
    }
    xq_sync();
    if (qt == 0)
#pragma unroll
      for (int i = 0; i < 8; ++i) rpv[i] = rowp[rq + 32 * i];
    const int n = n0 + qt * 64 + cc * 8;
    const bool col_ok = n < g.N;
    const u32x4_t(&gq)[8] = gp[qt & 1];
    const u32x4_t(&uq)[8] = up[qt & 1];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = rq + 32 * i;
      const bool ok = r < rows && col_ok;
      const float4 d0 = *reinterpret_cast<const float4*>(sm + r * 256 + (((2 * cc) ^ (r & 15)) << 4));
      const float4 d1 = *reinterpret_cast<const float4*>(sm + r * 256 + (((2 * cc + 1) ^ (r & 15)) << 4));
      const float dhv[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
      const uint32_t gw[4] = {gq[i].x, gq[i].y, gq[i].z, gq[i].w};
      const uint32_t uw[4] = {uq[i].x, uq[i].y, uq[i].z, uq[i].w};
      uint32_t dgw[4], duw[4];
#pragma unroll
      for (int e2 = 0; e2 < 4; ++e2) {
        float dg[2], du[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float gv = __uint_as_float(h ? (gw[e2] & 0xffff0000u) : (gw[e2] << 16));
          const float uv = __uint_as_float(h ? (uw[e2] & 0xffff0000u) : (uw[e2] << 16));
          const float dh = rwv[i] * dhv[2 * e2 + h];
          const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-gv));  // 1 ulp; dg, du are rounded to bf16
          dg[h] = dh * uv * sg * (1.0f + gv * (1.0f - sg));
          du[h] = dh * gv * sg;
        }
        dgw[e2] = pack_bf16x2(dg[0], dg[1]);
        duw[e2] = pack_bf16x2(du[0], du[1]);
      }
      // global (not flat) stores: a flat store also counts as an LDS access
      const int64_t dst = ok ? rpv[i] + 2 * (int64_t)n : reinterpret_cast<int64_t>(sink);
      const int64_t du_bytes = ok ? 2 * g.du_off : 0;
      *reinterpret_cast<xq_gv4u*>(dst) = u32x4_t{dgw[0], dgw[1], dgw[2], dgw[3]};
      *reinterpret_cast<xq_gv4u*>(dst + du_bytes) = u32x4_t{duw[0], duw[1], duw[2], duw[3]};
    }
  }
}

// ------------------------------------------------- persistent weight gradients
// Weight gradients without split-K (each routed expert's dW1 | dW3 and dW2)
// as a persistent loop.  One workgroup per CU walks the tiles of virtual
// blocks blockIdx.x, blockIdx.x + gridDim.x, ... (the XCD-chunked order of
// one block per tile; gridDim.x is a multiple of 8, so every virtual block
// stays on its block's XCD).  The ring index counts the slabs of all the
// workgroup's tiles in a row: the loads issued during a tile's last two slabs
// fetch the next tile's first two, so no tile after the first waits for its
// first slab, and the epilogue's stores drain while the next tile computes
// (one block per tile paid about 10 us per tile for its first slab, its
// epilogue and the block's launch).  Every tile runs at least two slabs (rows
// past its K range read zeros), so the loads never run more than one tile
// ahead.  All four waves compute every tile; rows past M and columns past N
// read clamped operands and are not stored.  A tile sums the same products
// in the same order as xgemm_q_kernel, so the outputs are bitwise the same.
//
// The slab keeps one fragment register set per K step (xgemm_q_kernel
// rotates three), so every slab starts in the same sets and the loop has one
// slab body beside the tile's first.

struct XQTileW {
  int grp, row0, rows, n0, kbeg, kend;
};

// Tile of virtual block vb; false when vb has none.  Scalar values only.
__device__ __forceinline__ bool xq_wgrad_tile(const XGemm& g, int64_t vb, XQTileW& t) {
  int grp, row0, rows, n_tile, kbeg, kend, split;
  if (!xtile_at<XQ_BM, XQ_BN>(g, vb, grp, row0, rows, n_tile, kbeg, kend, split)) return false;
  t.grp = __builtin_amdgcn_readfirstlane(grp);
  t.row0 = __builtin_amdgcn_readfirstlane(row0);
  t.rows = __builtin_amdgcn_readfirstlane(rows);
  t.n0 = __builtin_amdgcn_readfirstlane(n_tile) * XQ_BN;
  t.kbeg = __builtin_amdgcn_readfirstlane(kbeg);
  t.kend = __builtin_amdgcn_readfirstlane(kend);
  return true;
}

// Slabs of a tile in the persistent loop: at least two.
__device__ __forceinline__ int xq_wgrad_nk(const XQTileW& t) {
  return max(2, t.kend > t.kbeg ? (int)cdiv(t.kend - t.kbeg, XQ_BK) : 0);
}

// Loader of tile t whose slab 0 sits at ring index g0.
__device__ __forceinline__ void xq_wgrad_loader(const XGemm& g, const XQTileW& t, int g0, int wave, int lane,
                                                XQLoad& L) {
  L.kbeg = t.kbeg;
  L.kend = t.kend;
  L.nk = xq_wgrad_nk(t);
  L.g0 = g0;
  L.lds_off = wave * XQ_LD * 1024;
  L.krow0 = wave * 16;
  L.a = static_cast<const bf16_t*>(g.A) + (int64_t)t.grp * g.a_col;
  L.a_ld = g.lda;
  L.b0 = L.b1 = static_cast<const bf16_t*>(g.Bact) + (int64_t)t.grp * g.b_col;
  L.kseg = 0x7fffffff;
  L.b_ld = g.ldb;
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int kr = wave * 16 + (lane >> 5);
    const int c = (lane & 31) ^ (((kr + 2 * par) & 3) << 2);
    L.kma[par] = (uint32_t)((int64_t)kr * g.lda + min(t.row0 + 8 * c, g.M - 8));
    L.kmb[par] = (uint32_t)((int64_t)kr * g.ldb + min(t.n0 + 8 * c, g.N - 8));
  }
}

// Direct load i of A (KM) or B (activation KM rows) of ring slab kb for the
// persistent loop.  The row address is formed unconditionally (an opaque
// copy keeps the compiler from sinking it into a branch) and only the choice
// between it and the zero block depends on the row: a branch per load would
// cut the MFMA stream into blocks.
__device__ __forceinline__ void xqw_issue_a_one(const XQLoad& L, int ka, int lane, int i) {
  extern __shared__ __attribute__((aligned(16))) char xq_smem[];
  const uint32_t da = lds_addr(xq_smem) + L.lds_off + (ka & 1) * XQ_REG;
  const int k0 = L.kbeg + min(ka - L.g0, L.nk - 1) * XQ_BK;
  const int kr = k0 + L.krow0 + 2 * i + (lane >> 5);
  int64_t src = reinterpret_cast<int64_t>(L.a + (int64_t)k0 * L.a_ld +
                                          (L.kma[i & 1] + (uint32_t)(2 * i) * (uint32_t)L.a_ld));
  asm volatile("" : "+v"(src));
  dma16(reinterpret_cast<const void*>(kr < L.kend ? src : reinterpret_cast<int64_t>(g_xq_zero)), da + i * 1024);
}

__device__ __forceinline__ void xqw_issue_b_one(const XQLoad& L, int kb, int lane, int i) {
  extern __shared__ __attribute__((aligned(16))) char xq_smem[];
  const uint32_t db = lds_addr(xq_smem) + L.lds_off + XQ_BOFF + (kb % XQ_BSLOTS) * XQ_REG;
  const int k0 = L.kbeg + min(kb - L.g0, L.nk - 1) * XQ_BK;
  const int kr = k0 + L.krow0 + 2 * i + (lane >> 5);
  int64_t src = reinterpret_cast<int64_t>(L.b0 + (int64_t)k0 * L.b_ld +
                                          (L.kmb[i & 1] + (uint32_t)(2 * i) * (uint32_t)L.b_ld));
  asm volatile("" : "+v"(src));
  dma16(reinterpret_cast<const void*>(kr < L.kend ? src : reinterpret_cast<int64_t>(g_xq_zero)), db + i * 1024);
}

// MFMAs T0 .. T1-1 of one K step (t = j * 4 + ni); the NL direct loads
// LI0 .. LI0 + NL - 1 of A (LK 0) or B (LK 1) of ring slab kl spread evenly
// over them.  ZC: the step starts the accumulators (zero accumulator input).
template <int T0, int T1, int NL, int LK, int LI0, bool ZC>
__device__ __forceinline__ void xqw_mma(const bf16x8_t (&fa)[4], const bf16x8_t (&fb)[4], f32x16_t (&acc)[4][4],
                                        const XQLoad& L, int kl, int lane) {
  const f32x16_t zero = {};
#pragma unroll
  for (int t = T0; t < T1; ++t) {
    acc[t / 4][t % 4] =
        __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[t % 4], fa[t / 4], ZC ? zero : acc[t / 4][t % 4], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      if (T0 + i * (T1 - T0) / (NL > 0 ? NL : 1) == t) {
        __builtin_amdgcn_sched_barrier(0);
        if (LK == 0)
          xqw_issue_a_one(L, kl, lane, LI0 + i);
        else
          xqw_issue_b_one(L, kl, lane, LI0 + i);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
}

struct XQPipe4 {
  bf16x8_t fa[4][4];
  bf16x8_t fb[4][4];
};

// One slab of the persistent loop: xq_slab's schedule (fragment reads two K
// steps ahead, the barrier after step 1, B(kb + 2) during steps 0 and 1,
// A(kb + 2) during steps 2 and 3) with one register set per K step, so every
// slab starts with its steps 0 and 1 in sets 0 and 1.  FIRST: slab kb starts
// the tile.
template <bool FIRST>
__device__ __forceinline__ void xqw_slab(XQPipe4& P, const XQLoad& L, int kb, int wm, int wn, int lane,
                                         f32x16_t (&acc)[4][4]) {
  constexpr int NL = XQ_LD / 2;
  __builtin_amdgcn_sched_barrier(0);
  xq_read<XA_KMAJOR, 4>(kb, 2, wm, wn, lane, P.fa[2], P.fb[2]);
  __builtin_amdgcn_sched_barrier(0);
  xqw_mma<0, 16, NL, 1, 0, FIRST>(P.fa[0], P.fb[0], acc, L, kb + 2, lane);
  __builtin_amdgcn_sched_barrier(0);
  xq_read<XA_KMAJOR, 4>(kb, 3, wm, wn, lane, P.fa[3], P.fb[3]);
  __builtin_amdgcn_sched_barrier(0);
  xqw_mma<0, 16, NL, 1, NL, false>(P.fa[1], P.fb[1], acc, L, kb + 2, lane);
  __builtin_amdgcn_sched_barrier(0);
  // every read of slab kb has returned, and this wave's loads of slab kb + 1
  // (only the B(kb + 2) loads are younger; a tile's first slab has none left:
  // the wave waited for all its loads before the previous tile's stores, so
  // that this wait need not wait for those stores too)
  wait_lgkm0();
  if (!FIRST) wait_vm<XQ_LD>();
  xq_sync();
  xqw_mma<0, 4, 1, 0, 0, false>(P.fa[2], P.fb[2], acc, L, kb + 2, lane);
  __builtin_amdgcn_sched_barrier(0);
  xq_read<XA_KMAJOR, 4>(kb + 1, 0, wm, wn, lane, P.fa[0], P.fb[0]);
  __builtin_amdgcn_sched_barrier(0);
  xqw_mma<4, 16, NL - 1, 0, 1, false>(P.fa[2], P.fb[2], acc, L, kb + 2, lane);
  __builtin_amdgcn_sched_barrier(0);
  xq_read<XA_KMAJOR, 4>(kb + 1, 1, wm, wn, lane, P.fa[1], P.fb[1]);
  __builtin_amdgcn_sched_barrier(0);
  xqw_mma<0, 16, NL, 0, NL, false>(P.fa[3], P.fb[3], acc, L, kb + 2, lane);
}

// bf16 tile store of the persistent loop, wave by wave through the B slot of
// the tile's last slab (no load fills it before the next tile's first slab,
// and a wave's loads fill only its own 8 KB of a slot): each wave stages its
// 32 rows x 128 columns of accumulator row block j in its own 8 KB (8-byte
// unit u of row r at unit u ^ r), reads them back and stores 256-byte row
// pieces with global 16-byte stores (a flat store would also count against
// the LDS counter the slab loop waits on).  No barrier: the waves' epilogues
// are independent.
__device__ __forceinline__ void xq_wgrad_store_bf16(const XGemm& g, const XQTileW& t, char* slot, int wave, int wm,
                                                    int wn, int tid_, const f32x16_t (&acc)[4][4]) {
  // an opaque copy of the thread index keeps the address arithmetic below
  // here: hoisted out of the tile loop, its registers would be live through
  // every slab
  int tid = tid_;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  char* const reg = slot + wave * XQ_LD * 1024;
  const int64_t c0 = reinterpret_cast<int64_t>(g.Ctab0[t.grp]);
  // rows from msplit on go to Ctab1 from its row 0: its base shifted back by msplit rows
  const int64_t c1 = reinterpret_cast<int64_t>(g.Ctab1[t.grp]) - 2 * (int64_t)g.msplit * g.ldc;
  const int cc = lane & 15, n = t.n0 + wn * 128 + cc * 8;
  const bool col_ok = n < g.N;
  const int rw = lane & 31;
  wait_vm<0>();  // this wave's loads have landed before its first store
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int u = ni * 8 + q * 2 + (lane >> 5);
        u32x2_t w;
        w.x = pack_bf16x2(acc[j][ni][q * 4], acc[j][ni][q * 4 + 1]);
        w.y = pack_bf16x2(acc[j][ni][q * 4 + 2], acc[j][ni][q * 4 + 3]);
        *reinterpret_cast<u32x2_t*>(reg + rw * 256 + ((u ^ rw) << 3)) = w;
      }
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      const int rl = 4 * p + (lane >> 4);
      const int pu = (2 * cc) ^ rl;
      u32x4_t v = *reinterpret_cast<const u32x4_t*>(reg + rl * 256 + ((pu >> 1) << 4));
      if (rl & 1) v = u32x4_t{v.z, v.w, v.x, v.y};
      const int m = (2 * j + wm) * 32 + rl;
      const int r = t.row0 + m;
      const int64_t row = (r < g.msplit ? c0 : c1) + 2 * (int64_t)r * g.ldc;
      if (m < t.rows && col_ok) *reinterpret_cast<xq_gv4u*>(row + 2 * (int64_t)n) = v;
    }
  }
  wait_lgkm0();  // the reads are done before this wave's next loads into the slot
}

// fp32 tile store (fp32 master weights): straight from the accumulators, the
// 16 bytes of lanes l and l + 32 adjacent in a row.
__device__ __forceinline__ void xq_wgrad_store_f32(const XGemm& g, const XQTileW& t, int wm, int wn, int lane,
                                                   const f32x16_t (&acc)[4][4]) {
  const int64_t c0 = reinterpret_cast<int64_t>(g.Ctab0[t.grp]);
  const int64_t c1 = reinterpret_cast<int64_t>(g.Ctab1[t.grp]) - 4 * (int64_t)g.msplit * g.ldc;
  wait_vm<0>();  // this wave's loads have landed before its first store
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int m = (2 * j + wm) * 32 + (lane & 31);
    const int r = t.row0 + m;
    const int64_t row = (r < g.msplit ? c0 : c1) + 4 * (int64_t)r * g.ldc;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = t.n0 + wn * 128 + ni * 32 + q * 8 + (lane >> 5) * 4;
        if (m < t.rows && n < g.N)
          *reinterpret_cast<xq_gv4u*>(row + 4 * (int64_t)n) =
              u32x4_t{__float_as_uint(acc[j][ni][q * 4]), __float_as_uint(acc[j][ni][q * 4 + 1]),
                      __float_as_uint(acc[j][ni][q * 4 + 2]), __float_as_uint(acc[j][ni][q * 4 + 3])};
      }
  }
}

template <bool F32>
__global__ __launch_bounds__(256) void xgemm_wgrad_p_kernel(const XGemm g) {
  extern __shared__ __attribute__((aligned(16))) char xq_smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t G = gridDim.x;
  int64_t vb = blockIdx.x;
  XQTileW cur, nxt, nn;
  if (!xq_wgrad_tile(g, vb, cur)) return;
  bool more = xq_wgrad_tile(g, vb + G, nxt);
  // L loads the slabs two ahead of the MFMAs: the current tile's loader until
  // the loads cross into the next tile, then that tile's
  XQLoad L;
  xq_wgrad_loader(g, cur, 0, wave, lane, L);
  f32x16_t acc[4][4];  // started by each tile's first slab

  // first tile: A(0), B(0) and A(1), B(1) in flight together; both landed
  xq_issue_a<XA_KMAJOR, 0, XQ_LD>(L, 0, lane);
  xq_issue_b<XB_ACT_KMAJOR, 0, XQ_LD>(L, 0, lane);
  xq_issue_a<XA_KMAJOR, 0, XQ_LD>(L, 1, lane);
  xq_issue_b<XB_ACT_KMAJOR, 0, XQ_LD>(L, 1, lane);
  wait_vm<0>();  // slabs 0 and 1: the tile's first slab does not wait for loads
  xq_sync();
  XQPipe4 P;
  xq_read<XA_KMAJOR, 4>(0, 0, wm, wn, lane, P.fa[0], P.fb[0]);
  xq_read<XA_KMAJOR, 4>(0, 1, wm, wn, lane, P.fa[1], P.fb[1]);
  wait_lgkm0();
  int gs = 0;  // ring index of the current tile's first slab
  int kb = 0;
  for (;;) {
    const int nk = xq_wgrad_nk(cur);
    // before slab nk - 2 of the tile issues the loads of ring slab gs + nk,
    // L becomes the next tile's loader
    if (more && nk == 2) xq_wgrad_loader(g, nxt, gs + nk, wave, lane, L);
    xqw_slab<true>(P, L, kb, wm, wn, lane, acc);
    for (++kb; kb - gs < nk; ++kb) {
      if (more && kb - gs == nk - 2) xq_wgrad_loader(g, nxt, gs + nk, wave, lane, L);
      xqw_slab<false>(P, L, kb, wm, wn, lane, acc);
    }
    // the tile after next: its scalar loads run during the epilogue
    const bool more2 = more && xq_wgrad_tile(g, vb + 2 * G, nn);
    __builtin_amdgcn_sched_barrier(0);
    if (F32)
      xq_wgrad_store_f32(g, cur, wm, wn, lane, acc);
    else
      xq_wgrad_store_bf16(g, cur, xq_smem + XQ_BOFF + ((kb - 1) % XQ_BSLOTS) * XQ_REG, wave, wm, wn, tid, acc);
    __builtin_amdgcn_sched_barrier(0);
    if (!more) break;
    gs = kb;
    cur = nxt;
    nxt = nn;
    more = more2;
    vb += G;
    wait_lgkm0();  // no scalar load in flight at the loop head
  }
  __builtin_amdgcn_sched_barrier(0);
  wait_vm<0>();
}

// ---------------------------------------------------------------- host side
static bool xq_al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Shapes this kernel takes: identity KM rows (no K-side row map or scale),
// 16-byte aligned operands and strides, K slabs of 64 inside one weight
// segment, at most two weight segments, 32-bit operand offsets.
bool xgemm_q_ok(const XGemm& g, int epi) {
  const int64_t lim = int64_t(1) << 31;
  if (g.N % 8 || g.N < 8) return false;
  if (g.a_mode == XA_ROWS) {
    if (g.lda % 8 || !xq_al16(g.A) || g.K % XQ_BK) return false;
  } else {
    if (g.a_map || g.a_kscale || g.lda % 8 || g.a_col % 8 || g.M % 8 || g.M < 8 || !xq_al16(g.A)) return false;
    if ((int64_t)(XQ_BK + 1) * g.lda >= lim) return false;
  }
  if (g.b_mode == XB_W_NN) {
    if (g.a_mode != XA_ROWS || g.kseg % XQ_BK || g.ldb % 8 || g.nseg < 1 || g.nseg > 2) return false;
  } else if (g.b_mode == XB_ACT_KMAJOR) {
    if (g.a_mode != XA_KMAJOR || g.b_map || g.ldb % 8 || g.b_col % 8 || !xq_al16(g.Bact)) return false;
  } else {
    return false;
  }
  if ((int64_t)XQ_BK * g.ldb >= lim) return false;
  if (g.a_mode == XA_ROWS && g.sched_mode == XS_ROUTED && g.bm % XQ_BM) return false;
  if (g.a_mode == XA_ROWS) {
    const int64_t arows = g.sched_mode == XS_DENSE ? g.dense_rows : (int64_t)g.m_tiles_bound * g.bm;
    if (arows * g.lda >= lim && !g.a_map) return false;
  }
  if (epi == XE_WGRAD)
    return g.ldc % 8 == 0 && g.msplit % 4 == 0 && g.sched_mode == XS_WGRAD &&
           (g.ksplit <= 1 || (g.part && xq_al16(g.part)));
  if (epi == XE_SWIGLU_BWD)
    return g.ldc % 8 == 0 && g.c_group_col % 8 == 0 && xq_al16(g.C) && g.du_off % 8 == 0 && g.ld_gu % 8 == 0 &&
           g.gu_group_col % 8 == 0 && xq_al16(g.Gs) && xq_al16(g.Us);
  return g.ldc % 8 == 0 && g.c_group_col % 8 == 0 && xq_al16(g.C);
}

template <int EPI, int AMODE>
static int launch_xq_t(const XGemm& g, int64_t grid, hipStream_t st) {
  auto kern = xgemm_q_kernel<EPI, AMODE>;
  static const hipError_t attr =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)XQ_LDS);
  if (attr != hipSuccess) return fail(DSMOE_ERR_HIP, "xgemm_q: cannot raise LDS limit");
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), XQ_LDS, st, g);
  return check_launch("xgemm_q");
}

// Workgroups of the persistent weight-gradient loop: one per CU (the kernel
// takes a whole CU's LDS), rounded up to a multiple of 8.
static int64_t xq_persist_grid() {
  static std::atomic<int> ncu{0};
  int n = ncu.load(std::memory_order_relaxed);
  if (n == 0) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    ncu.store(n, std::memory_order_relaxed);
  }
  return 8 * cdiv(n, 8);
}

template <bool F32>
static int launch_xq_wgrad_p(const XGemm& g, int64_t grid, hipStream_t st) {
  auto kern = xgemm_wgrad_p_kernel<F32>;
  static const hipError_t attr =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)XQ_LDS);
  if (attr != hipSuccess) return fail(DSMOE_ERR_HIP, "xgemm_wgrad_p: cannot raise LDS limit");
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(256), XQ_LDS, st, g);
  return check_launch("xgemm_wgrad_p");
}

int launch_xgemm_q(const XGemm& g, int epi, hipStream_t st) {
  int64_t m_bound;
  if (g.sched_mode == XS_ROUTED)
    m_bound = (int64_t)g.m_tiles_bound * (g.bm / XQ_BM);
  else if (g.sched_mode == XS_DENSE)
    m_bound = cdiv(g.dense_rows, XQ_BM) * g.groups;
  else
    m_bound = cdiv(g.M, XQ_BM) * g.groups * std::max(g.ksplit, 1);
  const int64_t grid = 8 * cdiv(m_bound * cdiv(g.N, XQ_BN), 8);
  if (grid == 0) return DSMOE_OK;
  if (grid > 0x7fffffff) return fail(DSMOE_ERR_UNSUPPORTED, "xgemm_q: grid too large");
  if (epi == XE_SWIGLU_BWD) return launch_xq_t<XE_SWIGLU_BWD, XA_ROWS>(g, grid, st);
  if (epi == XE_STORE) return launch_xq_t<XE_STORE, XA_ROWS>(g, grid, st);
  if (g.ksplit <= 1) {
    const int64_t grid_p = std::min(grid, xq_persist_grid());
    return g.c_f32 ? launch_xq_wgrad_p<true>(g, grid_p, st) : launch_xq_wgrad_p<false>(g, grid_p, st);
  }
  const int rc = launch_xq_t<XE_WGRAD, XA_KMAJOR>(g, grid, st);
  if (rc || g.ksplit <= 1) return rc;
  return launch_wgrad_reduce(g, st);  // add the split-K partials in ascending part order
}

}  // namespace dsmoe
