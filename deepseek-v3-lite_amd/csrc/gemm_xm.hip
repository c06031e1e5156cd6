// Backward grouped GEMMs on gfx950 MFMA (bf16 in, fp32 accumulate).
//
// The backward of models/moe.py:127-131 (and of the operator in
// models/moe_triton.py:142-374) needs operands whose reduction index K is the
// ROW index of the stored matrix ("K-major"):
//   dh   = dY W2            B(n=i, k=d)  = W2[d][i]          (weights)
//   dx   = [dg|du][W1;W3]   B(n=d, k=i)  = W1[i][d] / W3[i][d]
//   dW13 = [dg|du]^T X      A(m=i, k=r)  = dgdu[r][i],  B(n=d, k=r) = X[tok(r)][d]
//   dW2  = (w dY)^T H       A(m=d, k=r)  = w_r dY[tok(r)][d], B(n=i, k=r) = H[r][i]
// v_mfma_f32_32x32x16_bf16 wants 8 consecutive K values per lane, so a
// K-major operand is transposed on its way into LDS: each thread loads a
// 4 (k) x 8 (columns) block as four 16-byte row pieces, transposes it in
// registers into eight 4-element column pieces and writes those as 8-byte
// LDS stores.  The LDS tile is then the same [row][64 k] layout as for a
// K-contiguous operand, and the MFMA inner loop is the forward kernel's.
//
// Block: 8 waves (4 x 2), 256 x 256 output tile, each wave 2 x 4 MFMA tiles
// of 32 x 32; K slabs of 64 are double-buffered through LDS (128 KiB), the
// next slab's global loads in flight during the current slab's MFMAs.
//
// LDS swizzle: chunk c of row r is stored at c ^ (((r >> 1) ^ ((r >> 2) & 4)) & 7).
// Fragment reads (16 consecutive rows per cycle at one chunk) see the 8
// distinct values of (r >> 1) & 7 XOR a constant: conflict-free.  The
// transposing writer stores rows 8j + i of four column chunks j at one k
// chunk; lanes of odd j write their rows in the order i ^ 1 so both row
// parities (both bank halves) are used, and the (r >> 4) term separates j = 0
// from j = 2: 32 lanes x 8 bytes land on 64 distinct banks.
//
// Determinism: one block owns each output tile and walks its K range in
// ascending order; no atomics, no split-K.
#include <algorithm>

#include "gemm_tile.h"
#include "mfma.h"

namespace dsmoe {

constexpr int XM_WM = 4, XM_WN = 2, XM_TM = 2, XM_TN = 4;
constexpr int XM_THREADS = 64 * XM_WM * XM_WN;  // 512
constexpr int XM_BM = XM_WM * XM_TM * 32;       // 256
constexpr int XM_BN = XM_WN * XM_TN * 32;       // 256
constexpr int XM_A_EL = XM_BM * MF_K;
constexpr int XM_B_EL = XM_BN * MF_K;
constexpr int XM_STAGE = XM_A_EL + XM_B_EL;
constexpr size_t XM_LDS_BYTES = 2ull * XM_STAGE * sizeof(bf16_t);  // 128 KiB of K slabs (then the staged tile)
constexpr size_t XM_LDS_ALLOC = XM_LDS_BYTES + 256 * sizeof(int64_t); // + the epilogue's output row pointers
static_assert(XM_BM == 256 && XM_BN == 256, "loader mappings assume 256 x 256 tiles and 512 threads");

__device__ __forceinline__ int xswz(int row, int chunk) {
  return row * MF_K + ((chunk ^ (((row >> 1) ^ ((row >> 2) & 4)) & 7)) << 3);
}

// Scales the 8 bf16 of v by s (fp32 product, rounded to nearest even once).
__device__ __forceinline__ u32x4_t scale8(u32x4_t v, float s) {
  u32x4_t o;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    const float lo = __uint_as_float(v[d] << 16) * s;
    const float hi = __uint_as_float(v[d] & 0xffff0000u) * s;
    o[d] = (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
  }
  return o;
}

// Transposes the 4 (k) x 8 (column) block v (row j = k offset j) and stores
// column i as 4 consecutive k at LDS row 8 * cc + i, k chunk q >> 1, half q & 1.
__device__ __forceinline__ void km_store(bf16_t* __restrict__ s, int cc, int odd, int q, const u32x4_t (&v)[4]) {
  u32x2_t o[8];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    o[2 * d].x = (v[0][d] & 0xffffu) | (v[1][d] << 16);
    o[2 * d].y = (v[2][d] & 0xffffu) | (v[3][d] << 16);
    o[2 * d + 1].x = (v[0][d] >> 16) | (v[1][d] & 0xffff0000u);
    o[2 * d + 1].y = (v[2][d] >> 16) | (v[3][d] & 0xffff0000u);
  }
  const int c = q >> 1, half = q & 1;
  const uint32_t msk = 0u - (uint32_t)odd;  // all ones for odd column chunks
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // odd lanes write column i ^ 1 at this step (a lane-dependent register
    // choice written as a bit blend, so no dynamic register indexing)
    u32x2_t val;
    val.x = (o[i].x & ~msk) | (o[i ^ 1].x & msk);
    val.y = (o[i].y & ~msk) | (o[i ^ 1].y & msk);
    *reinterpret_cast<u32x2_t*>(s + xswz(8 * cc + (i ^ odd), c) + 4 * half) = val;
  }
}

// K-major operand source for one tile: rows are k (optionally through a row
// map), 8-column chunks from `col` on.
struct KmSrc {
  const bf16_t* base;  // activations: matrix base (+ group column offset); weights: unused
  int64_t ld;
  const int32_t* map;
  const float* kscale;
};

template <int EPI, int AMODE, int BMODE>
__global__ __launch_bounds__(XM_THREADS) void xgemm_mfma_kernel(const XGemm g) {
  extern __shared__ __attribute__((aligned(16))) bf16_t smem_x[];
  int grp, row0, rows, n_tile, kbeg, kend, split;
  if (!xtile<XM_BM, XM_BN>(g, grp, row0, rows, n_tile, kbeg, kend, split)) return;
  const int n0 = n_tile * XM_BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / XM_WN, wn = wave % XM_WN;
  // K-contiguous loader: chunk lc of rows lr + 64 i
  const int lc = tid & 7, lr = tid >> 3;
  // K-major loader: column chunk cc (8 columns), k rows 4 q + j
  const int mc = lane & 3, q = lane >> 2;
  const int cc = wave * 4 + mc;
  const int odd = mc & 1;

  // ---- A operand set-up
  int64_t a_off[4];
  KmSrc as{};
  int a_col = 0;
  if (AMODE == XA_ROWS) {
    const bf16_t* A = static_cast<const bf16_t*>(g.A);
    (void)A;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = min(lr + i * 64, rows - 1);
      const int64_t arow = g.a_map ? (int64_t)g.a_map[row0 + r] : (int64_t)(row0 + r);
      a_off[i] = arow * g.lda + lc * 8;
    }
  } else {
    as.base = static_cast<const bf16_t*>(g.A) + (int64_t)grp * g.a_col;
    as.ld = g.lda;
    as.map = g.a_map;
    as.kscale = g.a_kscale;
    a_col = min(row0 + 8 * cc, g.M - 8);  // tile "rows" are the weight rows m
  }
  // ---- B operand set-up (always K-major)
  KmSrc bs{};
  const int b_col = min(n0 + 8 * cc, g.N - 8);
  const void* const* __restrict__ btab = nullptr;
  if (BMODE == XB_ACT_KMAJOR) {
    bs.base = static_cast<const bf16_t*>(g.Bact) + (int64_t)grp * g.b_col;
    bs.ld = g.ldb;
    bs.map = g.b_map;
  } else {
    btab = g.Btab + (int64_t)grp * g.nseg;
  }

  u32x4_t ra[4], rb[4];
  // Mapped K-major rows: the row indices (and scales) of a slab are fetched
  // one slab ahead of its data, so the data loads never wait for them.
  int32_t a_rows[4] = {0, 0, 0, 0}, b_rows[4] = {0, 0, 0, 0};
  float a_sc[4] = {1.0f, 1.0f, 1.0f, 1.0f};     // fetched for the next slab to load
  float a_sc_ld[4] = {1.0f, 1.0f, 1.0f, 1.0f};  // of the slab whose data is in flight
  auto fetch_rows = [&](int k0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int kk = min(k0 + 4 * q + j, kend - 1);
      if (AMODE == XA_KMAJOR) {
        a_rows[j] = as.map ? as.map[kk] : kk;
        if (as.kscale) a_sc[j] = as.kscale[kk];
      }
      if (BMODE == XB_ACT_KMAJOR) b_rows[j] = bs.map ? bs.map[kk] : kk;
    }
  };
  auto load_slab = [&](int k0) {
    // A
    if (AMODE == XA_ROWS) {
      const bf16_t* A = static_cast<const bf16_t*>(g.A);
#pragma unroll
      for (int i = 0; i < 4; ++i) ra[i] = ldg16(A + a_off[i] + k0);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        ra[j] = ldg16(as.base + (int64_t)a_rows[j] * as.ld + a_col);
        a_sc_ld[j] = a_sc[j];
      }
    }
    // B
    if (BMODE == XB_ACT_KMAJOR) {
#pragma unroll
      for (int j = 0; j < 4; ++j) rb[j] = ldg16(bs.base + (int64_t)b_rows[j] * bs.ld + b_col);
    } else {
      // weights: the 64-row slab lies inside one K segment (kseg % 64 == 0)
      const int seg = k0 / g.kseg;
      const bf16_t* W = static_cast<const bf16_t*>(btab[seg]);
      const int kin = k0 - seg * g.kseg + 4 * q;
#pragma unroll
      for (int j = 0; j < 4; ++j) rb[j] = ldg16(W + (int64_t)(kin + j) * g.ldb + b_col);
    }
  };
  // Rows past the K range read a clamped valid row; zero them (and apply the
  // per-row scale) once the data has arrived, right before the LDS store.
  auto fix_rows = [&](int k0) {
    if (AMODE == XA_KMAJOR) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (as.kscale) ra[j] = scale8(ra[j], a_sc_ld[j]);
        if (k0 + 4 * q + j >= kend) ra[j] = u32x4_t{0u, 0u, 0u, 0u};
      }
    }
    if (BMODE == XB_ACT_KMAJOR) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (k0 + 4 * q + j >= kend) rb[j] = u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  auto store_slab = [&](bf16_t* s) {
    if (AMODE == XA_ROWS) {
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4_t*>(s + xswz(lr + i * 64, lc)) = ra[i];
    } else {
      km_store(s, cc, odd, q, ra);
    }
    km_store(s + XM_A_EL, cc, odd, q, rb);
  };

  f32x16_t acc[XM_TM][XM_TN];
#pragma unroll
  for (int mi = 0; mi < XM_TM; ++mi)
#pragma unroll
    for (int ni = 0; ni < XM_TN; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.0f;

  const int nk = (kend > kbeg) ? (int)cdiv(kend - kbeg, MF_K) : 0;
  if (nk > 0) {
    fetch_rows(kbeg);
    load_slab(kbeg);
    if (nk > 1) fetch_rows(kbeg + MF_K);
    fix_rows(kbeg);
    store_slab(smem_x);
  }
  __syncthreads();
  for (int kb = 0; kb < nk; ++kb) {
    const int cur = kb & 1;
    const bool more = kb + 1 < nk;
    if (more) {
      load_slab(kbeg + (kb + 1) * MF_K);
      if (kb + 2 < nk) fetch_rows(kbeg + (kb + 2) * MF_K);
    }
    const bf16_t* sA = smem_x + cur * XM_STAGE;
    const bf16_t* sB = sA + XM_A_EL;
#pragma unroll
    for (int kk = 0; kk < MF_K / 16; ++kk) {
      const int c = kk * 2 + (lane >> 5);
      bf16x8_t af[XM_TM], bfr[XM_TN];
#pragma unroll
      for (int mi = 0; mi < XM_TM; ++mi)
        af[mi] = *reinterpret_cast<const bf16x8_t*>(sA + xswz((wm * XM_TM + mi) * 32 + (lane & 31), c));
#pragma unroll
      for (int ni = 0; ni < XM_TN; ++ni)
        bfr[ni] = *reinterpret_cast<const bf16x8_t*>(sB + xswz((wn * XM_TN + ni) * 32 + (lane & 31), c));
#pragma unroll
      for (int mi = 0; mi < XM_TM; ++mi)
#pragma unroll
        for (int ni = 0; ni < XM_TN; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[ni], af[mi], acc[mi][ni], 0, 0, 0);
    }
    if (more) {
      fix_rows(kbeg + (kb + 1) * MF_K);
      store_slab(smem_x + (cur ^ 1) * XM_STAGE);
    }
    __syncthreads();
  }

  // ---- epilogue.  Lane holds tile row m = (wm * 2 + mi) * 32 + (lane & 31)
  // and, per qq, columns n = (wn * 4 + ni) * 32 + 8 qq + 4 (lane >> 5) + {0..3}
  // (acc registers 4 qq ..).  Split-K partials, and fp32 weight gradients,
  // go straight out as fp32.
  if (EPI == XE_WGRAD && (g.ksplit > 1 || g.c_f32)) {
#pragma unroll
    for (int mi = 0; mi < XM_TM; ++mi) {
      const int m = (wm * XM_TM + mi) * 32 + (lane & 31);
      if (m >= rows) continue;
      const int r = row0 + m;
      float* prow = g.ksplit > 1
                        ? g.part + (((int64_t)split * g.groups + grp) * g.M + r) * g.N
                        : static_cast<float*>(r < g.msplit ? g.Ctab0[grp] : g.Ctab1[grp]) +
                              (int64_t)(r < g.msplit ? r : r - g.msplit) * g.ldc;
#pragma unroll
      for (int ni = 0; ni < XM_TN; ++ni)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int n = n0 + (wn * XM_TN + ni) * 32 + qq * 8 + (lane >> 5) * 4;
          if (n < g.N)
            *reinterpret_cast<float4*>(prow + n) = make_float4(acc[mi][ni][qq * 4], acc[mi][ni][qq * 4 + 1],
                                                               acc[mi][ni][qq * 4 + 2], acc[mi][ni][qq * 4 + 3]);
        }
    }
    return;
  }
  // Otherwise the tile goes through LDS and leaves as whole rows (direct
  // stores from the MFMA layout would split every cache line over several
  // store instructions).  Output row pointers are resolved once per row.
  char* sm = reinterpret_cast<char*>(smem_x);
  int64_t* rowp = reinterpret_cast<int64_t*>(sm + XM_LDS_BYTES);  // past the staged tile
  if (tid < 256) {
    const int r = row0 + min(tid, rows - 1);
    int64_t o;
    if (EPI == XE_WGRAD) {
      o = reinterpret_cast<int64_t>(static_cast<bf16_t*>(r < g.msplit ? g.Ctab0[grp] : g.Ctab1[grp]) +
                                    (int64_t)(r < g.msplit ? r : r - g.msplit) * g.ldc);
    } else {
      o = reinterpret_cast<int64_t>(static_cast<bf16_t*>(g.C) + (int64_t)grp * g.c_group_col +
                                    (g.c_map ? (int64_t)g.c_map[r] : (int64_t)r) * g.ldc);
    }
    rowp[tid] = o;
  }
  if (EPI != XE_SWIGLU_BWD) {
    // bf16 tile, 256 rows x 512 bytes; 8-byte unit u of row m at unit u ^ (m & 31)
#pragma unroll
    for (int mi = 0; mi < XM_TM; ++mi) {
      const int m = (wm * XM_TM + mi) * 32 + (lane & 31);
#pragma unroll
      for (int ni = 0; ni < XM_TN; ++ni)
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int u = ((wn * XM_TN + ni) * 32 + qq * 8 + (lane >> 5) * 4) >> 2;
          u32x2_t w;
          w.x = pack_bf16x2(acc[mi][ni][qq * 4], acc[mi][ni][qq * 4 + 1]);
          w.y = pack_bf16x2(acc[mi][ni][qq * 4 + 2], acc[mi][ni][qq * 4 + 3]);
          *reinterpret_cast<u32x2_t*>(sm + m * 512 + ((u ^ (m & 31)) << 3)) = w;
        }
    }
    __syncthreads();
    // 32 lanes per row, 16 bytes each; 16 rows per pass
    const int cc = tid & 31, n = n0 + cc * 8;
    for (int r = tid >> 5; r < rows; r += 16) {
      const int pu = (2 * cc) ^ (r & 31);
      u32x4_t v = *reinterpret_cast<const u32x4_t*>(sm + r * 512 + ((pu >> 1) << 4));
      if (r & 1) v = u32x4_t{v.z, v.w, v.x, v.y};
      if (n < g.N) *reinterpret_cast<u32x4_t*>(reinterpret_cast<bf16_t*>(rowp[r]) + n) = v;
    }
    return;
  }
  // SwiGLU backward: dh stays fp32 until dg and du are formed, so each column
  // half of the tile (128 columns, owned by the waves with wn == half) is
  // staged as fp32 in turn; 16-byte unit u (4 columns) of row m sits at unit
  // u ^ (m & 31).  The write-back reads g and u row pieces coalesced.
  const bf16_t* Gs = static_cast<const bf16_t*>(g.Gs);
  const bf16_t* Us = static_cast<const bf16_t*>(g.Us);
  for (int half = 0; half < 2; ++half) {
    if (half) __syncthreads();  // the first half's reads are done
    if (wn == half) {
#pragma unroll
      for (int mi = 0; mi < XM_TM; ++mi) {
        const int m = (wm * XM_TM + mi) * 32 + (lane & 31);
#pragma unroll
        for (int ni = 0; ni < XM_TN; ++ni)
#pragma unroll
          for (int qq = 0; qq < 4; ++qq) {
            const int u = (ni * 32 + qq * 8 + (lane >> 5) * 4) >> 2;
            *reinterpret_cast<float4*>(sm + m * 512 + ((u ^ (m & 31)) << 4)) =
                make_float4(acc[mi][ni][qq * 4], acc[mi][ni][qq * 4 + 1], acc[mi][ni][qq * 4 + 2],
                            acc[mi][ni][qq * 4 + 3]);
          }
      }
    }
    __syncthreads();
    const int cc = tid & 31, n = n0 + half * 128 + cc * 4;
    for (int r = tid >> 5; r < rows; r += 16) {
      const float4 dh4 = *reinterpret_cast<const float4*>(sm + r * 512 + ((cc ^ (r & 31)) << 4));
      if (n >= g.N) continue;
      const float rw = g.row_w ? g.row_w[row0 + r] : 1.0f;
      const int64_t ogu = (int64_t)(row0 + r) * g.ld_gu + (int64_t)grp * g.gu_group_col + n;
      const u32x2_t gp = *reinterpret_cast<const u32x2_t*>(Gs + ogu);
      const u32x2_t up = *reinterpret_cast<const u32x2_t*>(Us + ogu);
      const float dhv[4] = {dh4.x, dh4.y, dh4.z, dh4.w};
      float dg[4], du[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t gw = (e < 2) ? gp.x : gp.y, uw = (e < 2) ? up.x : up.y;
        const float gv = __uint_as_float((e & 1) ? (gw & 0xffff0000u) : (gw << 16));
        const float uv = __uint_as_float((e & 1) ? (uw & 0xffff0000u) : (uw << 16));
        const float dh = rw * dhv[e];
        const float sg = __builtin_amdgcn_rcpf(1.0f + __expf(-gv));  // 1 ulp; dg, du are rounded to bf16
        dg[e] = dh * uv * sg * (1.0f + gv * (1.0f - sg));
        du[e] = dh * gv * sg;
      }
      bf16_t* out = reinterpret_cast<bf16_t*>(rowp[r]);
      *reinterpret_cast<u32x2_t*>(out + n) = u32x2_t{pack_bf16x2(dg[0], dg[1]), pack_bf16x2(dg[2], dg[3])};
      *reinterpret_cast<u32x2_t*>(out + g.du_off + n) = u32x2_t{pack_bf16x2(du[0], du[1]), pack_bf16x2(du[2], du[3])};
    }
  }
}

// Adds the ksplit fp32 partials of a split-K weight gradient in ascending
// part order and writes the result, rounded to bf16 or (c_f32) as fp32 (4
// columns per thread).
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const XGemm g) {
  const int64_t q4 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_grp = (int64_t)g.M * (g.N / 4);
  if (q4 >= per_grp * g.groups) return;
  const int grp = (int)(q4 / per_grp);
  const int64_t rem = q4 - grp * per_grp;
  const int m = (int)(rem / (g.N / 4));
  const int n = (int)(rem - (int64_t)m * (g.N / 4)) * 4;
  const int64_t stride = (int64_t)g.groups * g.M * g.N;
  const float* p = g.part + ((int64_t)grp * g.M + m) * g.N + n;
  float4 s = *reinterpret_cast<const float4*>(p);
  for (int i = 1; i < g.ksplit; ++i) {
    const float4 v = *reinterpret_cast<const float4*>(p + i * stride);
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  const int64_t o = (int64_t)(m < g.msplit ? m : m - g.msplit) * g.ldc + n;
  if (g.c_f32) {
    *reinterpret_cast<float4*>(static_cast<float*>(m < g.msplit ? g.Ctab0[grp] : g.Ctab1[grp]) + o) = s;
    return;
  }
  bf16_t* out = static_cast<bf16_t*>(m < g.msplit ? g.Ctab0[grp] : g.Ctab1[grp]);
  const uint32_t p0 = (uint32_t)f2bf(s.x) | ((uint32_t)f2bf(s.y) << 16);
  const uint32_t p1 = (uint32_t)f2bf(s.z) | ((uint32_t)f2bf(s.w) << 16);
  *reinterpret_cast<u32x2_t*>(out + o) = u32x2_t{p0, p1};
}

// ---------------------------------------------------------------- host side
static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
static bool al8(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0; }

// Shapes and strides the MFMA kernel takes (pointer tables are checked by the
// caller, which holds the host copies).
bool xgemm_mfma_ok(const XGemm& g, int epi) {
  if (g.N % 8 != 0 || g.N < 8) return false;
  if (g.a_mode == XA_ROWS) {
    if (g.lda % 8 || !al16(g.A) || g.K % MF_K) return false;
  } else {
    if (g.lda % 8 || g.a_col % 8 || g.M % 8 || g.M < 8 || !al16(g.A)) return false;
  }
  if (g.b_mode == XB_W_NN) {
    if (g.kseg % MF_K || g.ldb % 8 || g.a_mode != XA_ROWS) return false;
  } else if (g.b_mode == XB_ACT_KMAJOR) {
    if (g.ldb % 8 || g.b_col % 8 || !al16(g.Bact) || g.a_mode != XA_KMAJOR) return false;
  } else {
    return false;
  }
  if (g.sched_mode == XS_ROUTED && g.bm % XM_BM) return false;
  // the staged epilogue writes 16-byte row pieces (XE_SWIGLU_BWD: 8-byte)
  if (epi == XE_WGRAD)
    return g.ldc % 8 == 0 && g.msplit % 4 == 0 && g.sched_mode == XS_WGRAD &&
           (g.ksplit <= 1 || (g.part && al16(g.part)));   // fp32 rows: ldc % 4 and 16-byte bases (caller)
  if (epi == XE_SWIGLU_BWD)
    return g.ldc % 4 == 0 && g.c_group_col % 4 == 0 && al8(g.C) && g.du_off % 4 == 0 && g.ld_gu % 4 == 0 &&
           g.gu_group_col % 4 == 0 && al8(g.Gs) && al8(g.Us);
  return g.ldc % 8 == 0 && g.c_group_col % 8 == 0 && al16(g.C);
}

template <int EPI, int AMODE, int BMODE>
static int launch_xm_t(const XGemm& g, int64_t grid, hipStream_t st) {
  auto kern = xgemm_mfma_kernel<EPI, AMODE, BMODE>;
  static const hipError_t attr =
      hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)XM_LDS_ALLOC);
  if (attr != hipSuccess) return fail(DSMOE_ERR_HIP, "xgemm: cannot raise LDS limit");
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(XM_THREADS), XM_LDS_ALLOC, st, g);
  return check_launch("xgemm_mfma");
}

int launch_xgemm_mfma(const XGemm& g, int epi, hipStream_t st) {
  int64_t m_bound;
  if (g.sched_mode == XS_ROUTED)
    m_bound = (int64_t)g.m_tiles_bound * (g.bm / XM_BM);
  else if (g.sched_mode == XS_DENSE)
    m_bound = cdiv(g.dense_rows, XM_BM) * g.groups;
  else
    m_bound = cdiv(g.M, XM_BM) * g.groups * std::max(g.ksplit, 1);
  const int64_t grid = 8 * cdiv(m_bound * cdiv(g.N, XM_BN), 8);
  if (grid == 0) return DSMOE_OK;
  if (grid > 0x7fffffff) return fail(DSMOE_ERR_UNSUPPORTED, "xgemm: grid too large");
  if (epi == XE_SWIGLU_BWD) return launch_xm_t<XE_SWIGLU_BWD, XA_ROWS, XB_W_NN>(g, grid, st);
  if (epi == XE_STORE) return launch_xm_t<XE_STORE, XA_ROWS, XB_W_NN>(g, grid, st);
  int rc = launch_xm_t<XE_WGRAD, XA_KMAJOR, XB_ACT_KMAJOR>(g, grid, st);
  if (rc || g.ksplit <= 1) return rc;
  return launch_wgrad_reduce(g, st);
}

int launch_wgrad_reduce(const XGemm& g, hipStream_t st) {
  const int64_t n4 = (int64_t)g.groups * g.M * (g.N / 4);
  if (n4 == 0) return DSMOE_OK;
  hipLaunchKernelGGL(wgrad_reduce_kernel, dim3((unsigned)cdiv(n4, 256)), dim3(256), 0, st, g);
  return check_launch("wgrad_reduce");
}

// Split count for a weight-gradient launch of `tiles` output tiles (K per
// tile = k_len rows): the smallest split, up to 8, that minimises rounds of
// 256 one-block-per-CU tiles per unit of work; 1 when the tiles already fill
// the GPU several times or K is short.
int xgemm_pick_ksplit(int64_t tiles, int64_t k_len) {
  if (tiles >= 1024 || k_len < 4 * 64) return 1;
  int best = 1;
  double best_cost = (double)cdiv(tiles, 256);
  for (int ks = 2; ks <= 8 && k_len / ks >= 128; ++ks) {
    const double cost = (double)cdiv(tiles * ks, 256) / ks + 0.02 * ks;  // small charge for partial traffic
    if (cost < best_cost - 1e-9) {
      best = ks;
      best_cost = cost;
    }
  }
  return best;
}

int64_t xgemm_tiles(int64_t M, int64_t N, int groups) { return cdiv(M, XM_BM) * cdiv(N, XM_BN) * groups; }

}  // namespace dsmoe
