// (f4) Multi-head latent attention forward on gfx950.  Restates the fused MLA
// attention of models/mla_triton.py:73-183 (_mla_flash_fwd_kernel, launched
// by triton_mla_attention, :303-329): per (batch, head)
//   K = [ctx_kv W_k^T | ctx_pe]   (S_kv x (D_nope + D_rope))
//   V =  ctx_kv W_v^T             (S_kv x D_v)
//   out = softmax(scale [q_nope | q_pe] K^T (+ causal mask)) V
// with the causal mask key <= query + q_start (no mask otherwise).
//
// Two launches:
//  * mla_kv_kernel materialises K and V once per (batch, head) in the
//    workspace: an MFMA GEMM of the latent rows with the head's W_k / W_v
//    rows (fp32 accumulation), V rounded to bf16, K_nope kept as an exact
//    pair of bf16 parts (hi = bf16(k), lo = bf16(k - hi)): a K row is
//    [k_hi | ctx_pe | k_lo] and the query side [q_nope | q_pe | q_nope], so
//    the scores carry K_nope to about 16 significant bits (the reference
//    keeps it in fp32 registers; bf16 alone moved peaked softmaxes by 1 %).
//    The split needs 2 D_nope + D_rope <= 256; wider heads use bf16 K_nope.
//    K is padded to DQKp columns (a multiple of 16, zeros) and V to DVp (a
//    multiple of 32), both to S_kvp rows (a multiple of 64, zero rows).  The reference kernel recomputes both
//    products for every 64-query block (at the 422m shape 70 % of its
//    flops); here they cost one pass over the latent cache.
//  * mla_fa_kernel: flash attention, one workgroup per 128 queries of a
//    (batch, head), four waves of 32 queries, 64-key blocks double-buffered
//    through LDS.  The score MFMA (v_mfma_f32_32x32x16_bf16) takes the K rows
//    as its first operand and the queries as its second, so a lane holds one
//    query and 16 keys per 32-key sub-tile: the online softmax is per lane
//    plus one permlane32 swap with the lane holding the query's other 16
//    keys, and the probabilities feed the PV MFMA straight from those
//    registers (its K order is the key order the score MFMA left in the
//    lane: keys {0-3, 8-11} in lanes 0-31 and {4-7, 12-15} in lanes 32-63 of
//    each 16-key step; the V operand is read in the same order with
//    transposing LDS reads).
#include <algorithm>
#include <climits>
#include <cstring>
#include <type_traits>

#include "common.h"
#include "mfma.h"

namespace dsmoe {

typedef short mla_v4s __attribute__((ext_vector_type(4)));
typedef float mla_f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned int mla_u32x4 __attribute__((ext_vector_type(4)));

constexpr int MLA_QB = 128;    // queries per workgroup (four waves of 32)
constexpr int MLA_KB = 64;     // keys per block
constexpr int MLA_RB = 64;     // latent rows per materialisation tile
constexpr float MLA_LOG2E = 1.4426950408889634f;

struct MlaArgs {
  const bf16_t* q_nope;   // (B, H, S_q, Dn)
  const bf16_t* q_pe;     // (B, H, S_q, Dr)
  const bf16_t* ctx_kv;   // (B, S_kv, R)
  const bf16_t* ctx_pe;   // (B, S_kv, Dr)
  const bf16_t* w_k;      // (H, Dn, R)
  const bf16_t* w_v;      // (H, Dv, R)
  bf16_t* out;            // (B, S_q, H, Dv)
  float* lse;             // (B, H, S_q): c m + log2(sum of p), the base-2 log-sum-exp of the scaled scores, or null
  // backward
  const bf16_t* dout;     // (B, S_q, H, Dv)
  bf16_t* qpk;            // (B, H, S_qp, DQKp) packed query rows as the score MFMA takes them (q_eff)
  bf16_t* dopk;           // (B, H, S_qp, DVp) packed dO rows (zeros past D_v and S_q)
  float* lsep;            // (B, H, S_qp) lse (+inf past S_q)
  float* deltap;          // (B, H, S_qp) D = rowsum(dO * O) (0 past S_q)
  int S_qp;               // S_q rounded up to a multiple of 64
  float* dq_nope;         // (B, H, S_q, Dn) fp32
  float* dq_pe;           // (B, H, S_q, Dr)
  bf16_t* dkv;            // (B, S_kv, H, Dn + Dv) bf16 rows [dk_nope | dv]: latent positions, heads side by side
  float* dk_pe;           // (B, S_kv, H, Dr)
  int kvec;               // 8-byte dkv stores (Dn, Dv % 4 == 0, dkv 8-byte aligned)
  int dovec;              // 16-byte dO row loads (Dv % 8 == 0, dout 16-byte aligned)
  int outvec;             // 16-byte O row loads in the backward (Dv % 8 == 0, out 16-byte aligned)
  int dqvec;              // 16-byte dq stores (Dn, Dr % 8 == 0, dq_nope / dq_pe 16-byte aligned)
  float scale;            // softmax_scale
  bf16_t* kbuf;           // (B, H, S_kvp, DQKp)
  bf16_t* vbuf;           // (B, H, S_kvp, DVp)
  int B, H, S_q, S_kv, R, Dn, Dr, Dv;
  int Rp, DQKp, DVp, S_kvp;
  int causal, q_start;
  int ksplit;             // K row = [k_hi | pe | k_lo] (else [k | pe])
  int negq;               // softmax_scale < 0: q is negated on load and c = |scale| log2(e)
  int qvec;               // 16-byte query loads (Dn, Dr % 8 == 0, q_nope / q_pe 16-byte aligned)
  int kvvec;              // 16-byte latent / weight row loads (R % 8 == 0, aligned)
  int pevec;              // 16-byte rope copies and K, V row pieces (Dn, Dr % 8 == 0, ctx_pe aligned)
  int ovec;               // 8-byte output stores (Dv % 4 == 0, out 8-byte aligned)
  float c;                // |softmax_scale| * log2(e) >= 0
};

// ---------------------------------------------------------------- K, V materialisation
// Grid (B * S_kvp / 64, H).  A workgroup computes 64 latent rows of one batch
// against one head's Dn + Dv weight rows, in column passes of up to 128.
// Wave (wr, wc) owns rows 32 wr.. and the pass's 32-column tiles wc, wc + 2;
// it loads its MFMA fragments straight from global memory (16 bytes per lane
// and K step, a row's 32 bytes per lane pair; every K step of the latent rows
// and then of one weight tile in flight at once), with the latent rows as the
// first operand, so a lane holds one output column and 16 rows.  The bf16
// results (and the k_lo parts) are staged in LDS and leave as 16-byte row
// pieces.  Rows past S_kv read as zeros, so their K and V rows come out
// zero; the rope and padding columns are copied directly.
// NKS = Rp / 16 K steps with 16-byte loads (R % 8 == 0, aligned rows): every
// fragment load of a batch is issued unconditionally from a valid address
// before any of them is used (a load under a branch, or one whose result is
// used at once, makes the compiler wait for it there).  Dead latent rows read
// row S_kv - 1 (finite values; their K and V rows then get probability 0 or
// are never read), dead weight rows read the last one (never stored), and
// with R % 16 == 8 the weight columns past R of the last K step are zeroed
// after the batch.  NKS = 0: element loads, any R.
constexpr int MLA_KVN = 128;   // output columns per pass
constexpr int MLA_KS = 16;     // K steps of 16 at most (R <= 256)

template <int NKS>
__global__ __launch_bounds__(256) void mla_kv_kernel(const MlaArgs a) {
  extern __shared__ __attribute__((aligned(16))) char mla_kv_smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int hi = lane >> 5, l32 = lane & 31;
  const int tiles_per_b = a.S_kvp / MLA_RB;
  const int b = blockIdx.x / tiles_per_b;
  const int s0 = (blockIdx.x - b * tiles_per_b) * MLA_RB;
  const int h = blockIdx.y;
  const int nks = a.Rp / 16;
  const int ncols = a.Dn + a.Dv;
  const int lo_end = a.ksplit ? 2 * a.Dn + a.Dr : a.Dn + a.Dr;
  const bool vout = a.pevec;   // 16-byte output pieces stay in one part
  const int64_t bh = (int64_t)b * a.H + h;
  bf16_t* krow0 = a.kbuf + (bh * a.S_kvp + s0) * a.DQKp;
  bf16_t* vrow0 = a.vbuf + (bh * a.S_kvp + s0) * a.DVp;
  constexpr int KS = NKS > 0 ? NKS : MLA_KS;
  // 8 bf16 of a row at column c (zeros past R or for a dead row); row is a
  // valid row address (clamped) on the vector path
  auto frag = [&](const bf16_t* row, bool ok, int c) -> bf16x8_t {
    mla_u32x4 v = {0u, 0u, 0u, 0u};
    if (NKS > 0) {
      v = *reinterpret_cast<const mla_u32x4*>(row + min(c, a.R - 8));
    } else if (ok) {
      bf16_t e8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) e8[e] = c + e < a.R ? row[c + e] : bf16_t(0);
      v = *reinterpret_cast<const mla_u32x4*>(e8);
    }
    return __builtin_bit_cast(bf16x8_t, v);
  };
  // latent fragments of this wave's rows, every K step
  const int srow = s0 + 32 * wr + l32;
  const bf16_t* xrow = a.ctx_kv + ((int64_t)b * a.S_kv + min(srow, a.S_kv - 1)) * a.R;
  bf16x8_t fx[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    if (NKS > 0 || ks < nks) fx[ks] = frag(xrow, srow < a.S_kv, 16 * ks + 8 * hi);
  // rope columns [Dn, Dn + Dr) and zero columns [lo_end, DQKp) of K, [Dv, DVp) of V
  {
    const int r = tid >> 2, q = tid & 3;    // four threads per row
    const int s = s0 + r;
    const bool live = s < a.S_kv;
    bf16_t* kr = krow0 + (int64_t)r * a.DQKp;
    const bf16_t* pe = a.ctx_pe + ((int64_t)b * a.S_kv + (live ? s : 0)) * a.Dr;
    if (vout) {
      for (int j = 8 * q; j < a.Dr; j += 32)
        *reinterpret_cast<mla_u32x4*>(kr + a.Dn + j) =
            live ? *reinterpret_cast<const mla_u32x4*>(pe + j) : mla_u32x4{0u, 0u, 0u, 0u};
    } else {
      for (int j = q; j < a.Dr; j += 4) kr[a.Dn + j] = live ? pe[j] : bf16_t(0);
    }
    for (int j = lo_end + q; j < a.DQKp; j += 4) kr[j] = bf16_t(0);
    for (int j = a.Dv + q; j < a.DVp; j += 4) vrow0[(int64_t)r * a.DVp + j] = bf16_t(0);
  }
  bf16_t* sho = reinterpret_cast<bf16_t*>(mla_kv_smem);   // staged outputs: hi [64][128], lo [64][128]
  char* sw = mla_kv_smem;                                    // (first) the pass's weight rows, LDS rows rs
  const int rs = a.Rp * 2 + 16;
  const int cpr = a.Rp / 8;
  for (int n0 = 0; n0 < ncols; n0 += MLA_KVN) {
    const int np = min(MLA_KVN, ncols - n0);
    if (n0 > 0) __syncthreads();              // the previous pass's staged outputs are stored
    if (NKS > 0) {
      // the pass's weight rows into LDS: one batch of loads per thread, all
      // issued before the stores (row and chunk indices clamped, so every
      // load reads valid memory; columns past R are zeroed afterwards)
      constexpr int PER = NKS > 0 ? (MLA_KVN * NKS * 2 + 255) / 256 : 1;
      const int tot = ((np + 31) / 32 * 32) * cpr;
      mla_u32x4 wv[PER];
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int i = min(tid + 256 * u, tot - 1);
        const int r = i / cpr, c = i - r * cpr;
        const int nc = min(n0 + r, ncols - 1);
        const bf16_t* wrow = nc < a.Dn ? a.w_k + ((int64_t)h * a.Dn + nc) * a.R
                                       : a.w_v + ((int64_t)h * a.Dv + (nc - a.Dn)) * a.R;
        wv[u] = *reinterpret_cast<const mla_u32x4*>(wrow + min(c * 8, a.R - 8));
      }
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int i = tid + 256 * u;
        if (i < tot) {
          const int r = i / cpr, c = i - r * cpr;
          *reinterpret_cast<mla_u32x4*>(sw + r * rs + c * 16) = c * 8 < a.R ? wv[u] : mla_u32x4{0u, 0u, 0u, 0u};
        }
      }
      __syncthreads();
    }
    mla_f32x16 accs[MLA_KVN / 64];
#pragma unroll
    for (int j = 0; j < MLA_KVN / 64; ++j) {
      const int t = wc + 2 * j;
      if (32 * t >= np) continue;
      const int n = n0 + 32 * t + l32;        // this lane's weight row (output column)
      bf16x8_t fw[KS];
      if (NKS > 0) {
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          fw[ks] = *reinterpret_cast<const bf16x8_t*>(sw + (32 * t + l32) * rs + (16 * ks + 8 * hi) * 2);
      } else {
        const int nc = min(n, ncols - 1);
        const bf16_t* wrow = nc < a.Dn ? a.w_k + ((int64_t)h * a.Dn + nc) * a.R
                                       : a.w_v + ((int64_t)h * a.Dv + (nc - a.Dn)) * a.R;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          if (ks < nks) fw[ks] = frag(wrow, n < ncols, 16 * ks + 8 * hi);
      }
      mla_f32x16& acc = accs[j];
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        if (NKS > 0 || ks < nks) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fx[ks], fw[ks], acc, 0, 0, 0);
    }
    if (NKS > 0) __syncthreads();             // every wave is done with the weight rows
#pragma unroll
    for (int j = 0; j < MLA_KVN / 64; ++j) {
      const int t = wc + 2 * j;
      if (32 * t >= np) continue;
      const mla_f32x16& acc = accs[j];
      const int col = 32 * t + l32;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        // hardware round-to-nearest-even conversions (v_cvt_pk_bf16_f32)
        const int r = 32 * wr + 8 * (i >> 2) + 4 * hi + (i & 3);
        const __bf16 v = (__bf16)acc[i];
        sho[r * MLA_KVN + col] = __builtin_bit_cast(bf16_t, v);
        sho[MLA_RB * MLA_KVN + r * MLA_KVN + col] = __builtin_bit_cast(bf16_t, (__bf16)(acc[i] - (float)v));
      }
    }
    __syncthreads();
    for (int i = tid; i < MLA_RB * (MLA_KVN / 8); i += 256) {
      const int r = i / (MLA_KVN / 8), c8 = (i - r * (MLA_KVN / 8)) * 8;
      if (c8 >= np) continue;
      const int n = n0 + c8;
      const bf16_t* hp = sho + r * MLA_KVN + c8;
      const bf16_t* lp = sho + MLA_RB * MLA_KVN + r * MLA_KVN + c8;
      if (vout && c8 + 8 <= np) {
        const mla_u32x4 vh = *reinterpret_cast<const mla_u32x4*>(hp);
        if (n < a.Dn) {
          *reinterpret_cast<mla_u32x4*>(krow0 + (int64_t)r * a.DQKp + n) = vh;
          if (a.ksplit)
            *reinterpret_cast<mla_u32x4*>(krow0 + (int64_t)r * a.DQKp + a.Dn + a.Dr + n) =
                *reinterpret_cast<const mla_u32x4*>(lp);
        } else {
          *reinterpret_cast<mla_u32x4*>(vrow0 + (int64_t)r * a.DVp + (n - a.Dn)) = vh;
        }
      } else {
        for (int e = 0; e < 8 && c8 + e < np; ++e) {
          const int ne = n + e;
          if (ne < a.Dn) {
            krow0[(int64_t)r * a.DQKp + ne] = hp[e];
            if (a.ksplit) krow0[(int64_t)r * a.DQKp + a.Dn + a.Dr + ne] = lp[e];
          } else {
            vrow0[(int64_t)r * a.DVp + (ne - a.Dn)] = hp[e];
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------- staged tiles
// Staged tiles are read both as MFMA fragments (ds_read_b128: eight columns
// of a row per lane) and transposed (ds_read_b64_tr_b16: four consecutive
// rows of a column per lane), so 16-byte chunk c of row r sits at
// c ^ mlb_g(r) inside each group of 16 chunks; sixteen consecutive rows at one
// chunk, and four consecutive rows (r = 0 mod 4) at four consecutive chunks
// (c = 0 mod 4), then fall on distinct banks.
// The backward kernels' tile loops come in a masked and an unmasked copy
// for the common widths; the widest take the masked one everywhere (two
// copies of their bodies exceed what the register allocator handles).
#define MLB_SPLIT_EDGE(NSTEP, NV) ((NSTEP) + 2 * (NV) <= 16)
constexpr int MLB_KW = 128;   // keys per workgroup of the dK, dV kernel
constexpr int MLB_QI = 64;    // queries per staged tile of the dK, dV kernel (two halves of 32)
constexpr int MLB_KT = 64;    // keys per staged tile of the dQ kernel

__device__ __forceinline__ int mlb_off(int r, int c, int rb) {
  const int g = ((r & 3) << 2) | ((r >> 2) & 3);
  return r * rb + (((c & ~15) | ((c & 15) ^ g)) << 4);
}

// Reads of a staged tile with row bytes RB, the lane-dependent part of their
// offsets computed once per kernel (the swizzle sees only a row's low four
// bits and a chunk's low four, so rows R + .. with R = 0 mod 16 and chunk
// group k add R RB + 256 k as immediates):
//  * frag(t, R, st): the MFMA fragment of row R + (l & 31), 16-byte chunk
//    2 st + hi (columns 16 st + 8 hi .. + 7);
//  * tfrag(t, r0, ct): columns 32 ct .. + 31 over rows r0 .. r0 + 15
//    (r0 = 0 mod 16) by two ds_read_b64_tr_b16, the rows in the order the
//    score MFMA leaves in a lane's registers (lanes 0-31: r0 + {0-3, 8-11},
//    lanes 32-63: r0 + {4-7, 12-15}); lane l gets column 32 ct + (l & 31).
//    In a 16-lane group lane s addresses row s >> 2, columns 4 (s & 3) ..
//    + 3 (8-byte unit u), and receives one column of the four rows.
template <int RB>
struct MlbLane {
  int f[8], t0[4], t1[4];
  __device__ __forceinline__ explicit MlbLane(int lane) {
    const int hi = lane >> 5, l32 = lane & 31;
#pragma unroll
    for (int st = 0; st < 8; ++st) f[st] = mlb_off(l32, 2 * st + hi, RB);
    const int gq = lane >> 4, sl = lane & 15;
    const int r = 4 * (gq >> 1) + (sl >> 2);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      const int u = 8 * ct + 4 * (gq & 1) + (sl & 3);
      t0[ct] = mlb_off(r, u >> 1, RB) + ((u & 1) << 3);
      t1[ct] = mlb_off(r + 8, u >> 1, RB) + ((u & 1) << 3);
    }
  }
  __device__ __forceinline__ bf16x8_t frag(const char* t, int R, int st) const {
    return *reinterpret_cast<const bf16x8_t*>(t + f[st & 7] + R * RB + 256 * (st >> 3));
  }
  __device__ __forceinline__ bf16x8_t tfrag(const char* t, int r0, int ct) const {
    const int k = r0 * RB + 256 * (ct >> 2);
    const mla_v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) mla_v4s*)(t + t0[ct & 3] + k));
    const mla_v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) mla_v4s*)(t + t1[ct & 3] + k));
    typedef short v8s __attribute__((ext_vector_type(8)));
    const v8s v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8_t, v);
  }
};

// ---------------------------------------------------------------- work items
// The attention kernels' work items are (batch-head pair hb, rank) with rank
// r the r-th longest of a pair's items under the causal mask (the forward
// and dQ kernels: query blocks from the last; the dK, dV kernel: key blocks
// from the first).  Block i runs on XCD i % 8 (local index j = i / 8).  With
// at least MLA_SPREAD pairs, XCD x owns the pairs x, x + 8, ... (their K, V
// or query-side rows share its L2) and walks them rank-major, so the
// dispatcher, which starts blocks in order as slots free up, runs every
// pair's longest item first and the short ones fill the tail.  Fewer pairs:
// the XCDs take contiguous eighths of the pair-major list (every XCD busy).
// Grid: 8 * ceil(BH / 8) * nrank blocks; false for a block past the items.
constexpr int MLA_SPREAD = 32;

__device__ __forceinline__ bool mla_item(int blk, int BH, int nrank, int& hb, int& rank) {
  const int x = blk & 7, j = blk >> 3;
  if (BH >= MLA_SPREAD) {
    const int nh = (BH - x + 7) >> 3;   // pairs on this XCD
    if (j >= nh * nrank) return false;
    rank = j / nh;
    hb = x + 8 * (j - rank * nh);
    return true;
  }
  const int total = BH * nrank, per = (total + 7) / 8;
  const int item = x * per + j;
  if (j >= per || item >= total) return false;
  hb = item / nrank;
  rank = item - hb * nrank;
  return true;
}

__host__ __device__ inline int64_t mla_grid(int BH, int nrank) { return 8 * (int64_t)((BH + 7) / 8) * nrank; }

// ---------------------------------------------------------------- attention
// LDS per buffer: K tile 64 x KRB bytes in the mlb_off layout, then V tile
// 64 x DVp * 2 bytes with 8-byte unit u of key row k stored at
// u ^ mla_vswz(k): the transposing reads of 32 lanes cover four consecutive
// key rows and eight units each, which this spreads over distinct banks.  The
// swizzle moves whole 16-byte chunks (it is a multiple of 8 units), so a tile
// arrives by direct 16-byte loads.
template <int NV>
__device__ __forceinline__ int mla_vswz(int k) {
  return NV == 1 ? 0 : NV == 2 ? 8 * ((k >> 1) & 1) : 8 * (k & 3);
}

template <int NSTEP, int NV>
struct MlaCfg {
  static constexpr int DQKp = NSTEP * 16;
  static constexpr int DVp = NV * 32;
  static constexpr int KRB = (DQKp + 127) / 128 * 256;   // K tile row bytes (mlb_off layout)
  static constexpr int KT = MLA_KB * KRB;              // K tile bytes
  static constexpr int VT = MLA_KB * DVp * 2;          // V tile bytes
  static constexpr int BUF = KT + VT;
  static constexpr int NLK = KT / 4096;                // 1 KB direct loads per wave and tile
  static constexpr int NLV = VT / 4096;
};

__device__ __forceinline__ float mla_pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}
__device__ __forceinline__ float mla_pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}

// Work items (batch, head, query block) as mla_item orders them, a pair's
// query blocks last-first (causal: the longest first).
template <int NSTEP, int NV>
__global__ __launch_bounds__(256) void mla_fa_kernel(const MlaArgs a) {
  using C = MlaCfg<NSTEP, NV>;
  extern __shared__ __attribute__((aligned(16))) char mla_smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hi = lane >> 5, ql = lane & 31;
  const int nq = (a.S_q + MLA_QB - 1) / MLA_QB;
  int hb, rank;
  if (!mla_item((int)blockIdx.x, a.B * a.H, nq, hb, rank)) return;
  const int h = hb % a.H, b = hb / a.H;
  const int q0 = (nq - 1 - rank) * MLA_QB;
  const int qi = q0 + 32 * wave + ql;          // this lane's query
  const int64_t bh = (int64_t)b * a.H + h;

  // query fragments: step st holds columns 16 st + 8 hi .. +7 of
  // [q_nope | q_pe | q_nope (split K) | 0]
  bf16x8_t qf[NSTEP];
  const bf16_t* qn = a.q_nope + (bh * a.S_q + qi) * a.Dn;
  const bf16_t* qp = a.q_pe + (bh * a.S_q + qi) * a.Dr;
  if (a.qvec) {
    // each 8-column group lies in one part: one 16-byte load, issued
    // unconditionally from a valid address (the row clamped to S_q - 1, a
    // padding group reads q_nope) and zeroed by a select
    const int qc = min(qi, a.S_q - 1);
    const bf16_t* qnc = a.q_nope + (bh * a.S_q + qc) * a.Dn;
    const bf16_t* qpc = a.q_pe + (bh * a.S_q + qc) * a.Dr;
    const int qend = a.ksplit ? 2 * a.Dn + a.Dr : a.Dn + a.Dr;
#pragma unroll
    for (int st = 0; st < NSTEP; ++st) {
      const int d = 16 * st + 8 * hi;
      // padding groups read real q values: K is zero there; a dead query's
      // row is finite and never stored
      const bf16_t* src = d < a.Dn ? qnc + d : d < a.Dn + a.Dr ? qpc + (d - a.Dn) : d < qend ? qnc + (d - a.Dn - a.Dr) : qnc;
      qf[st] = *reinterpret_cast<const bf16x8_t*>(src);
    }
    if (a.negq)
#pragma unroll
      for (int st = 0; st < NSTEP; ++st)
        qf[st] = __builtin_bit_cast(bf16x8_t, __builtin_bit_cast(mla_u32x4, qf[st]) ^
                                                   mla_u32x4{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u});
  } else {
#pragma unroll
    for (int st = 0; st < NSTEP; ++st) {
      bf16_t v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int d = 16 * st + 8 * hi + e;
        v[e] = bf16_t(0);
        if (qi < a.S_q) {
          if (d < a.Dn)
            v[e] = qn[d];
          else if (d < a.Dn + a.Dr)
            v[e] = qp[d - a.Dn];
          else if (a.ksplit && d < 2 * a.Dn + a.Dr)
            v[e] = qn[d - a.Dn - a.Dr];
          if (a.negq) v[e] ^= 0x8000;   // exact: the scores change sign, c stays >= 0
        }
      }
      qf[st] = *reinterpret_cast<const bf16x8_t*>(v);
    }
  }

  // keys this workgroup needs
  int kend = a.S_kv;
  if (a.causal) kend = min(kend, min(q0 + MLA_QB, a.S_q) - 1 + a.q_start + 1);
  const int nkb = (kend + MLA_KB - 1) / MLA_KB;
  const char* kg = reinterpret_cast<const char*>(a.kbuf + bh * a.S_kvp * C::DQKp);
  const char* vg = reinterpret_cast<const char*>(a.vbuf + bh * a.S_kvp * C::DVp);
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  // block j straight into LDS buffer j & 1: the wave's 1 KB pieces of the K
  // and V tiles (lane: 16 bytes at LDS offset 16 lane, which hold the chunk
  // the tile's swizzle puts there)
  auto issue = [&](int j) {
    const uint32_t lds0 = lds_addr(mla_smem + (j & 1) * C::BUF);
    const int64_t k0 = (int64_t)j * MLA_KB;
#pragma unroll
    for (int u = 0; u < C::NLK; ++u) {
      const int blk = wv * C::NLK + u;
      const int ofs = blk * 1024 + 16 * lane;
      const int row = ofs / C::KRB, pc = (ofs % C::KRB) >> 4;
      const int g = ((row & 3) << 2) | ((row >> 2) & 3);
      const int cl = (pc & ~15) | ((pc & 15) ^ g);
      if (cl < C::DQKp / 8)
        dma16s(kg + k0 * C::DQKp * 2, (uint32_t)(row * C::DQKp * 2 + 16 * cl), lds0 + blk * 1024);
    }
#pragma unroll
    for (int u = 0; u < C::NLV; ++u) {
      const int blk = wv * C::NLV + u;
      const int ofs = blk * 1024 + 16 * lane;
      const int row = ofs / (C::DVp * 2), pc = (ofs % (C::DVp * 2)) >> 4;
      const int cl = pc ^ (mla_vswz<NV>(row) >> 1);
      dma16s(vg + k0 * C::DVp * 2, (uint32_t)(row * C::DVp * 2 + 16 * cl), lds0 + C::KT + blk * 1024);
    }
  };
  const MlbLane<C::KRB> lk(lane);

  mla_f32x16 o[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[v][i] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  const int qpos = qi + a.q_start;

  if (nkb > 0) issue(0);
  for (int kb = 0; kb < nkb; ++kb) {
    // block kb has landed for every wave, and every wave is done with block kb - 1
    wait_vm<0>();
    wait_lgkm0();
    lds_barrier();
    if (kb + 1 < nkb) issue(kb + 1);
    const int k0 = kb * MLA_KB;
    const char* kt = mla_smem + (kb & 1) * C::BUF;
    const char* vt = kt + C::KT;
    // scores: sub-tile t, register i -> key k0 + 32 t + 8 (i / 4) + 4 hi + i % 4
    mla_f32x16 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[t][i] = 0.0f;
#pragma unroll
      for (int st = 0; st < NSTEP; ++st)
        s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lk.frag(kt, 32 * t, st), qf[st], s[t], 0, 0, 0);
    }
    // masks: keys past S_kv and, with the causal mask, keys past the query;
    // p = exp2(c s - c m) with c >= 0, so the running max of s is the max
    const bool edge = k0 + MLA_KB > a.S_kv || (a.causal && k0 + MLA_KB - 1 > q0 + a.q_start);
    if (edge) {
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int key = k0 + 32 * t + 8 * (i >> 2) + 4 * hi + (i & 3);
          if (key >= a.S_kv || (a.causal && key > qpos)) s[t][i] = -INFINITY;
        }
    }
    float mb = s[0][0];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i) mb = fmaxf(mb, s[t][i]);
    mb = mla_pair_max(mb);
    const float mn = fmaxf(m, mb);
    // a query whose keys so far are all masked keeps p = 0 (mn = -inf)
    const float mc = mn == -INFINITY ? 0.0f : mn * a.c;
    const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(m, a.c, -mc));
    const bool moved = m != mn;
    m = mn;
    float ls = 0.0f;
    bf16x8_t pf[4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          p[e] = __builtin_amdgcn_exp2f(fmaf(s[t][8 * half + e], a.c, -mc));
          ls += p[e];
        }
        bf16x2_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          w[e][0] = (__bf16)p[2 * e];
          w[e][1] = (__bf16)p[2 * e + 1];
        }
        pf[2 * t + half] = __builtin_bit_cast(bf16x8_t, w);
      }
    l = l * alpha + ls;
    // the accumulators are rescaled only when some lane's maximum moved
    if (__builtin_amdgcn_ballot_w64(moved)) {
#pragma unroll
      for (int v = 0; v < NV; ++v)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[v][i] *= alpha;
    }
    // PV: step ps covers keys k0 + 16 ps .. +15 in the order above; the V
    // operand of lane l is column 32 v + (l & 31) at the same keys
    {
      const int gq = lane >> 4, sl = lane & 15;
#pragma unroll
      for (int ps = 0; ps < 4; ++ps) {
        const int kr = 16 * ps + 4 * (gq >> 1) + (sl >> 2);
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          const int u = 8 * v + 4 * (gq & 1) + (sl & 3);
          const mla_v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) mla_v4s*)(vt + kr * (C::DVp * 2) + ((u ^ mla_vswz<NV>(kr)) << 3)));
          const mla_v4s hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) mla_v4s*)(vt + (kr + 8) * (C::DVp * 2) +
                                                           ((u ^ mla_vswz<NV>(kr + 8)) << 3)));
          typedef short v8s __attribute__((ext_vector_type(8)));
          const v8s vv = {lo[0], lo[1], lo[2], lo[3], hi4[0], hi4[1], hi4[2], hi4[3]};
          o[v] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vv), pf[ps], o[v], 0, 0, 0);
        }
      }
    }
  }

  // out[b, qi, h, dv]: lane holds dv = 32 v + 8 (i / 4) + 4 hi + i % 4
  const float lt = mla_pair_sum(l);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  if (qi >= a.S_q) return;
  // the backward's probabilities are exp2(c s - lse); a query without a
  // visible key gets +inf (probability 0)
  if (a.lse && hi == 0) a.lse[bh * a.S_q + qi] = lt > 0.0f ? m * a.c + log2f(lt) : INFINITY;
  bf16_t* orow = a.out + (((int64_t)b * a.S_q + qi) * a.H + h) * a.Dv;
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int dv = 32 * v + 8 * g + 4 * hi;
      if (a.ovec && dv + 3 < a.Dv) {
        bf16x2_t w0, w1;
        w0[0] = (__bf16)(o[v][4 * g] * inv);
        w0[1] = (__bf16)(o[v][4 * g + 1] * inv);
        w1[0] = (__bf16)(o[v][4 * g + 2] * inv);
        w1[1] = (__bf16)(o[v][4 * g + 3] * inv);
        u32x2_t w;
        w.x = __builtin_bit_cast(uint32_t, w0);
        w.y = __builtin_bit_cast(uint32_t, w1);
        *reinterpret_cast<u32x2_t*>(orow + dv) = w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (dv + e < a.Dv) orow[dv + e] = f2bf(o[v][4 * g + e] * inv);
      }
    }
}

// ---------------------------------------------------------------- backward
// The attention's backward in two deterministic kernels (no atomics), with
// P = exp2(c s - lse) (the forward's probabilities, rebuilt from its
// per-query base-2 log-sum-exp), D = rowsum(dO * O) and z = scale q.k:
//   dV = P^T dO,  dZ = P (dO V^T - D),  dK = scale dZ^T Q,  dQ = scale dZ K.
// mla_bwd_q_kernel runs first: it owns 128 queries, computes their D, walks
// their keys accumulating dQ, and leaves the query rows as the score MFMA
// takes them, the dO rows, lse and D packed in the workspace;
// mla_bwd_kv_kernel then owns 128 keys (four waves of 32) and walks the
// query tiles that see them, accumulating dV and dK in registers.
// Both rebuild s with the forward's operands (K rows [k_hi | pe | k_lo] from
// mla_kv_kernel, query rows [q_nope | q_pe | q_nope], q negated when the
// scale is negative), so dK comes out as |scale| dZ^T q_eff and dQ over the
// K columns, k_hi and k_lo parts added at the end.  The probabilities and dZ
// enter the MFMAs as bf16.
//
// 16 bf16 probabilities (or dZ values) of a lane's registers as the two
// 16-key (16-query) K-steps of the next MFMAs.
__device__ __forceinline__ void mlb_pack(const float (&p)[16], bf16x8_t (&f)[2]) {
#pragma unroll
  for (int ps = 0; ps < 2; ++ps) {
    bf16x2_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w[e][0] = (__bf16)p[8 * ps + 2 * e];
      w[e][1] = (__bf16)p[8 * ps + 2 * e + 1];
    }
    f[ps] = __builtin_bit_cast(bf16x8_t, w);
  }
}

// 8 columns d .. d + 7 of query row q (B H S_q layout) in the forward's
// query layout [q_nope | q_pe | q_nope (split K) | 0], negated for a negative
// scale; zeros past S_q.
__device__ __forceinline__ mla_u32x4 mlb_qchunk(const MlaArgs& a, int64_t bh, int q, int d) {
  mla_u32x4 v = {0u, 0u, 0u, 0u};
  if (q >= a.S_q) return v;
  const int qend = a.ksplit ? 2 * a.Dn + a.Dr : a.Dn + a.Dr;
  const bf16_t* qn = a.q_nope + (bh * a.S_q + q) * a.Dn;
  const bf16_t* qp = a.q_pe + (bh * a.S_q + q) * a.Dr;
  if (a.qvec) {
    // each 8-column group lies in one part (D_nope, D_rope multiples of 8)
    if (d < a.Dn) v = *reinterpret_cast<const mla_u32x4*>(qn + d);
    else if (d < a.Dn + a.Dr) v = *reinterpret_cast<const mla_u32x4*>(qp + (d - a.Dn));
    else if (d < qend) v = *reinterpret_cast<const mla_u32x4*>(qn + (d - a.Dn - a.Dr));
  } else {
    bf16_t e8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int c = d + e;
      e8[e] = c < a.Dn ? qn[c] : c < a.Dn + a.Dr ? qp[c - a.Dn] : c < qend ? qn[c - a.Dn - a.Dr] : bf16_t(0);
    }
    v = *reinterpret_cast<const mla_u32x4*>(e8);
  }
  if (a.negq) v ^= mla_u32x4{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
  return v;
}

// 8 values d .. d + 7 of query q of dO or O ((B, S_q, H, D_v) layout);
// zeros past S_q or D_v.
__device__ __forceinline__ mla_u32x4 mlb_dochunk(const MlaArgs& a, const bf16_t* t, int b, int h, int q, int d) {
  mla_u32x4 v = {0u, 0u, 0u, 0u};
  if (q >= a.S_q || d >= a.Dv) return v;
  const bf16_t* row = t + (((int64_t)b * a.S_q + q) * a.H + h) * a.Dv;
  if (a.dovec) return *reinterpret_cast<const mla_u32x4*>(row + d);
  bf16_t e8[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) e8[e] = d + e < a.Dv ? row[d + e] : bf16_t(0);
  return *reinterpret_cast<const mla_u32x4*>(e8);
}

template <int NSTEP, int NV>
struct MlbKvCfg {
  static constexpr int DQKp = NSTEP * 16;
  static constexpr int DVp = NV * 32;
  static constexpr int QRB = (DQKp + 127) / 128 * 256;   // Q tile row bytes
  static constexpr int ORB = (DVp + 127) / 128 * 256;    // dO tile row bytes
  static constexpr int QT = MLB_QI * QRB;
  static constexpr int OT = MLB_QI * ORB;
  static constexpr int BUF = QT + OT + 2 * MLB_QI * 4;   // Q, dO, lse, D
  static constexpr int NQI = QT / 4096;                  // 1 KB direct loads per wave and tile
  static constexpr int NOI = OT / 4096;
};

// Work items (batch, head, 128-key block) as mla_item orders them, a pair's
// key blocks first-first (causal: the longest first).  Wave w owns keys k0 + 32 w ..; a lane one key, with its
// K and V rows (the B operands of the score and dP MFMAs) in registers.  The
// query tiles (64 queries, two halves of 32) come from the packed rows
// mla_bwd_q_kernel leaves in the workspace (q_eff, dO, lse and D padded to
// S_qp rows), straight into LDS by direct loads (no staging registers), two
// buffers: tile i + 1 loads while tile i is used.
template <int NSTEP, int NV>
__global__ __launch_bounds__(256) void mla_bwd_kv_kernel(const MlaArgs a) {
  using C = MlbKvCfg<NSTEP, NV>;
  extern __shared__ __attribute__((aligned(16))) char mlb_smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hi = lane >> 5, l32 = lane & 31;
  const int nkb = (a.S_kv + MLB_KW - 1) / MLB_KW;
  int hb, rank;
  if (!mla_item((int)blockIdx.x, a.B * a.H, nkb, hb, rank)) return;
  const int h = hb % a.H, b = hb / a.H;
  const int k0 = rank * MLB_KW;
  const int kw0 = k0 + 32 * wave;
  const int key = kw0 + l32;
  const int64_t bh = (int64_t)b * a.H + h;
  const int nc = (a.Dn + a.Dr + 31) / 32;   // 32-column tiles of dK

  bf16x8_t kf[NSTEP], vf[2 * NV];
  {
    const int kr = min(key, a.S_kvp - 1);   // rows past S_kv are zero and masked below
    const bf16_t* krow = a.kbuf + (bh * a.S_kvp + kr) * C::DQKp;
    const bf16_t* vrow = a.vbuf + (bh * a.S_kvp + kr) * C::DVp;
#pragma unroll
    for (int st = 0; st < NSTEP; ++st) kf[st] = *reinterpret_cast<const bf16x8_t*>(krow + 16 * st + 8 * hi);
#pragma unroll
    for (int st = 0; st < 2 * NV; ++st) vf[st] = *reinterpret_cast<const bf16x8_t*>(vrow + 16 * st + 8 * hi);
  }
  mla_f32x16 dva[NV], dka[NSTEP / 2];
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int i = 0; i < 16; ++i) dva[v][i] = 0.0f;
#pragma unroll
  for (int t = 0; t < NSTEP / 2; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) dka[t][i] = 0.0f;

  // query tiles that see a key of this block: q >= k0 - q_start when causal
  const int qb = a.causal ? max(0, k0 - a.q_start) / MLB_QI * MLB_QI : 0;
  const int nqt = a.S_q > qb ? (a.S_q - qb + MLB_QI - 1) / MLB_QI : 0;
  const char* qsrc = reinterpret_cast<const char*>(a.qpk + (bh * a.S_qp + qb) * C::DQKp);
  const char* osrc = reinterpret_cast<const char*>(a.dopk + (bh * a.S_qp + qb) * C::DVp);
  const char* lsrc = reinterpret_cast<const char*>((wave == 0 ? a.lsep : a.deltap) + bh * a.S_qp + qb);
  // tile j into buffer j & 1: the wave's 1 KB blocks of the Q and dO tiles
  // (lane: 16 bytes at LDS offset 16 lane, physical chunk pc of its row,
  // which holds logical chunk pc ^ mlb_g(row)); chunks past the data width
  // are never read and not loaded.  Waves 0 and 1: the tile's 64 lse and D.
  auto issue = [&](int j) {
    const uint32_t lds0 = lds_addr(mlb_smem + (j & 1) * C::BUF);
    const int64_t q0 = (int64_t)j * MLB_QI;
#pragma unroll
    for (int u = 0; u < C::NQI; ++u) {
      const int blk = wave * C::NQI + u;
      const int ofs = blk * 1024 + 16 * lane;
      const int row = ofs / C::QRB, pc = (ofs % C::QRB) >> 4;
      const int g = ((row & 3) << 2) | ((row >> 2) & 3);
      const int cl = (pc & ~15) | ((pc & 15) ^ g);
      if (cl < C::DQKp / 8)
        dma16s(qsrc + q0 * C::DQKp * 2, (uint32_t)(row * C::DQKp * 2 + 16 * cl), lds0 + blk * 1024);
    }
#pragma unroll
    for (int u = 0; u < C::NOI; ++u) {
      const int blk = wave * C::NOI + u;
      const int ofs = blk * 1024 + 16 * lane;
      const int row = ofs / C::ORB, pc = (ofs % C::ORB) >> 4;
      const int g = ((row & 3) << 2) | ((row >> 2) & 3);
      const int cl = (pc & ~15) | ((pc & 15) ^ g);
      if (cl < C::DVp / 8)
        dma16s(osrc + q0 * C::DVp * 2, (uint32_t)(row * C::DVp * 2 + 16 * cl), lds0 + C::QT + blk * 1024);
    }
    if (wave < 2 && lane < MLB_QI / 4) dma16s(lsrc + q0 * 4, 16u * lane, lds0 + C::QT + C::OT + wave * MLB_QI * 4);
  };

  const MlbLane<C::QRB> lq(lane);
  const MlbLane<C::ORB> lo(lane);
  // tile i: EDGE = with the masks (q < S_q, key < S_kv, causal key <= q + q_start)
  auto tile = [&](int i, auto edge_c) {
    constexpr bool EDGE = decltype(edge_c)::value;
    // tile i has landed for every wave, and every wave is done with tile i - 1
    wait_vm<0>();
    wait_lgkm0();
    lds_barrier();
    if (i + 1 < nqt) issue(i + 1);
    const char* tq = mlb_smem + (i & 1) * C::BUF;
    const char* to = tq + C::QT;
    const float* tl = reinterpret_cast<const float*>(to + C::OT);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int qt = qb + i * MLB_QI + 32 * half;
      const int r0 = 32 * half;
      // a wave whose keys the half-tile cannot see skips it
      if (EDGE && (kw0 >= a.S_kv || qt >= a.S_q || (a.causal && qt + 31 + a.q_start < kw0))) continue;
      // s, dP: lane = key, register r = query qt + 8 (r / 4) + 4 hi + r % 4
      mla_f32x16 sc, dp;
#pragma unroll
      for (int i2 = 0; i2 < 16; ++i2) {
        sc[i2] = 0.0f;
        dp[i2] = 0.0f;
      }
#pragma unroll
      for (int st = 0; st < NSTEP; ++st)
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lq.frag(tq, r0, st), kf[st], sc, 0, 0, 0);
#pragma unroll
      for (int st = 0; st < 2 * NV; ++st)
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo.frag(to, r0, st), vf[st], dp, 0, 0, 0);
      // the pair is visible when q = qt + 4 hi + off(r) has qlo <= off(r) <= qhi
      const int qlo = (key < a.S_kv ? (a.causal ? key - a.q_start : INT_MIN / 2) : INT_MAX / 2) - qt - 4 * hi;
      const int qhi = a.S_q - 1 - qt - 4 * hi;
      float p[16], dz[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 l4 = *reinterpret_cast<const float4*>(tl + r0 + 8 * g + 4 * hi);
        const float4 d4 = *reinterpret_cast<const float4*>(tl + MLB_QI + r0 + 8 * g + 4 * hi);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
        const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          p[r] = __builtin_amdgcn_exp2f(fmaf(sc[r], a.c, -lv[e]));
          if (EDGE) p[r] = 8 * g + e >= qlo && 8 * g + e <= qhi ? p[r] : 0.0f;
          dz[r] = p[r] * (dp[r] - dv[e]);
        }
      }
      bf16x8_t pf[2], zf[2];
      mlb_pack(p, pf);
      mlb_pack(dz, zf);
#pragma unroll
      for (int ps = 0; ps < 2; ++ps) {
#pragma unroll
        for (int v = 0; v < NV; ++v)
          dva[v] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo.tfrag(to, r0 + 16 * ps, v), pf[ps], dva[v], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < NSTEP / 2; ++t)
          if (t < nc)
            dka[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lq.tfrag(tq, r0 + 16 * ps, t), zf[ps], dka[t], 0, 0, 0);
      }
    }
  };
  // tiles every pair of which is visible: queries qt .. qt + 63 < S_q, keys
  // k0 .. k0 + 127 < S_kv and (causal) k0 + 127 <= qt + q_start; the others,
  // the diagonal's before them and the S_q edge after, take the masks
  int i_lo = 0, i_hi = 0;   // 0 <= i_lo <= i_hi <= nqt
  if (k0 + MLB_KW <= a.S_kv) {
    i_lo = a.causal ? min(nqt, max(0, (k0 + MLB_KW - 1 - a.q_start - qb + MLB_QI - 1) / MLB_QI)) : 0;
    i_hi = max(i_lo, (a.S_q - qb) / MLB_QI);
  }
  if (nqt > 0) issue(0);
  int i = 0;
  for (; i < i_lo; ++i) tile(i, std::true_type{});
  for (; i < i_hi; ++i) tile(i, std::bool_constant<!MLB_SPLIT_EDGE(NSTEP, NV)>{});
  for (; i < nqt; ++i) tile(i, std::true_type{});

  // dK = |scale| dZ^T q_eff (lane = key, register r: column 32 t + 8 (r / 4)
  // + 4 hi + r % 4), dV = P^T dO (dv likewise): the bf16 row [dk_nope | dv]
  // of (batch, key, head), four consecutive columns per 8-byte store when
  // D_nope and D_v are multiples of 4; dk_pe in fp32
  if (key >= a.S_kv) return;
  const float sk = a.c * (1.0f / MLA_LOG2E);
  const int64_t kh = ((int64_t)b * a.S_kv + key) * a.H + h;
  bf16_t* dkv = a.dkv + kh * (a.Dn + a.Dv);
  float* dkp = a.dk_pe + kh * a.Dr;
  auto put4 = [&](int c, float v0, float v1, float v2, float v3) {   // columns c .. c + 3 of the row
    u32x2_t w;
    w.x = pack_bf16x2(v0, v1);
    w.y = pack_bf16x2(v2, v3);
    *reinterpret_cast<u32x2_t*>(dkv + c) = w;
  };
#pragma unroll
  for (int t = 0; t < NSTEP / 2; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = 32 * t + 8 * g + 4 * hi;
      if (t >= nc) continue;
      if (a.kvec && c + 3 < a.Dn) {
        put4(c, sk * dka[t][4 * g], sk * dka[t][4 * g + 1], sk * dka[t][4 * g + 2], sk * dka[t][4 * g + 3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (c + e < a.Dn)
            dkv[c + e] = f2bf(sk * dka[t][4 * g + e]);
          else if (c + e < a.Dn + a.Dr)
            dkp[c + e - a.Dn] = sk * dka[t][4 * g + e];
        }
      }
    }
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = 32 * v + 8 * g + 4 * hi;
      if (a.kvec && c + 3 < a.Dv) {
        put4(a.Dn + c, dva[v][4 * g], dva[v][4 * g + 1], dva[v][4 * g + 2], dva[v][4 * g + 3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (c + e < a.Dv) dkv[a.Dn + c + e] = f2bf(dva[v][4 * g + e]);
      }
    }
}

template <int NSTEP, int NV>
struct MlbQCfg {
  static constexpr int DQKp = NSTEP * 16;
  static constexpr int DVp = NV * 32;
  static constexpr int KRB = (DQKp + 127) / 128 * 256;
  static constexpr int VRB = (DVp + 127) / 128 * 256;
  static constexpr int KT = MLB_KT * KRB;
  static constexpr int BUF = KT + MLB_KT * VRB;
  static constexpr int NLK = KT / 4096;                    // 1 KB direct loads per wave and tile
  static constexpr int NLV = MLB_KT * VRB / 4096;
  static constexpr int SRS = DQKp + 4;                     // fp32 dQ staging row (floats)
  static constexpr int STG = 4 * 32 * SRS * 4;
  static constexpr int LDS = 2 * BUF > STG ? 2 * BUF : STG;
};

// Work items as the forward's: (batch, head, 128-query block), a pair's
// blocks longest first.  Lane: one query, its query fragments and dO row (the
// B operands of the score and dP MFMAs) in registers.  The 64-key K and V
// tiles go straight into LDS by direct loads, two buffers: tile i + 1 loads
// while tile i is used.
template <int NSTEP, int NV>
__global__ __launch_bounds__(256) void mla_bwd_q_kernel(const MlaArgs a) {
  using C = MlbQCfg<NSTEP, NV>;
  extern __shared__ __attribute__((aligned(16))) char mlb_smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hi = lane >> 5, l32 = lane & 31;
  const int nq = (a.S_q + MLA_QB - 1) / MLA_QB;
  int hb, rank;
  if (!mla_item((int)blockIdx.x, a.B * a.H, nq, hb, rank)) return;
  const int h = hb % a.H, b = hb / a.H;
  const int q0 = (nq - 1 - rank) * MLA_QB;
  const int qi = q0 + 32 * wave + l32;
  const int64_t bh = (int64_t)b * a.H + h;

  // the lane's query fragments, dO and O row pieces: with 16-byte rows every
  // load is issued unconditionally from a valid address (the row clamped to
  // S_q - 1, padding columns reading the row's start) and zeroed by a select
  // afterwards, so the batch stays in flight (a load under a runtime guard is
  // waited for at the guard's end)
  bf16x8_t qf[NSTEP], of[2 * NV], o8[2 * NV];
  const int qc = min(qi, a.S_q - 1);
  const bool qok = qi < a.S_q;
  if (a.qvec) {
    const int qend = a.ksplit ? 2 * a.Dn + a.Dr : a.Dn + a.Dr;
    const bf16_t* qn = a.q_nope + (bh * a.S_q + qc) * a.Dn;
    const bf16_t* qp = a.q_pe + (bh * a.S_q + qc) * a.Dr;
    mla_u32x4 v[NSTEP];
#pragma unroll
    for (int st = 0; st < NSTEP; ++st) {
      const int d = 16 * st + 8 * hi;
      const bf16_t* src = d < a.Dn ? qn + d : d < a.Dn + a.Dr ? qp + (d - a.Dn) : d < qend ? qn + (d - a.Dn - a.Dr) : qn;
      v[st] = *reinterpret_cast<const mla_u32x4*>(src);
    }
    const mla_u32x4 sgn = a.negq ? mla_u32x4{0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u}
                                 : mla_u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int st = 0; st < NSTEP; ++st) {
      const bool ok = qok && 16 * st + 8 * hi < qend;
      qf[st] = __builtin_bit_cast(bf16x8_t, ok ? v[st] ^ sgn : mla_u32x4{0u, 0u, 0u, 0u});
    }
  } else {
#pragma unroll
    for (int st = 0; st < NSTEP; ++st) qf[st] = __builtin_bit_cast(bf16x8_t, mlb_qchunk(a, bh, qi, 16 * st + 8 * hi));
  }
  {
    const int64_t orow = (((int64_t)b * a.S_q + qc) * a.H + h) * a.Dv;
    mla_u32x4 vd[2 * NV], vo[2 * NV];
#pragma unroll
    for (int st = 0; st < 2 * NV; ++st) {
      const int d = min(16 * st + 8 * hi, a.Dv - 8);
      if (a.dovec) vd[st] = *reinterpret_cast<const mla_u32x4*>(a.dout + orow + d);
      if (a.outvec) vo[st] = *reinterpret_cast<const mla_u32x4*>(a.out + orow + d);
    }
#pragma unroll
    for (int st = 0; st < 2 * NV; ++st) {
      const bool ok = qok && 16 * st + 8 * hi < a.Dv;
      of[st] = __builtin_bit_cast(bf16x8_t, a.dovec ? (ok ? vd[st] : mla_u32x4{0u, 0u, 0u, 0u})
                                                    : mlb_dochunk(a, a.dout, b, h, qi, 16 * st + 8 * hi));
      o8[st] = __builtin_bit_cast(bf16x8_t, a.outvec ? (ok ? vo[st] : mla_u32x4{0u, 0u, 0u, 0u})
                                                     : mlb_dochunk(a, a.out, b, h, qi, 16 * st + 8 * hi));
    }
  }
  const float lq = qok ? a.lse[bh * a.S_q + qc] : INFINITY;
  // D = rowsum(dO * O): this lane's columns 16 st + 8 hi .., then the other half of the row
  float dq = 0.0f;
#pragma unroll
  for (int st = 0; st < 2 * NV; ++st)
#pragma unroll
    for (int e = 0; e < 8; ++e) dq = fmaf((float)o8[st][e], (float)of[st][e], dq);
  dq += __shfl_xor(dq, 32);
  // the packed rows and padded lse, D the dK, dV kernel loads (rows up to S_qp)
  if (qi < a.S_qp) {
    bf16_t* qrow = a.qpk + (bh * a.S_qp + qi) * C::DQKp;
    bf16_t* orow = a.dopk + (bh * a.S_qp + qi) * C::DVp;
#pragma unroll
    for (int st = 0; st < NSTEP; ++st) *reinterpret_cast<bf16x8_t*>(qrow + 16 * st + 8 * hi) = qf[st];
#pragma unroll
    for (int st = 0; st < 2 * NV; ++st) *reinterpret_cast<bf16x8_t*>(orow + 16 * st + 8 * hi) = of[st];
    if (hi == 0) {
      a.lsep[bh * a.S_qp + qi] = lq;
      a.deltap[bh * a.S_qp + qi] = dq;
    }
  }
  const int qpos = qi + a.q_start;
  mla_f32x16 dqa[NSTEP / 2];
#pragma unroll
  for (int t = 0; t < NSTEP / 2; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) dqa[t][i] = 0.0f;

  int kend = a.S_kv;
  if (a.causal) kend = min(kend, min(q0 + MLA_QB, a.S_q) - 1 + a.q_start + 1);
  const int nkb = (kend + MLB_KT - 1) / MLB_KT;
  const char* kg = reinterpret_cast<const char*>(a.kbuf + bh * a.S_kvp * C::DQKp);
  const char* vg = reinterpret_cast<const char*>(a.vbuf + bh * a.S_kvp * C::DVp);
  // tile j into buffer j & 1 (the dK, dV kernel's scheme: lane 16 bytes at
  // LDS offset 16 lane, physical chunk pc holding logical chunk pc ^ mlb_g)
  auto issue = [&](int j) {
    const uint32_t lds0 = lds_addr(mlb_smem + (j & 1) * C::BUF);
    const int64_t k0 = (int64_t)j * MLB_KT;
#pragma unroll
    for (int u = 0; u < C::NLK; ++u) {
      const int blk = wave * C::NLK + u;
      const int ofs = blk * 1024 + 16 * lane;
      const int row = ofs / C::KRB, pc = (ofs % C::KRB) >> 4;
      const int g = ((row & 3) << 2) | ((row >> 2) & 3);
      const int cl = (pc & ~15) | ((pc & 15) ^ g);
      if (cl < C::DQKp / 8)
        dma16s(kg + k0 * C::DQKp * 2, (uint32_t)(row * C::DQKp * 2 + 16 * cl), lds0 + blk * 1024);
    }
#pragma unroll
    for (int u = 0; u < C::NLV; ++u) {
      const int blk = wave * C::NLV + u;
      const int ofs = blk * 1024 + 16 * lane;
      const int row = ofs / C::VRB, pc = (ofs % C::VRB) >> 4;
      const int g = ((row & 3) << 2) | ((row >> 2) & 3);
      const int cl = (pc & ~15) | ((pc & 15) ^ g);
      if (cl < C::DVp / 8)
        dma16s(vg + k0 * C::DVp * 2, (uint32_t)(row * C::DVp * 2 + 16 * cl), lds0 + C::KT + blk * 1024);
    }
  };

  const int qw = q0 + 32 * wave;   // this wave's first query
  const MlbLane<C::KRB> lk(lane);
  const MlbLane<C::VRB> lv(lane);
  // tile kb: EDGE = with the masks (q < S_q, key < S_kv, causal key <= q + q_start)
  auto tile = [&](int kb, auto edge_c) {
    constexpr bool EDGE = decltype(edge_c)::value;
    // tile kb has landed for every wave, and every wave is done with tile kb - 1
    wait_vm<0>();
    wait_lgkm0();
    lds_barrier();
    if (kb + 1 < nkb) issue(kb + 1);
    const int kk = kb * MLB_KT;
    const char* tk = mlb_smem + (kb & 1) * C::BUF;
    const char* tv = tk + C::KT;
#pragma unroll
    for (int t = 0; t < MLB_KT / 32; ++t) {
      const int ks = kk + 32 * t;
      // a wave whose queries see no key of the sub-tile skips it
      if (EDGE && (qw >= a.S_q || ks >= a.S_kv || (a.causal && ks > qw + 31 + a.q_start))) continue;
      // s, dP: lane = query, register r = key ks + 8 (r / 4) + 4 hi + r % 4
      mla_f32x16 sc, dp;
#pragma unroll
      for (int i2 = 0; i2 < 16; ++i2) {
        sc[i2] = 0.0f;
        dp[i2] = 0.0f;
      }
#pragma unroll
      for (int st = 0; st < NSTEP; ++st)
        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lk.frag(tk, 32 * t, st), qf[st], sc, 0, 0, 0);
#pragma unroll
      for (int st = 0; st < 2 * NV; ++st)
        dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lv.frag(tv, 32 * t, st), of[st], dp, 0, 0, 0);
      // keys past min(S_kv - 1, the query's position) and queries past S_q get p = 0
      const int klim = qi < a.S_q ? min(a.S_kv - 1, a.causal ? qpos : a.S_kv) - ks - 4 * hi : -1;
      float dz[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = __builtin_amdgcn_exp2f(fmaf(sc[r], a.c, -lq));
        if (EDGE) p = 8 * (r >> 2) + (r & 3) <= klim ? p : 0.0f;
        dz[r] = p * (dp[r] - dq);
      }
      bf16x8_t zf[2];
      mlb_pack(dz, zf);
#pragma unroll
      for (int ps = 0; ps < 2; ++ps)
#pragma unroll
        for (int ct = 0; ct < NSTEP / 2; ++ct)
          dqa[ct] =
              __builtin_amdgcn_mfma_f32_32x32x16_bf16(lk.tfrag(tk, 32 * t + 16 * ps, ct), zf[ps], dqa[ct], 0, 0, 0);
    }
  };
  // leading tiles every pair of which is visible: queries q0 .. q0 + 127 <
  // S_q and keys kk .. kk + 63 below min(S_kv, q0 + q_start + 1 when causal)
  int kfull = 0;
  if (q0 + MLA_QB <= a.S_q) kfull = min(nkb, (a.causal ? min(a.S_kv, q0 + a.q_start + 1) : a.S_kv) / MLB_KT);
  if (nkb > 0) issue(0);
  int kb = 0;
  for (; kb < kfull; ++kb) tile(kb, std::bool_constant<!MLB_SPLIT_EDGE(NSTEP, NV)>{});
  for (; kb < nkb; ++kb) tile(kb, std::true_type{});

  // every wave is done with the last tile before its buffer is reused
  wait_lgkm0();
  lds_barrier();
  // dQ over the K columns (lane = query, register r: column 32 ct + 8 (r / 4)
  // + 4 hi + r % 4), staged per wave as fp32 rows, then dq_nope = scale
  // (k_hi part + k_lo part), dq_pe = scale pe part, written row by row
  float* stg = reinterpret_cast<float*>(mlb_smem) + wave * 32 * C::SRS;
#pragma unroll
  for (int ct = 0; ct < NSTEP / 2; ++ct)
#pragma unroll
    for (int g = 0; g < 4; ++g)
      *reinterpret_cast<float4*>(stg + l32 * C::SRS + 32 * ct + 8 * g + 4 * hi) =
          make_float4(dqa[ct][4 * g], dqa[ct][4 * g + 1], dqa[ct][4 * g + 2], dqa[ct][4 * g + 3]);
  __syncthreads();
  const float sq = a.scale;
  const int nr = min(32, a.S_q - qw);
  if (a.dqvec) {
    // a lane pair per row, each lane every other 4-column group: 16-byte LDS
    // reads and global stores, all of a lane's independent
    const int r = lane >> 1, c0 = 4 * (lane & 1);
    if (r < nr) {
      const float* srow = stg + r * C::SRS;
      float* dn = a.dq_nope + (bh * a.S_q + qw + r) * a.Dn;
      float* dp = a.dq_pe + (bh * a.S_q + qw + r) * a.Dr;
      const int lo = a.ksplit ? a.Dn + a.Dr : 0;
      for (int d = c0; d < a.Dn; d += 8) {
        float4 v = *reinterpret_cast<const float4*>(srow + d);
        if (a.ksplit) {
          const float4 w = *reinterpret_cast<const float4*>(srow + lo + d);
          v.x += w.x; v.y += w.y; v.z += w.z; v.w += w.w;
        }
        *reinterpret_cast<float4*>(dn + d) = make_float4(sq * v.x, sq * v.y, sq * v.z, sq * v.w);
      }
      for (int d = c0; d < a.Dr; d += 8) {
        const float4 v = *reinterpret_cast<const float4*>(srow + a.Dn + d);
        *reinterpret_cast<float4*>(dp + d) = make_float4(sq * v.x, sq * v.y, sq * v.z, sq * v.w);
      }
    }
  } else {
    for (int r = 0; r < nr; ++r) {
      const float* srow = stg + r * C::SRS;
      float* dn = a.dq_nope + (bh * a.S_q + qw + r) * a.Dn;
      float* dp = a.dq_pe + (bh * a.S_q + qw + r) * a.Dr;
      for (int d = lane; d < a.Dn; d += 64) dn[d] = sq * (srow[d] + (a.ksplit ? srow[a.Dn + a.Dr + d] : 0.0f));
      for (int d = lane; d < a.Dr; d += 64) dp[d] = sq * srow[a.Dn + d];
    }
  }
}

// ---------------------------------------------------------------- host side
static int mla_pad(int v, int m) { return (v + m - 1) / m * m; }
// Supported K / V column buckets (16-column MFMA steps, 32-column V tiles).
static int mla_nstep(int dqk) {
  const int n = (dqk + 15) / 16;
  for (int s : {2, 4, 6, 8, 12, 16})
    if (n <= s) return s;
  return 0;
}
static int mla_nv(int dv) {
  const int n = (dv + 31) / 32;
  for (int s : {1, 2, 4, 8})
    if (n <= s) return s;
  return 0;
}

static int mla_validate(const dsmoe_mla_dims* d) {
  DSMOE_REQUIRE(d, DSMOE_ERR_INVALID, "mla: NULL dims");
  DSMOE_REQUIRE(d->B > 0 && d->H > 0 && d->S_q > 0 && d->S_kv > 0, DSMOE_ERR_INVALID,
                "mla: B, H, S_q and S_kv must be positive");
  DSMOE_REQUIRE(d->R > 0 && d->D_nope > 0 && d->D_rope > 0 && d->D_v > 0, DSMOE_ERR_INVALID,
                "mla: R, D_nope, D_rope and D_v must be positive");
  DSMOE_REQUIRE(d->R <= 256 && d->D_nope <= 256 && d->D_rope <= 256 && d->D_v <= 256, DSMOE_ERR_INVALID,
                "mla: R, D_nope, D_rope and D_v must not exceed 256");
  DSMOE_REQUIRE(d->D_nope + d->D_rope <= 256, DSMOE_ERR_UNSUPPORTED, "mla: D_nope + D_rope > 256 is not supported");
  DSMOE_REQUIRE(d->dtype == DSMOE_BF16, DSMOE_ERR_UNSUPPORTED, "mla: bf16 tensors only");
  DSMOE_REQUIRE(d->q_start >= 0, DSMOE_ERR_INVALID, "mla: q_start must be >= 0");
  DSMOE_REQUIRE((int64_t)d->B * d->H * mla_pad(d->S_kv, MLA_KB) * 512 < (int64_t(1) << 31) &&
                    (int64_t)d->B * d->H * d->S_q * 512 < (int64_t(1) << 31) &&
                    (int64_t)d->B * d->H * cdiv(d->S_q, MLA_QB) < (int64_t(1) << 30),
                DSMOE_ERR_UNSUPPORTED, "mla: tensors too large for 32-bit row indices");
  return DSMOE_OK;
}

static MlaArgs mla_args(const dsmoe_mla_dims* d) {
  MlaArgs a;
  std::memset(static_cast<void*>(&a), 0, sizeof(a));
  a.B = d->B; a.H = d->H; a.S_q = d->S_q; a.S_kv = d->S_kv;
  a.R = d->R; a.Dn = d->D_nope; a.Dr = d->D_rope; a.Dv = d->D_v;
  a.Rp = mla_pad(d->R, 16);
  a.ksplit = 2 * d->D_nope + d->D_rope <= 256 ? 1 : 0;
  a.DQKp = 16 * mla_nstep(a.ksplit ? 2 * d->D_nope + d->D_rope : d->D_nope + d->D_rope);
  a.DVp = 32 * mla_nv(d->D_v);
  a.S_kvp = mla_pad(d->S_kv, MLA_KB);
  a.S_qp = mla_pad(d->S_q, MLB_QI);
  a.causal = d->is_causal ? 1 : 0;
  a.q_start = d->q_start;
  a.negq = d->softmax_scale < 0.0f ? 1 : 0;
  a.c = (d->softmax_scale < 0.0f ? -d->softmax_scale : d->softmax_scale) * MLA_LOG2E;
  a.scale = d->softmax_scale;
  return a;
}

template <int NSTEP, int NV>
static int mla_launch_fa(const MlaArgs& a, hipStream_t st) {
  using C = MlaCfg<NSTEP, NV>;
  constexpr size_t lds = 2 * (size_t)C::BUF;
  auto kern = mla_fa_kernel<NSTEP, NV>;
  if (lds > 64 * 1024) {
    static const hipError_t attr =
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return fail(DSMOE_ERR_HIP, "mla: cannot raise LDS limit");
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)mla_grid(a.B * a.H, (int)cdiv(a.S_q, MLA_QB))), dim3(256), lds, st, a);
  return check_launch("mla_fa");
}

template <int NSTEP>
static int mla_launch_fa_nv(const MlaArgs& a, hipStream_t st) {
  switch (a.DVp / 32) {
    case 1: return mla_launch_fa<NSTEP, 1>(a, st);
    case 2: return mla_launch_fa<NSTEP, 2>(a, st);
    case 4: return mla_launch_fa<NSTEP, 4>(a, st);
    default: return mla_launch_fa<NSTEP, 8>(a, st);
  }
}

// mla_bwd_q_kernel (dQ; D and the packed rows), then mla_bwd_kv_kernel (dK, dV).
template <int NSTEP, int NV>
static int mla_launch_bwd(const MlaArgs& a, hipStream_t st) {
  {
    using C = MlbQCfg<NSTEP, NV>;
    constexpr size_t lds = (size_t)C::LDS;
    auto kern = mla_bwd_q_kernel<NSTEP, NV>;
    if (lds > 64 * 1024) {
      static const hipError_t attr =
          hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (attr != hipSuccess) return fail(DSMOE_ERR_HIP, "mla: cannot raise LDS limit");
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)mla_grid(a.B * a.H, (int)cdiv(a.S_q, MLA_QB))), dim3(256), lds, st, a);
    const int rc = check_launch("mla_bwd_q");
    if (rc) return rc;
  }
  using C = MlbKvCfg<NSTEP, NV>;
  constexpr size_t lds = 2 * (size_t)C::BUF;
  auto kern = mla_bwd_kv_kernel<NSTEP, NV>;
  if (lds > 64 * 1024) {
    static const hipError_t attr =
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (attr != hipSuccess) return fail(DSMOE_ERR_HIP, "mla: cannot raise LDS limit");
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)mla_grid(a.B * a.H, (int)cdiv(a.S_kv, MLB_KW))), dim3(256), lds, st, a);
  return check_launch("mla_bwd_kv");
}

template <int NSTEP>
static int mla_launch_bwd_nv(const MlaArgs& a, hipStream_t st) {
  switch (a.DVp / 32) {
    case 1: return mla_launch_bwd<NSTEP, 1>(a, st);
    case 2: return mla_launch_bwd<NSTEP, 2>(a, st);
    case 4: return mla_launch_bwd<NSTEP, 4>(a, st);
    default: return mla_launch_bwd<NSTEP, 8>(a, st);
  }
}

// K and V rows of every (batch, head) into the workspace (mla_kv_kernel).
static int mla_launch_kv(const MlaArgs& a, hipStream_t st) {
  // the pass's weight rows, then the staged outputs (hi and lo [64][128] bf16)
  const size_t kv_lds = std::max((size_t)MLA_KVN * (a.Rp * 2 + 16), (size_t)2 * MLA_RB * MLA_KVN * sizeof(bf16_t));
  const dim3 kv_grid((unsigned)(a.B * (a.S_kvp / MLA_RB)), (unsigned)a.H);
  switch (a.kvvec ? a.Rp / 16 : 0) {
#define MLA_KV_CASE(n) \
  case n: hipLaunchKernelGGL(mla_kv_kernel<n>, kv_grid, dim3(256), kv_lds, st, a); break;
    MLA_KV_CASE(1) MLA_KV_CASE(2) MLA_KV_CASE(3) MLA_KV_CASE(4) MLA_KV_CASE(5) MLA_KV_CASE(6) MLA_KV_CASE(7)
    MLA_KV_CASE(8) MLA_KV_CASE(9) MLA_KV_CASE(10) MLA_KV_CASE(11) MLA_KV_CASE(12) MLA_KV_CASE(13) MLA_KV_CASE(14)
    MLA_KV_CASE(15) MLA_KV_CASE(16)
#undef MLA_KV_CASE
    default: hipLaunchKernelGGL(mla_kv_kernel<0>, kv_grid, dim3(256), kv_lds, st, a); break;
  }
  return check_launch("mla_kv");
}

// The forward's operands, vector-load flags and K, V buffers of a call.
static MlaArgs mla_bind(const void* q_nope, const void* q_pe, const void* ctx_kv, const void* ctx_pe,
                        const void* wkv_b_k, const void* wkv_b_v, const dsmoe_mla_dims* dims, void* workspace) {
  MlaArgs a = mla_args(dims);
  a.q_nope = static_cast<const bf16_t*>(q_nope);
  a.q_pe = static_cast<const bf16_t*>(q_pe);
  a.ctx_kv = static_cast<const bf16_t*>(ctx_kv);
  a.ctx_pe = static_cast<const bf16_t*>(ctx_pe);
  a.w_k = static_cast<const bf16_t*>(wkv_b_k);
  a.w_v = static_cast<const bf16_t*>(wkv_b_v);
  auto al = [](const void* p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; };
  a.qvec = (a.Dn % 8 == 0 && a.Dr % 8 == 0 && al(q_nope, 16) && al(q_pe, 16)) ? 1 : 0;
  a.kvvec = (a.R % 8 == 0 && al(ctx_kv, 16) && al(wkv_b_k, 16) && al(wkv_b_v, 16)) ? 1 : 0;
  a.pevec = (a.Dn % 8 == 0 && a.Dr % 8 == 0 && al(ctx_pe, 16)) ? 1 : 0;
  a.kbuf = static_cast<bf16_t*>(workspace);
  a.vbuf = a.kbuf + (size_t)a.B * a.H * a.S_kvp * a.DQKp;
  return a;
}

}  // namespace dsmoe

using namespace dsmoe;

extern "C" size_t dsmoe_mla_attn_workspace_size(const dsmoe_mla_dims* dims) {
  if (mla_validate(dims) != DSMOE_OK) return 0;
  const MlaArgs a = mla_args(dims);
  return (size_t)a.B * a.H * a.S_kvp * (a.DQKp + a.DVp) * sizeof(bf16_t) + 256;
}

static int mla_fwd(const void* q_nope, const void* q_pe, const void* ctx_kv, const void* ctx_pe, const void* wkv_b_k,
                   const void* wkv_b_v, const dsmoe_mla_dims* dims, void* out, float* lse, void* workspace,
                   size_t workspace_bytes, void* stream) {
  int rc = mla_validate(dims);
  if (rc) return rc;
  DSMOE_REQUIRE(q_nope && q_pe && ctx_kv && ctx_pe && wkv_b_k && wkv_b_v && out, DSMOE_ERR_INVALID,
                "mla: NULL tensor pointer");
  const size_t need = dsmoe_mla_attn_workspace_size(dims);
  DSMOE_REQUIRE(workspace && workspace_bytes >= need, DSMOE_ERR_WORKSPACE, "mla: workspace too small");
  DSMOE_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0, DSMOE_ERR_INVALID,
                "mla: workspace must be 16-byte aligned");
  MlaArgs a = mla_bind(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, dims, workspace);
  a.out = static_cast<bf16_t*>(out);
  a.lse = lse;
  a.ovec = (a.Dv % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0) ? 1 : 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  rc = mla_launch_kv(a, st);
  if (rc) return rc;
  switch (a.DQKp / 16) {
    case 2: return mla_launch_fa_nv<2>(a, st);
    case 4: return mla_launch_fa_nv<4>(a, st);
    case 6: return mla_launch_fa_nv<6>(a, st);
    case 8: return mla_launch_fa_nv<8>(a, st);
    case 12: return mla_launch_fa_nv<12>(a, st);
    default: return mla_launch_fa_nv<16>(a, st);
  }
}

extern "C" int dsmoe_mla_attn_fwd(const void* q_nope, const void* q_pe, const void* ctx_kv, const void* ctx_pe,
                                  const void* wkv_b_k, const void* wkv_b_v, const dsmoe_mla_dims* dims, void* out,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  return mla_fwd(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, dims, out, nullptr, workspace, workspace_bytes,
                 stream);
}

extern "C" int dsmoe_mla_attn_fwd_lse(const void* q_nope, const void* q_pe, const void* ctx_kv, const void* ctx_pe,
                                      const void* wkv_b_k, const void* wkv_b_v, const dsmoe_mla_dims* dims, void* out,
                                      float* lse, void* workspace, size_t workspace_bytes, void* stream) {
  DSMOE_REQUIRE(lse, DSMOE_ERR_INVALID, "mla: NULL lse pointer");
  return mla_fwd(q_nope, q_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, dims, out, lse, workspace, workspace_bytes, stream);
}

// K and V alone: the forward's first launch, for a backward whose caller did
// not keep the forward's workspace.
extern "C" int dsmoe_mla_attn_kv(const void* ctx_kv, const void* ctx_pe, const void* wkv_b_k, const void* wkv_b_v,
                                 const dsmoe_mla_dims* dims, void* kv_ws, size_t kv_bytes, void* stream) {
  const int rc = mla_validate(dims);
  if (rc) return rc;
  DSMOE_REQUIRE(ctx_kv && ctx_pe && wkv_b_k && wkv_b_v, DSMOE_ERR_INVALID, "mla: NULL tensor pointer");
  DSMOE_REQUIRE(kv_ws && kv_bytes >= dsmoe_mla_attn_workspace_size(dims), DSMOE_ERR_WORKSPACE,
                "mla: workspace too small");
  DSMOE_REQUIRE((reinterpret_cast<uintptr_t>(kv_ws) & 15) == 0, DSMOE_ERR_INVALID,
                "mla: workspace must be 16-byte aligned");
  // (no queries: the query-load flag, which K, V do not use, sees ctx_kv)
  const MlaArgs a = mla_bind(ctx_kv, ctx_pe, ctx_kv, ctx_pe, wkv_b_k, wkv_b_v, dims, kv_ws);
  return mla_launch_kv(a, static_cast<hipStream_t>(stream));
}

// Workspace of dsmoe_mla_attn_bwd: the packed query and dO rows and the
// padded lse and D (S_qp rows each), each part a multiple of 256 bytes.
static size_t mla_bwd_part(const MlaArgs& a, int part) {
  const size_t rows = (size_t)a.B * a.H * a.S_qp;
  switch (part) {
    case 1: return rows * a.DQKp * sizeof(bf16_t);
    case 2: return rows * a.DVp * sizeof(bf16_t);
    default: return rows * sizeof(float);   // lse, D
  }
}

extern "C" size_t dsmoe_mla_attn_bwd_workspace_size(const dsmoe_mla_dims* dims) {
  if (mla_validate(dims) != DSMOE_OK) return 0;
  const MlaArgs a = mla_args(dims);
  return mla_bwd_part(a, 1) + mla_bwd_part(a, 2) + 2 * mla_bwd_part(a, 3) + 256;
}

extern "C" int dsmoe_mla_attn_bwd(const void* q_nope, const void* q_pe, const dsmoe_mla_dims* dims,
                                  const void* kv_ws, size_t kv_bytes, const void* out, const void* dout,
                                  const float* lse, float* dq_nope, float* dq_pe, void* dkv, float* dk_pe,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  int rc = mla_validate(dims);
  if (rc) return rc;
  DSMOE_REQUIRE(q_nope && q_pe && out && dout && lse, DSMOE_ERR_INVALID, "mla: NULL tensor pointer");
  DSMOE_REQUIRE(dq_nope && dq_pe && dkv && dk_pe, DSMOE_ERR_INVALID, "mla: NULL gradient pointer");
  DSMOE_REQUIRE(kv_ws && kv_bytes >= dsmoe_mla_attn_workspace_size(dims), DSMOE_ERR_WORKSPACE,
                "mla: K, V workspace too small");
  const size_t need = dsmoe_mla_attn_bwd_workspace_size(dims);
  DSMOE_REQUIRE(workspace && workspace_bytes >= need, DSMOE_ERR_WORKSPACE, "mla: workspace too small");
  DSMOE_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0 && (reinterpret_cast<uintptr_t>(kv_ws) & 15) == 0,
                DSMOE_ERR_INVALID, "mla: workspaces must be 16-byte aligned");
  // queries, and K, V as the forward left them
  MlaArgs a = mla_args(dims);
  a.q_nope = static_cast<const bf16_t*>(q_nope);
  a.q_pe = static_cast<const bf16_t*>(q_pe);
  a.qvec = (a.Dn % 8 == 0 && a.Dr % 8 == 0 && (reinterpret_cast<uintptr_t>(q_nope) & 15) == 0 &&
            (reinterpret_cast<uintptr_t>(q_pe) & 15) == 0) ? 1 : 0;
  a.kbuf = static_cast<bf16_t*>(const_cast<void*>(kv_ws));
  a.vbuf = a.kbuf + (size_t)a.B * a.H * a.S_kvp * a.DQKp;
  a.out = static_cast<bf16_t*>(const_cast<void*>(out));   // read only (D)
  a.dout = static_cast<const bf16_t*>(dout);
  a.lse = const_cast<float*>(lse);                          // read only
  a.dovec = (a.Dv % 8 == 0 && (reinterpret_cast<uintptr_t>(dout) & 15) == 0) ? 1 : 0;
  a.outvec = (a.Dv % 8 == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0) ? 1 : 0;
  a.dqvec = (a.Dn % 8 == 0 && a.Dr % 8 == 0 && (reinterpret_cast<uintptr_t>(dq_nope) & 15) == 0 &&
             (reinterpret_cast<uintptr_t>(dq_pe) & 15) == 0) ? 1 : 0;
  // parts: packed query rows, packed dO rows, lse, D (S_qp = 64-row
  // multiples): every part starts 256-byte aligned
  char* ws = static_cast<char*>(workspace);
  size_t off = 0;
  a.qpk = reinterpret_cast<bf16_t*>(ws + off);
  off += mla_bwd_part(a, 1);
  a.dopk = reinterpret_cast<bf16_t*>(ws + off);
  off += mla_bwd_part(a, 2);
  a.lsep = reinterpret_cast<float*>(ws + off);
  off += mla_bwd_part(a, 3);
  a.deltap = reinterpret_cast<float*>(ws + off);
  a.dq_nope = dq_nope;
  a.dq_pe = dq_pe;
  a.dkv = static_cast<bf16_t*>(dkv);
  a.dk_pe = dk_pe;
  a.kvec = (a.Dn % 4 == 0 && a.Dv % 4 == 0 && (reinterpret_cast<uintptr_t>(dkv) & 7) == 0) ? 1 : 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (a.DQKp / 16) {
    case 2: return mla_launch_bwd_nv<2>(a, st);
    case 4: return mla_launch_bwd_nv<4>(a, st);
    case 6: return mla_launch_bwd_nv<6>(a, st);
    case 8: return mla_launch_bwd_nv<8>(a, st);
    case 12: return mla_launch_bwd_nv<12>(a, st);
    default: return mla_launch_bwd_nv<16>(a, st);
  }
}
