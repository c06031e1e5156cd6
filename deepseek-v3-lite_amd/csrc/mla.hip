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
#include <cstring>

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
  bf16_t* kbuf;           // (B, H, S_kvp, DQKp)
  bf16_t* vbuf;           // (B, H, S_kvp, DVp)
  int B, H, S_q, S_kv, R, Dn, Dr, Dv;
  int Rp, DQKp, DVp, S_kvp;
  int causal, q_start;
  int ksplit;             // K row = [k_hi | pe | k_lo] (else [k | pe])
  float c;                // softmax_scale * log2(e)
};

// ---------------------------------------------------------------- K, V materialisation
// Grid (B * S_kvp / 64, H).  A workgroup takes 64 latent rows of one batch
// and one head and walks the head's Dn + Dv output columns in chunks of 64:
// LDS holds the rows (64 x Rp) and the chunk's weight rows (64 x Rp), each
// row padded by 16 bytes so the 16-byte fragment reads of 16 lanes hit 16
// distinct bank groups.  Wave (wr, wc) computes rows 32 wr.., columns 32 wc..
// with the latent rows as the first MFMA operand: a lane holds one output
// column and 16 rows, so each store instruction writes 32 consecutive
// columns of a row.  Rows past S_kv are loaded as zeros, so their K and V
// rows come out zero; the rope and padding columns are written directly.
__global__ __launch_bounds__(256) void mla_kv_kernel(const MlaArgs a) {
  extern __shared__ __attribute__((aligned(16))) char mla_kv_smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = wave >> 1, wc = wave & 1;
  const int tiles_per_b = a.S_kvp / MLA_RB;
  const int b = blockIdx.x / tiles_per_b;
  const int s0 = (blockIdx.x - b * tiles_per_b) * MLA_RB;
  const int h = blockIdx.y;
  const int rs = a.Rp * 2 + 16;            // LDS row stride (bytes)
  char* sa = mla_kv_smem;                  // latent rows
  char* sb = mla_kv_smem + MLA_RB * rs;    // weight rows of the chunk
  const int cpr = a.Rp / 8;                // 16-byte chunks per row
  // latent rows (zeros past S_kv and past R); 16-byte loads when rows are
  // 16-byte aligned (R % 8 == 0)
  const bool vec = (a.R & 7) == 0;
  auto load_row8 = [&](const bf16_t* row, bool ok, int c) -> mla_u32x4 {
    if (!ok) return mla_u32x4{0u, 0u, 0u, 0u};
    if (vec) return *reinterpret_cast<const mla_u32x4*>(row + c * 8);
    bf16_t v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = c * 8 + e < a.R ? row[c * 8 + e] : bf16_t(0);
    return *reinterpret_cast<const mla_u32x4*>(v);
  };
  for (int i = tid; i < MLA_RB * cpr; i += 256) {
    const int r = i / cpr, c = i - r * cpr;
    const int s = s0 + r;
    *reinterpret_cast<mla_u32x4*>(sa + r * rs + c * 16) =
        load_row8(a.ctx_kv + ((int64_t)b * a.S_kv + s) * a.R, s < a.S_kv && c * 8 < a.R, c);
  }
  const int64_t bh = (int64_t)b * a.H + h;
  bf16_t* krow0 = a.kbuf + (bh * a.S_kvp + s0) * a.DQKp;
  bf16_t* vrow0 = a.vbuf + (bh * a.S_kvp + s0) * a.DVp;
  // rope columns and the zero padding of K (the k_lo columns come from the
  // GEMM below), padding of V
  const int lo_end = a.ksplit ? 2 * a.Dn + a.Dr : a.Dn + a.Dr;
  for (int i = tid; i < MLA_RB * (a.DQKp - a.Dn); i += 256) {
    const int r = i / (a.DQKp - a.Dn), j = a.Dn + (i - r * (a.DQKp - a.Dn));
    const int s = s0 + r;
    if (j >= a.Dn + a.Dr && j < lo_end) continue;
    bf16_t v = bf16_t(0);
    if (s < a.S_kv && j < a.Dn + a.Dr) v = a.ctx_pe[((int64_t)b * a.S_kv + s) * a.Dr + (j - a.Dn)];
    krow0[(int64_t)r * a.DQKp + j] = v;
  }
  for (int i = tid; i < MLA_RB * (a.DVp - a.Dv); i += 256) {
    const int r = i / (a.DVp - a.Dv), j = a.Dv + (i - r * (a.DVp - a.Dv));
    vrow0[(int64_t)r * a.DVp + j] = bf16_t(0);
  }
  const int ncols = a.Dn + a.Dv;
  for (int n0 = 0; n0 < ncols; n0 += 64) {
    __syncthreads();   // the previous chunk's weight rows are read (first pass: the latent rows are written)
    for (int i = tid; i < 64 * cpr; i += 256) {
      const int r = i / cpr, c = i - r * cpr;
      const int n = n0 + r;
      const bf16_t* wrow = n < a.Dn ? a.w_k + ((int64_t)h * a.Dn + n) * a.R
                                    : a.w_v + ((int64_t)h * a.Dv + (n - a.Dn)) * a.R;
      *reinterpret_cast<mla_u32x4*>(sb + r * rs + c * 16) = load_row8(wrow, n < ncols && c * 8 < a.R, c);
    }
    __syncthreads();
    mla_f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    const int rl = 32 * wr + (lane & 31), nl = 32 * wc + (lane & 31);
    for (int k = 0; k < a.Rp; k += 16) {
      const int cb = (k + 8 * (lane >> 5)) * 2;
      const bf16x8_t fw = *reinterpret_cast<const bf16x8_t*>(sb + nl * rs + cb);
      const bf16x8_t fx = *reinterpret_cast<const bf16x8_t*>(sa + rl * rs + cb);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fx, fw, acc, 0, 0, 0);
    }
    // lane: column n = n0 + 32 wc + (lane & 31), latent rows
    // 32 wr + 8 (i / 4) + 4 (lane >> 5) + i % 4
    const int n = n0 + nl;
    if (n < ncols) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 32 * wr + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        const bf16_t v = f2bf(acc[i]);
        if (n < a.Dn) {
          krow0[(int64_t)r * a.DQKp + n] = v;
          if (a.ksplit) krow0[(int64_t)r * a.DQKp + a.Dn + a.Dr + n] = f2bf(acc[i] - bf2f(v));
        } else {
          vrow0[(int64_t)r * a.DVp + (n - a.Dn)] = v;
        }
      }
    }
  }
}

// ---------------------------------------------------------------- attention
// LDS per buffer: K tile 64 x (DQKp * 2 + 16) bytes, then V tile 64 x DVp * 2
// bytes with 8-byte unit u of key row k stored at u ^ mla_vswz(k): the
// transposing reads of 32 lanes cover four consecutive key rows and eight
// units each, which this spreads over distinct banks.
template <int NV>
__device__ __forceinline__ int mla_vswz(int k) {
  return NV == 1 ? 0 : NV == 2 ? 8 * ((k >> 1) & 1) : 8 * (k & 3);
}

template <int NSTEP, int NV>
struct MlaCfg {
  static constexpr int DQKp = NSTEP * 16;
  static constexpr int DVp = NV * 32;
  static constexpr int KRS = DQKp * 2 + 16;            // K row stride (bytes)
  static constexpr int KT = MLA_KB * KRS;              // K tile bytes
  static constexpr int VT = MLA_KB * DVp * 2;          // V tile bytes
  static constexpr int BUF = KT + VT;
  static constexpr int KCH = MLA_KB * DQKp / 8;        // 16-byte chunks of a K tile
  static constexpr int VCH = MLA_KB * DVp / 8;
  static constexpr int NLK = (KCH + 255) / 256;        // loads per thread
  static constexpr int NLV = (VCH + 255) / 256;
};

__device__ __forceinline__ float mla_pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}
__device__ __forceinline__ float mla_pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}

// Work items (batch, head, query block) are numbered (batch, head)-major with
// a head's query blocks last-first (causal: the longest first); block i runs
// on XCD i % 8 and the XCDs take contiguous eighths of the items, so the
// query blocks of a head share their XCD's L2 copy of its K and V.
template <int NSTEP, int NV>
__global__ __launch_bounds__(256) void mla_fa_kernel(const MlaArgs a) {
  using C = MlaCfg<NSTEP, NV>;
  extern __shared__ __attribute__((aligned(16))) char mla_smem[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hi = lane >> 5, ql = lane & 31;
  const int nq = (a.S_q + MLA_QB - 1) / MLA_QB;
  const int total = nq * a.H * a.B;
  const int per = (total + 7) / 8;
  const int item = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
  if (item >= total) return;
  const int hb = item / nq;
  const int h = hb % a.H, b = hb / a.H;
  const int q0 = (nq - 1 - (item - hb * nq)) * MLA_QB;
  const int qi = q0 + 32 * wave + ql;          // this lane's query
  const int64_t bh = (int64_t)b * a.H + h;

  // query fragments: step st holds columns 16 st + 8 hi .. +7 of
  // [q_nope | q_pe | q_nope (split K) | 0]
  bf16x8_t qf[NSTEP];
  {
    const bf16_t* qn = a.q_nope + (bh * a.S_q + qi) * a.Dn;
    const bf16_t* qp = a.q_pe + (bh * a.S_q + qi) * a.Dr;
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
        }
      }
      qf[st] = *reinterpret_cast<const bf16x8_t*>(v);
    }
  }

  // keys this workgroup needs
  int kend = a.S_kv;
  if (a.causal) kend = min(kend, min(q0 + MLA_QB, a.S_q) - 1 + a.q_start + 1);
  const int nkb = (kend + MLA_KB - 1) / MLA_KB;
  const bf16_t* kg = a.kbuf + bh * a.S_kvp * C::DQKp;
  const bf16_t* vg = a.vbuf + bh * a.S_kvp * C::DVp;

  mla_u32x4 kst[C::NLK], vst[C::NLV];
  auto gload = [&](int kb) {
    const int k0 = kb * MLA_KB;
#pragma unroll
    for (int i = 0; i < C::NLK; ++i) {
      const int c = tid + 256 * i;
      if (c < C::KCH) {
        const int r = c / (C::DQKp / 8), cc = c - r * (C::DQKp / 8);
        kst[i] = *reinterpret_cast<const mla_u32x4*>(kg + (int64_t)(k0 + r) * C::DQKp + cc * 8);
      }
    }
#pragma unroll
    for (int i = 0; i < C::NLV; ++i) {
      const int c = tid + 256 * i;
      if (c < C::VCH) {
        const int r = c / (C::DVp / 8), cc = c - r * (C::DVp / 8);
        vst[i] = *reinterpret_cast<const mla_u32x4*>(vg + (int64_t)(k0 + r) * C::DVp + cc * 8);
      }
    }
  };
  auto lstore = [&](int buf) {
    char* kt = mla_smem + buf * C::BUF;
    char* vt = kt + C::KT;
#pragma unroll
    for (int i = 0; i < C::NLK; ++i) {
      const int c = tid + 256 * i;
      if (c < C::KCH) {
        const int r = c / (C::DQKp / 8), cc = c - r * (C::DQKp / 8);
        *reinterpret_cast<mla_u32x4*>(kt + r * C::KRS + cc * 16) = kst[i];
      }
    }
#pragma unroll
    for (int i = 0; i < C::NLV; ++i) {
      const int c = tid + 256 * i;
      if (c < C::VCH) {
        const int r = c / (C::DVp / 8), cc = c - r * (C::DVp / 8);
        *reinterpret_cast<mla_u32x4*>(vt + r * (C::DVp * 2) + (((2 * cc) ^ mla_vswz<NV>(r)) << 3)) = vst[i];
      }
    }
  };

  mla_f32x16 o[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[v][i] = 0.0f;
  float m = -INFINITY, l = 0.0f;
  const int qpos = qi + a.q_start;

  if (nkb > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int k0 = kb * MLA_KB;
    if (kb + 1 < nkb) gload(kb + 1);
    const char* kt = mla_smem + (kb & 1) * C::BUF;
    const char* vt = kt + C::KT;
    // scores: sub-tile t, register i -> key k0 + 32 t + 8 (i / 4) + 4 hi + i % 4
    mla_f32x16 s[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[t][i] = 0.0f;
#pragma unroll
      for (int st = 0; st < NSTEP; ++st) {
        const bf16x8_t kf = *reinterpret_cast<const bf16x8_t*>(kt + (32 * t + ql) * C::KRS + (2 * st + hi) * 16);
        s[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[st], s[t], 0, 0, 0);
      }
    }
    // scores in log2 units (scale * log2 e); masks: keys past S_kv and, with
    // the causal mask, keys past the query
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[t][i] *= a.c;
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
    const float mc = mn == -INFINITY ? 0.0f : mn;
    const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mc);
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
          p[e] = __builtin_amdgcn_exp2f(s[t][8 * half + e] - mc);
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
#pragma unroll
    for (int v = 0; v < NV; ++v)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[v][i] *= alpha;
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
    if (kb + 1 < nkb) lstore((kb + 1) & 1);
    __syncthreads();
  }

  // out[b, qi, h, dv]: lane holds dv = 32 v + 8 (i / 4) + 4 hi + i % 4
  const float lt = mla_pair_sum(l);
  const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
  if (qi >= a.S_q) return;
  bf16_t* orow = a.out + (((int64_t)b * a.S_q + qi) * a.H + h) * a.Dv;
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int dv = 32 * v + 8 * g + 4 * hi;
      if (dv + 3 < a.Dv && (a.Dv & 3) == 0) {
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
  a.causal = d->is_causal ? 1 : 0;
  a.q_start = d->q_start;
  a.c = d->softmax_scale * MLA_LOG2E;
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
  const int64_t total = cdiv(a.S_q, MLA_QB) * a.H * a.B;
  hipLaunchKernelGGL(kern, dim3((unsigned)(8 * cdiv(total, 8))), dim3(256), lds, st, a);
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

}  // namespace dsmoe

using namespace dsmoe;

extern "C" size_t dsmoe_mla_attn_workspace_size(const dsmoe_mla_dims* dims) {
  if (mla_validate(dims) != DSMOE_OK) return 0;
  const MlaArgs a = mla_args(dims);
  return (size_t)a.B * a.H * a.S_kvp * (a.DQKp + a.DVp) * sizeof(bf16_t) + 256;
}

extern "C" int dsmoe_mla_attn_fwd(const void* q_nope, const void* q_pe, const void* ctx_kv, const void* ctx_pe,
                                  const void* wkv_b_k, const void* wkv_b_v, const dsmoe_mla_dims* dims, void* out,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  int rc = mla_validate(dims);
  if (rc) return rc;
  DSMOE_REQUIRE(q_nope && q_pe && ctx_kv && ctx_pe && wkv_b_k && wkv_b_v && out, DSMOE_ERR_INVALID,
                "mla: NULL tensor pointer");
  const size_t need = dsmoe_mla_attn_workspace_size(dims);
  DSMOE_REQUIRE(workspace && workspace_bytes >= need, DSMOE_ERR_WORKSPACE, "mla: workspace too small");
  DSMOE_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 15) == 0, DSMOE_ERR_INVALID,
                "mla: workspace must be 16-byte aligned");
  MlaArgs a = mla_args(dims);
  a.q_nope = static_cast<const bf16_t*>(q_nope);
  a.q_pe = static_cast<const bf16_t*>(q_pe);
  a.ctx_kv = static_cast<const bf16_t*>(ctx_kv);
  a.ctx_pe = static_cast<const bf16_t*>(ctx_pe);
  a.w_k = static_cast<const bf16_t*>(wkv_b_k);
  a.w_v = static_cast<const bf16_t*>(wkv_b_v);
  a.out = static_cast<bf16_t*>(out);
  a.kbuf = static_cast<bf16_t*>(workspace);
  a.vbuf = a.kbuf + (size_t)a.B * a.H * a.S_kvp * a.DQKp;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const size_t kv_lds = 2 * (size_t)MLA_RB * (a.Rp * 2 + 16);
  static const hipError_t kv_attr = hipFuncSetAttribute((const void*)mla_kv_kernel,
                                                        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  if (kv_attr != hipSuccess) return fail(DSMOE_ERR_HIP, "mla: cannot raise LDS limit");
  hipLaunchKernelGGL(mla_kv_kernel, dim3((unsigned)(a.B * (a.S_kvp / MLA_RB)), (unsigned)a.H), dim3(256), kv_lds,
                     st, a);
  rc = check_launch("mla_kv");
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
