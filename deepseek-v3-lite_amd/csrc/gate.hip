// (a) Fused gate: fp32 logits = x . W_gate^T, sigmoid, +bias, top-k,
// renormalisation, per-expert histogram.  Restates models/moe.py:29-37 and
// the bincount of models/moe.py:114 (see dsmoe.h for the tie rule).
//
// Logits, bf16 x: MFMA.  Each fp32 gate weight is split exactly into three
// bf16 parts by truncation (w = hi + mid + lo: hi keeps the top 8 significand
// bits, mid the next 8, lo the last 8), so x.w = x.lo + x.mid + x.hi with
// every product exact; the MFMA accumulates in fp32.  A workgroup takes
// GP_TOK = 128 tokens (wave w: tokens 32w .. 32w + 31) and every expert over
// one K split of D / ks columns: the workgroup's W rows of each K chunk are
// loaded once (row-contiguous 16-byte loads), split, and staged in LDS as
// three bf16 planes (double-buffered, one barrier per chunk), so the split
// work and the W traffic per workgroup shrink with ks.  With ks splits the
// partial logits go to a workspace and the routing launch adds them in split
// order; without a workspace (ks = 1) the workgroup routes its own tokens.
// fp32 x: SIMT FMA tiles.
//
// Routing.  One wave per token, one lane per expert (E <= 64; E <= 256 with
// several experts per lane): sigmoid in double rounded once, + bias, then k
// rounds of a wave-wide arg-max ordered by (value desc, expert id asc).  The
// routing launch of the MFMA gate takes rank blocks of 64 tokens and also
// ranks their slots for the permute (rank.h).
#include <cstdlib>
#include <cstring>
#include <type_traits>
#include <mutex>
#include <vector>

#include "rank.h"
#include "route.h"

namespace dsmoe {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 g_bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float g_f32x16_t;
typedef float g_f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int g_u32x4_t __attribute__((ext_vector_type(4)));

constexpr int GATE_THREADS = 256;
constexpr int GATE_KC = 32;        // SIMT: K chunk staged through LDS
constexpr int GP_TOK = 128;        // MFMA: tokens per workgroup
constexpr int GP_THREADS = 512;    // MFMA: 8 waves = 4 token groups x 2 expert halves

// MFMA gate tiling.  A workgroup takes GP_TOK tokens (wave w: token group
// w & 3 of 32, expert tiles (w >> 2) + 2i of 32) over its K split, in
// super-chunks of SC columns.  The super-chunk's W rows (all experts) are
// loaded by every thread (row-contiguous 16-byte loads), split, and staged as
// three bf16 planes in LDS (at most 96 KB); its x rows are loaded the same way
// (each wave instruction reads 1 KB of whole rows) and staged as a fourth
// plane of GP_TOK rows.  Each wave then runs all its MFMAs of the super-chunk
// from LDS without another barrier, while the loads of the next super-chunk
// are in flight in registers.
// The widest super-chunk of NT expert tiles (planes of at most 96 KB).
constexpr int gp_sc_max(int nt) { return nt <= 2 ? 256 : nt <= 4 ? 128 : 64; }

template <int NT, int SC_ = gp_sc_max(NT)>
struct GPCfg {
  static constexpr int EP = NT * 32;                          // experts padded to whole 32-row tiles
  static constexpr int SC = SC_;                              // super-chunk K
  static constexpr int ROWB = SC * 2;                         // bytes of one plane row (bf16)
  static constexpr int SWZ = (ROWB / 16 >= 16 ? 16 : ROWB / 16) - 1;  // 16-byte unit swizzle mask
  static constexpr int PLANE = EP * ROWB;
  static constexpr int F4R = SC / 4;                          // float4 loads per W row and super-chunk
  static constexpr int NLD = EP * F4R / GP_THREADS;           // float4 loads per thread and super-chunk
  static constexpr int STEPS = SC / 16;                       // MFMA K steps per super-chunk
  static constexpr int NTW = (NT + 1) / 2;                    // expert tiles per wave (at most)
  static constexpr int XUR = SC / 8;                          // 16-byte units of one x row
  static constexpr int NXL = GP_TOK * XUR / GP_THREADS;       // x loads per thread and super-chunk
  static constexpr int XPLANE = 3 * PLANE;                    // LDS offset of the x plane (GP_TOK rows)
  static constexpr int LDS = XPLANE + GP_TOK * ROWB;
};

template <int NT, int SC>
constexpr size_t gp_lds(bool route) {
  // routing: lg[GP_TOK][EP + 1] | bias[EP] | hist[EP] | scratch (64 ints per wave)
  constexpr size_t r = (size_t)4 * (GP_TOK * (NT * 32 + 1) + 2 * NT * 32 + GP_THREADS);
  return route && r > (size_t)GPCfg<NT, SC>::LDS ? r : (size_t)GPCfg<NT, SC>::LDS;
}

// Splits 4 fp32 weights into three bf16x4 words (hi, mid, lo) whose sum is
// exact: hi = w truncated to bf16, r1 = w - hi (exact, <= 16 significant
// bits), mid = r1 truncated, lo = r1 - mid (exact, <= 8 significant bits).
__device__ __forceinline__ void split3x4(const g_f32x4_t& w, uint2& hi, uint2& mid, uint2& lo) {
  uint32_t h[4], m[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t wb = __float_as_uint(w[i]);
    const float r1 = w[i] - __uint_as_float(wb & 0xffff0000u);
    const uint32_t rb = __float_as_uint(r1);
    const float r2 = r1 - __uint_as_float(rb & 0xffff0000u);
    h[i] = wb;
    m[i] = rb;
    l[i] = __float_as_uint(r2);
  }
  hi = make_uint2((h[0] >> 16) | (h[1] & 0xffff0000u), (h[2] >> 16) | (h[3] & 0xffff0000u));
  mid = make_uint2((m[0] >> 16) | (m[1] & 0xffff0000u), (m[2] >> 16) | (m[3] & 0xffff0000u));
  lo = make_uint2((l[0] >> 16) | (l[1] & 0xffff0000u), (l[2] >> 16) | (l[3] & 0xffff0000u));
}

// LDS plane layout: row e of a plane holds the super-chunk's SC bf16 of
// expert e; its 16-byte unit u sits at unit u ^ (e & SWZ).
template <class C>
__device__ __forceinline__ int gp_unit_off(int row, int unit) {
  return row * C::ROWB + ((unit ^ (row & C::SWZ)) << 4);
}

// ROUTE = false: partial logits of split blockIdx.x % ks for token tile
// blockIdx.x / ks go to part[(split * T + t) * E + e].  ROUTE = true (ks = 1):
// the workgroup routes its tokens (logits in LDS).
template <int NT, int SC, bool ROUTE>
__global__ __launch_bounds__(GP_THREADS) void gate_mfma_kernel(const bf16_t* __restrict__ x,
                                                               const float* __restrict__ gw,
                                                               const float* __restrict__ bias, int T, int D, int E,
                                                               int k, float route_scale, GateOut out,
                                                               float* __restrict__ part, int ks, const PtrChunk tables,
                                                               const void** tab_dst) {
  using C = GPCfg<NT, SC>;
  extern __shared__ __attribute__((aligned(16))) char gsm[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (blockIdx.x == 0)
    for (int i = tid; i < tables.n; i += blockDim.x) tab_dst[tables.off + i] = tables.p[i];
  const int split = (int)(blockIdx.x % ks);
  const int t0 = (int)(blockIdx.x / ks) * GP_TOK;
  const int dk = D / ks;
  const int kbeg = split * dk;
  const int nsc = dk / C::SC;
  // W staging: load i of this thread reads float4 c4 of row r0 + i * (GP_THREADS / F4R)
  constexpr int RSTEP = GP_THREADS / C::F4R;
  const int c4 = tid % C::F4R, r0 = tid / C::F4R;
  const float* wsrc = gw + (int64_t)kbeg + c4 * 4;
  // x staging: load q of this thread reads unit xu of token row xr0 + q * (GP_THREADS / XUR)
  constexpr int XRSTEP = GP_THREADS / C::XUR;
  const int xu = tid % C::XUR, xr0 = tid / C::XUR;
  const bf16_t* xsrc = x + (int64_t)kbeg + xu * 8;
  const int tg = wave & 3, eh = wave >> 2;
  const int ntw = (NT - eh + 1) / 2;                  // this wave's expert tiles: eh, eh + 2, ...
  const bool wave_live = t0 + tg * 32 < T && ntw > 0;
  const int m = lane & 31;
  g_f32x4_t wr[C::NLD];
  g_u32x4_t xv[C::NXL];
  g_f32x16_t acc[C::NTW];
#pragma unroll
  for (int i = 0; i < C::NTW; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;

  auto xload = [&](int sc) {
#pragma unroll
    for (int q = 0; q < C::NXL; ++q)
      xv[q] = *reinterpret_cast<const g_u32x4_t*>(xsrc + (int64_t)min(t0 + xr0 + q * XRSTEP, T - 1) * D + sc * C::SC);
  };
  auto xstage = [&]() {
#pragma unroll
    for (int q = 0; q < C::NXL; ++q)
      *reinterpret_cast<g_u32x4_t*>(gsm + C::XPLANE + gp_unit_off<C>(xr0 + q * XRSTEP, xu)) = xv[q];
  };
  auto wload = [&](int sc) {
#pragma unroll
    for (int i = 0; i < C::NLD; ++i)
      wr[i] = *reinterpret_cast<const g_f32x4_t*>(wsrc + (int64_t)min(r0 + i * RSTEP, E - 1) * D + sc * C::SC);
  };
  auto wstage = [&]() {
#pragma unroll
    for (int i = 0; i < C::NLD; ++i) {
      uint2 hi, mid, lo;
      split3x4(wr[i], hi, mid, lo);
      const int o = gp_unit_off<C>(r0 + i * RSTEP, c4 >> 1) + ((c4 & 1) << 3);
      *reinterpret_cast<uint2*>(gsm + o) = hi;
      *reinterpret_cast<uint2*>(gsm + C::PLANE + o) = mid;
      *reinterpret_cast<uint2*>(gsm + 2 * C::PLANE + o) = lo;
    }
  };
  // x fragment: token row tg * 32 + (lane & 31), 8 bf16 at K offset (lane >> 5) * 8 + 16 s
  auto compute = [&]() {
    if (!wave_live) return;
#pragma unroll
    for (int s = 0; s < C::STEPS; ++s) {
      const g_bf16x8_t xa =
          *reinterpret_cast<const g_bf16x8_t*>(gsm + C::XPLANE + gp_unit_off<C>(tg * 32 + m, 2 * s + (lane >> 5)));
#pragma unroll
      for (int i = 0; i < C::NTW; ++i) {
        if (i < ntw) {
          const int o = gp_unit_off<C>((eh + 2 * i) * 32 + m, 2 * s + (lane >> 5));
          const g_bf16x8_t bhi = *reinterpret_cast<const g_bf16x8_t*>(gsm + o);
          const g_bf16x8_t bmid = *reinterpret_cast<const g_bf16x8_t*>(gsm + C::PLANE + o);
          const g_bf16x8_t blo = *reinterpret_cast<const g_bf16x8_t*>(gsm + 2 * C::PLANE + o);
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(blo, xa, acc[i], 0, 0, 0);
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bmid, xa, acc[i], 0, 0, 0);
          acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bhi, xa, acc[i], 0, 0, 0);
        }
      }
    }
  };

  // super-chunk sc: stage its W planes and x rows, barrier, issue the loads
  // of sc + 1 into registers, run the MFMAs, barrier (the planes are
  // rewritten next)
  xload(0);
  wload(0);
  for (int sc = 0; sc < nsc; ++sc) {
    wstage();
    xstage();
    __syncthreads();
    if (sc + 1 < nsc) {
      wload(sc + 1);
      xload(sc + 1);
    }
    compute();
    __syncthreads();
  }
  // lane holds token m of its group, experts ni*32 + 8*(r/4) + 4*(lane/32) + r%4
  const int t = t0 + tg * 32 + m;
  if constexpr (!ROUTE) {
    if (t < T && wave_live) {
      float* pr = part + ((int64_t)split * T + t) * E;
#pragma unroll
      for (int i = 0; i < C::NTW; ++i) {
        if (i >= ntw) break;
        const int ni = eh + 2 * i;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int e = ni * 32 + 8 * g + 4 * (lane >> 5);
          if ((E & 3) == 0) {
            if (e < E)
              *reinterpret_cast<g_f32x4_t*>(pr + e) =
                  g_f32x4_t{acc[i][4 * g], acc[i][4 * g + 1], acc[i][4 * g + 2], acc[i][4 * g + 3]};
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              if (e + q < E) pr[e + q] = acc[i][4 * g + q];
          }
        }
      }
    }
  } else {
    // the W planes are dead (the loop ended on a barrier): logits in LDS
    constexpr int LDP = C::EP + 1;
    float* lg = reinterpret_cast<float*>(gsm);     // [GP_TOK][LDP]
    float* bias_s = lg + GP_TOK * LDP;
    int* hist = reinterpret_cast<int*>(bias_s + C::EP);
    int32_t* scr = hist + C::EP;
    for (int e = tid; e < E; e += blockDim.x) {
      bias_s[e] = bias[e];
      hist[e] = 0;
    }
    if (wave_live) {
      float* pw = lg + (tg * 32 + m) * LDP;
#pragma unroll
      for (int i = 0; i < C::NTW; ++i) {
        if (i >= ntw) break;
        const int ni = eh + 2 * i;
#pragma unroll
        for (int r = 0; r < 16; ++r) pw[ni * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)] = acc[i][r];
      }
    }
    __syncthreads();
    const int ntok = min(GP_TOK, T - t0);
    if (out.logits)
      for (int i = tid; i < ntok * E; i += blockDim.x) {
        const int tt = i / E, e = i - tt * E;
        out.logits[(int64_t)(t0 + tt) * E + e] = lg[tt * LDP + e];
      }
    route_tokens(lg, LDP, ntok, t0, bias_s, E, k, route_scale, DSMOE_BF16, out, out.counts ? hist : nullptr, nullptr,
                 scr);
    __syncthreads();
    flush_hist(hist, E, out.counts);
  }
}

// Routing launch: logits = the ks partial logits added in split order (ks = 1:
// given logits), one workgroup of RR_WAVES waves per rank block of
// RANK_TOKENS tokens (four tokens per wave).  With po.offsets set it also
// ranks the block's slots (rank.h), and a call of one rank block finishes its
// permute here.
// LDS (4-byte words): lg[64][E + 1] | bias[E] | hist[E] | sel[64 k] | rank[64 k] | off[E + 1] | til[E + 1] |
// routing scratch[64 per wave]
constexpr int RR_WAVES = RANK_TOKENS / 4;

// KS > 0: ks == KS at compile time, so the split loads are unconditional and
// stay in flight together (a guarded load is waited for at its guard).
template <int KB, int KS>
__global__ __launch_bounds__(RR_WAVES * 64) void route_rank_kernel(const float* __restrict__ part, int ks_,
                                                                  const float* __restrict__ bias, int T, int E, int k,
                                                                  float route_scale, int xdtype, GateOut out,
                                                                  PermuteOut po, int nb) {
  extern __shared__ __attribute__((aligned(16))) float rsm[];
  const int ks = KS > 0 ? KS : ks_;
  const int ldl = E + 1;
  float* lg = rsm;
  float* bias_s = lg + RANK_TOKENS * ldl;
  int32_t* hist = reinterpret_cast<int32_t*>(bias_s + E);
  int32_t* sel = hist + E;
  int32_t* rank_lds = sel + RANK_TOKENS * k;
  int32_t* off = rank_lds + RANK_TOKENS * k;
  int32_t* til = off + E + 1;
  int32_t* scr = til + E + 1;
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const int t0 = b * RANK_TOKENS;
  const int ntok = max(0, min(RANK_TOKENS, T - t0));
  const bool rank = po.offsets != nullptr;
  for (int e = tid; e < E; e += blockDim.x) {
    bias_s[e] = bias[e];
    hist[e] = 0;
  }
  for (int i = tid; i < RANK_TOKENS * k; i += blockDim.x) sel[i] = -1;
  const int64_t split_stride = (int64_t)T * E;
  // each thread's loads of every split are issued before the adds (one
  // memory latency), then added in split order
  const bool lvec = (reinterpret_cast<uintptr_t>(out.logits) & 15) == 0;
  if ((E & 3) == 0) {
    const int E4 = E >> 2;
    for (int i = tid; i < ntok * E4; i += blockDim.x) {
      const int tt = i / E4, e = (i - tt * E4) * 4;
      const float* p = part + (int64_t)(t0 + tt) * E + e;
      g_f32x4_t pv[GATE_KS_MAX];
#pragma unroll
      for (int sp = 0; sp < GATE_KS_MAX; ++sp)
        if (KS > 0 ? sp < KS : sp < ks) pv[sp] = *reinterpret_cast<const g_f32x4_t*>(p + sp * split_stride);
      g_f32x4_t v = pv[0];
#pragma unroll
      for (int sp = 1; sp < GATE_KS_MAX; ++sp)
        if (sp < ks) v += pv[sp];
#pragma unroll
      for (int q = 0; q < 4; ++q) lg[tt * ldl + e + q] = v[q];
      if (out.logits) {
        float* lo = out.logits + (int64_t)(t0 + tt) * E + e;
        if (lvec)
          *reinterpret_cast<g_f32x4_t*>(lo) = v;
        else
#pragma unroll
          for (int q = 0; q < 4; ++q) lo[q] = v[q];
      }
    }
  } else {
    for (int i = tid; i < ntok * E; i += blockDim.x) {
      const int tt = i / E, e = i - tt * E;
      const float* p = part + (int64_t)(t0 + tt) * E + e;
      float pv[GATE_KS_MAX];
#pragma unroll
      for (int sp = 0; sp < GATE_KS_MAX; ++sp)
        if (KS > 0 ? sp < KS : sp < ks) pv[sp] = p[sp * split_stride];
      float v = pv[0];
#pragma unroll
      for (int sp = 1; sp < GATE_KS_MAX; ++sp)
        if (sp < ks) v += pv[sp];
      lg[tt * ldl + e] = v;
      if (out.logits) out.logits[(int64_t)(t0 + tt) * E + e] = v;
    }
  }
  __syncthreads();
  route_tokens(lg, ldl, ntok, t0, bias_s, E, k, route_scale, xdtype, out, (!rank && out.counts) ? hist : nullptr,
               rank ? sel : nullptr, scr);
  __syncthreads();
  if (!rank) {
    flush_hist(hist, E, out.counts);
    return;
  }
  const bool single = nb <= 1;
  rank_block<KB>(sel, ntok, k, E, b, po, hist, single ? rank_lds : nullptr);
  if (single) finish_single_block(sel, rank_lds, ntok, k, E, po, hist, off, til);
}

// ------------------------------------------------------------------ SIMT logits (fp32 x, or D % 64 != 0)
// LDS layout (floats): xs[KC][TB+4] | ws[KC][EC+4] | lg[TB][E+1] | bias[E] | hist[E] (int) | routing scratch
// (64 ints per wave)
template <typename XT, int EC>
__global__ __launch_bounds__(GATE_THREADS) void gate_kernel(const XT* __restrict__ x, const float* __restrict__ gw,
                                                            const float* __restrict__ bias, int T, int D, int E, int k,
                                                            float route_scale, int xdtype, GateOut out) {
  constexpr int TX = EC / 4;                   // threads along experts
  constexpr int TB = (GATE_THREADS / TX) * 4;  // tokens per block
  extern __shared__ float smem[];
  float* xs = smem;                             // [KC][TB+4]
  float* ws = xs + GATE_KC * (TB + 4);          // [KC][EC+4]
  float* lg = ws + GATE_KC * (EC + 4);          // [TB][E+1]
  float* bias_s = lg + TB * (E + 1);            // [E]
  int* hist = reinterpret_cast<int*>(bias_s + E);  // [E]
  int32_t* scr = hist + E;                      // [GATE_THREADS]

  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * TB;
  const int ldl = E + 1;
  for (int e = tid; e < E; e += GATE_THREADS) {
    bias_s[e] = bias[e];
    hist[e] = 0;
  }
  const int tx = tid % TX, ty = tid / TX;
  for (int e0 = 0; e0 < E; e0 += EC) {
    float acc[4][4] = {};
    for (int kc = 0; kc < D; kc += GATE_KC) {
      for (int i = tid; i < TB * GATE_KC; i += GATE_THREADS) {
        int t = i / GATE_KC, kk = i - t * GATE_KC;
        float v = 0.0f;
        if (t0 + t < T && kc + kk < D) v = to_f<XT>(x[(int64_t)(t0 + t) * D + kc + kk]);
        xs[kk * (TB + 4) + t] = v;
      }
      for (int i = tid; i < EC * GATE_KC; i += GATE_THREADS) {
        int e = i / GATE_KC, kk = i - e * GATE_KC;
        float v = 0.0f;
        if (e0 + e < E && kc + kk < D) v = gw[(int64_t)(e0 + e) * D + kc + kk];
        ws[kk * (EC + 4) + e] = v;
      }
      __syncthreads();
#pragma unroll 8
      for (int kk = 0; kk < GATE_KC; ++kk) {
        float4 a = *reinterpret_cast<const float4*>(&xs[kk * (TB + 4) + ty * 4]);
        float4 b = *reinterpret_cast<const float4*>(&ws[kk * (EC + 4) + tx * 4]);
        float av[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bw[j], acc[i][j]);
      }
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int e = e0 + tx * 4 + j;
        if (e < E) lg[(ty * 4 + i) * ldl + e] = acc[i][j];
      }
  }
  __syncthreads();
  const int ntok = min(TB, T - t0);
  if (out.logits) {
    for (int i = tid; i < ntok * E; i += GATE_THREADS) {
      int t = i / E, e = i - t * E;
      out.logits[(int64_t)(t0 + t) * E + e] = lg[t * ldl + e];
    }
  }
  route_tokens(lg, ldl, ntok, t0, bias_s, E, k, route_scale, xdtype, out, out.counts ? hist : nullptr, nullptr, scr);
  __syncthreads();
  flush_hist(hist, E, out.counts);
}

__global__ void fill_i32_kernel(int32_t* p, int n, int32_t v) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Raises a kernel's dynamic LDS limit to the CU's 160 KB, once per kernel and
// process (the call costs far more than a launch).
static int set_lds(const void* kern, size_t lds) {
  constexpr size_t kMax = 160 * 1024;
  if (lds <= 64 * 1024) return DSMOE_OK;
  if (lds > kMax) return fail(DSMOE_ERR_UNSUPPORTED, "gate: LDS need exceeds 160 KB");
  static std::mutex mu;
  static std::vector<const void*> raised;
  std::lock_guard<std::mutex> lock(mu);
  for (const void* p : raised)
    if (p == kern) return DSMOE_OK;
  if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kMax) != hipSuccess)
    return fail(DSMOE_ERR_HIP, "gate: cannot raise LDS limit");
  raised.push_back(kern);
  return DSMOE_OK;
}

template <typename XT, int EC>
static int launch_gate_t(const void* x, const float* gw, const float* bias, const dsmoe_dims& d, const GateOut& out,
                         hipStream_t st) {
  constexpr int TX = EC / 4;
  constexpr int TB = (GATE_THREADS / TX) * 4;
  const size_t lds = sizeof(float) * (GATE_KC * (TB + 4) + GATE_KC * (EC + 4) + TB * (d.E + 1) + d.E) +
                     sizeof(int) * (d.E + GATE_THREADS) + 16;
  auto kern = gate_kernel<XT, EC>;
  int rc = set_lds((const void*)kern, lds);
  if (rc) return rc;
  int blocks = (int)cdiv(d.T, TB);
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(GATE_THREADS), lds, st, static_cast<const XT*>(x), gw, bias, d.T, d.D,
                     d.E, d.k, d.route_scale, d.dtype, out);
  return check_launch("gate");
}

// The routing launch over ks partial (or given, ks = 1) logits.
static int launch_route(const float* part, int ks, const float* bias, const dsmoe_dims& d, const GateOut& out,
                        const PermuteOut* po, bool* ranked, hipStream_t st) {
  PermuteOut none;
  std::memset(static_cast<void*>(&none), 0, sizeof(none));
  const int nb = (int)cdiv(d.T, RANK_TOKENS);
  const size_t lds =
      sizeof(float) * (RANK_TOKENS * (d.E + 1) + 2 * d.E + 2 * RANK_TOKENS * d.k + 2 * (d.E + 1) + RR_WAVES * 64);
  // split counts are powers of two up to GATE_KS_MAX (gate_k_splits); given
  // logits (ks = 1) take the KS = 1 instantiation too
  auto pick = [&](auto kb) -> decltype(&route_rank_kernel<8, 0>) {
    constexpr int KB = decltype(kb)::value;
    switch (ks) {
      case 1: return route_rank_kernel<KB, 1>;
      case 2: return route_rank_kernel<KB, 2>;
      case 4: return route_rank_kernel<KB, 4>;
      case 8: return route_rank_kernel<KB, 8>;
      default: return route_rank_kernel<KB, 0>;
    }
  };
  auto kern = d.k <= 8 ? pick(std::integral_constant<int, 8>{}) : pick(std::integral_constant<int, MAX_TOPK>{});
  int rc = set_lds((const void*)kern, lds);
  if (rc) return rc;
  hipLaunchKernelGGL(kern, dim3((unsigned)max(nb, 1)), dim3(RR_WAVES * 64), lds, st, part, ks, bias, d.T, d.E, d.k,
                     d.route_scale, d.dtype, out, po ? *po : none, nb);
  rc = check_launch("route");
  if (!rc && po && ranked) *ranked = true;
  return rc;
}

template <int NT, int SC>
static int launch_gate_mfma(const void* x, const float* gw, const float* bias, const dsmoe_dims& d, const GateOut& out,
                            float* part, const PtrChunk* tables, const void** tab_dst, const PermuteOut* po,
                            bool* ranked, hipStream_t st) {
  PtrChunk none;
  none.n = 0;
  none.off = 0;
  const bool route = part == nullptr;
  const int ks = route ? 1 : gate_k_splits(d);
  auto kern = route ? gate_mfma_kernel<NT, SC, true> : gate_mfma_kernel<NT, SC, false>;
  const size_t lds = gp_lds<NT, SC>(route);
  int rc = set_lds((const void*)kern, lds);
  if (rc) return rc;
  const int64_t blocks = cdiv(d.T, GP_TOK) * ks;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(GP_THREADS), lds, st, static_cast<const bf16_t*>(x), gw, bias,
                     d.T, d.D, d.E, d.k, d.route_scale, out, part, ks, tables ? *tables : none, tab_dst);
  rc = check_launch("gate_mfma");
  if (rc || route) return rc;
  return launch_route(part, ks, bias, d, out, po, ranked, st);
}

// Super-chunk of the MFMA gate: the widest one for the expert count when it
// divides D, else 64 columns.
template <int NT>
static int launch_gate_mfma_nt(const void* x, const float* gw, const float* bias, const dsmoe_dims& d,
                               const GateOut& out, float* part, const PtrChunk* tables, const void** tab_dst,
                               const PermuteOut* po, bool* ranked, hipStream_t st) {
  if (d.D % gp_sc_max(NT) == 0)
    return launch_gate_mfma<NT, gp_sc_max(NT)>(x, gw, bias, d, out, part, tables, tab_dst, po, ranked, st);
  return launch_gate_mfma<NT, 64>(x, gw, bias, d, out, part, tables, tab_dst, po, ranked, st);
}

static int gate_nt(int E) { return E <= 32 ? 1 : E <= 64 ? 2 : E <= 96 ? 3 : E <= 128 ? 4 : 8; }
static int gate_sc(const dsmoe_dims& d) {
  const int w = gp_sc_max(gate_nt(d.E));
  return d.D % w == 0 ? w : 64;
}

int gate_k_splits(const dsmoe_dims& d) {
  const int64_t tiles = cdiv(d.T, GP_TOK);
  const int sc = gate_sc(d);
  int ks = 1;
  // about one workgroup per CU; a split keeps whole super-chunks
  while (ks < GATE_KS_MAX && tiles * ks * 2 <= 256 && d.D % (sc * ks * 2) == 0) ks *= 2;
  return ks;
}

size_t gate_part_floats(const dsmoe_dims& d) { return (size_t)gate_k_splits(d) * d.T * d.E; }

static bool gate_mfma_ok(const void* x, const float* gw, const dsmoe_dims& d) {
  return d.dtype == DSMOE_BF16 && d.D % 64 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(gw) & 15) == 0;
}

bool gate_uses_mfma(const void* x, const float* gw, const dsmoe_dims& d) { return d.T > 0 && gate_mfma_ok(x, gw, d); }

int launch_gate(const void* x, const float* logits_in, const float* gw, const float* bias, const dsmoe_dims& d,
                const GateOut& out, hipStream_t st, float* part, const PtrChunk* tables, const void** tab_dst,
                const PermuteOut* po, bool* ranked) {
  if (ranked) *ranked = false;
  if (tables && (logits_in || !gate_uses_mfma(x, gw, d)))
    return fail(DSMOE_ERR_INVALID, "gate: a pointer table rides only with the MFMA gate");
  if (out.counts) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)cdiv(d.E, 256)), dim3(256), 0, st, out.counts, d.E, 0);
  }
  if (d.T == 0) return check_launch("gate(fill)");
  if (logits_in) return launch_route(logits_in, 1, bias, d, out, nullptr, nullptr, st);
  if (gate_mfma_ok(x, gw, d)) {
    switch (gate_nt(d.E)) {
      case 1: return launch_gate_mfma_nt<1>(x, gw, bias, d, out, part, tables, tab_dst, po, ranked, st);
      case 2: return launch_gate_mfma_nt<2>(x, gw, bias, d, out, part, tables, tab_dst, po, ranked, st);
      case 3: return launch_gate_mfma_nt<3>(x, gw, bias, d, out, part, tables, tab_dst, po, ranked, st);
      case 4: return launch_gate_mfma_nt<4>(x, gw, bias, d, out, part, tables, tab_dst, po, ranked, st);
      default: return launch_gate_mfma_nt<8>(x, gw, bias, d, out, part, tables, tab_dst, po, ranked, st);
    }
  }
  if (d.dtype == DSMOE_BF16) {
    if (d.E <= 16) return launch_gate_t<bf16_t, 16>(x, gw, bias, d, out, st);
    if (d.E <= 32) return launch_gate_t<bf16_t, 32>(x, gw, bias, d, out, st);
    return launch_gate_t<bf16_t, 64>(x, gw, bias, d, out, st);
  }
  if (d.E <= 16) return launch_gate_t<float, 16>(x, gw, bias, d, out, st);
  if (d.E <= 32) return launch_gate_t<float, 32>(x, gw, bias, d, out, st);
  return launch_gate_t<float, 64>(x, gw, bias, d, out, st);
}

void launch_fill_i32(int32_t* p, int n, int32_t v, hipStream_t st) {
  if (n > 0) hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, p, n, v);
}

}  // namespace dsmoe
