// (a) Fused gate: fp32 logits = x . W_gate^T, sigmoid, +bias, top-k,
// renormalisation, per-expert histogram.  Restates models/moe.py:29-37 and
// the bincount of models/moe.py:114 (see dsmoe.h for the tie rule).
//
// Logits.  bf16 x: MFMA.  Each fp32 gate weight is split exactly into three
// bf16 parts by truncation (w = hi + mid + lo: hi keeps the top 8 significand
// bits, mid the next 8, lo the last 8), so x.w = x.hi + x.mid + x.lo with
// every product exact; the MFMA accumulates in fp32.  A block takes 32 tokens
// and all experts; its 4 waves split D in quarters and the four partial sums
// are added in a fixed order, so the result is deterministic.  fp32 x: SIMT
// FMA tiles.
//
// Routing.  One wave per token, one lane per expert (E <= 64; E <= 256 with
// several experts per lane): sigmoid in double rounded once, + bias, then k
// rounds of a wave-wide arg-max ordered by (value desc, expert id asc).
#include <cstdlib>

#include "route.h"

namespace dsmoe {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 g_bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float g_f32x16_t;
typedef float g_f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int g_u32x4_t __attribute__((ext_vector_type(4)));

constexpr int GATE_THREADS = 256;
// MFMA gate: 4 waves when one 32-expert tile covers E, else 8 (the second four
// take the odd expert tiles of the same K quarters)
constexpr int gm_waves(int nt) { return nt >= 2 ? 8 : 4; }
constexpr int GATE_KC = 32;        // SIMT: K chunk staged through LDS
constexpr int GM_TOK = 32;         // MFMA: tokens per block

// ------------------------------------------------------------------ MFMA logits (bf16 x)
// Splits 8 consecutive fp32 weights into three bf16x8 vectors whose sum is exact.
__device__ __forceinline__ void split3(const g_f32x4_t& a, const g_f32x4_t& b, g_bf16x8_t& hi, g_bf16x8_t& mid,
                                       g_bf16x8_t& lo) {
  const float w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  unsigned short h[8], m[8], l[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t wb = __float_as_uint(w[i]);
    const float fh = __uint_as_float(wb & 0xffff0000u);
    const float r1 = w[i] - fh;                       // exact
    const uint32_t rb = __float_as_uint(r1);
    const float fm = __uint_as_float(rb & 0xffff0000u);
    const float r2 = r1 - fm;                         // exact, <= 8 significant bits
    h[i] = (unsigned short)(wb >> 16);
    m[i] = (unsigned short)(rb >> 16);
    l[i] = (unsigned short)(__float_as_uint(r2) >> 16);
  }
  __builtin_memcpy(&hi, h, 16);
  __builtin_memcpy(&mid, m, 16);
  __builtin_memcpy(&lo, l, 16);
}


// LDS: part[4][GM_TOK][EP+1] fp32 partial logits (reused for the reduced
// logits), bias[E], hist[E], routing scratch.
template <int NT>
__global__ __launch_bounds__(gm_waves(NT) * 64) void gate_mfma_kernel(const bf16_t* __restrict__ x,
                                                                 const float* __restrict__ gw,
                                                                 const float* __restrict__ bias, int T, int D, int E,
                                                                 int k, float route_scale, GateOut out,
                                                                 float* __restrict__ part_out, int ks,
                                                                 const PtrChunk tables, const void** tab_dst) {
  constexpr int EP = NT * 32;
  constexpr int LDP = EP + 1;
  extern __shared__ float gsm[];
  float* part = gsm;                                   // [4][GM_TOK][LDP]
  float* bias_s = part + 4 * GM_TOK * LDP;
  int* hist = reinterpret_cast<int*>(bias_s + E);
  constexpr int NWV = gm_waves(NT);
  constexpr int NTH = NWV * 64;
  // wave w: K quarter w & 3; expert tiles ni = w >> 2, w >> 2 + NWV / 4, ...
  constexpr int TSTEP = NWV / 4;
  constexpr int NTW = (NT + TSTEP - 1) / TSTEP;       // expert tiles per wave (upper bound)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int quarter = wave & 3, tfirst = wave >> 2;
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < tables.n; i += blockDim.x) tab_dst[tables.off + i] = tables.p[i];
  // K split (part_out != nullptr): block b takes token tile b / ks and the
  // K range of split b % ks, and writes partial logits instead of routing.
  const int split = part_out ? (int)(blockIdx.x % ks) : 0;
  const int t0 = (part_out ? (int)(blockIdx.x / ks) : (int)blockIdx.x) * GM_TOK;
  for (int e = tid; e < E; e += NTH) {
    bias_s[e] = bias[e];
    hist[e] = 0;
  }
  const int dk = part_out ? D / ks : D;
  const int kq = dk / 4;
  const int kbeg = split * dk + quarter * kq;
  const int m = lane & 31;
  const int row = min(t0 + m, T - 1);
  const bf16_t* xr = x + (int64_t)row * D + (lane >> 5) * 8;
  const float* wr[NTW];
#pragma unroll
  for (int i = 0; i < NTW; ++i) {
    const int ni = min(tfirst + i * TSTEP, NT - 1);
    wr[i] = gw + (int64_t)min(ni * 32 + m, E - 1) * D + (lane >> 5) * 8;
  }
  const int ntw = min(NTW, (NT - tfirst + TSTEP - 1) / TSTEP);   // this wave's tiles

  g_f32x16_t acc[NTW];
#pragma unroll
  for (int i = 0; i < NTW; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;

  // K loop in chunks of PF steps of 16, double-buffered: the loads of chunk
  // c + 1 are issued before the MFMAs of chunk c, so the global round trips
  // overlap the split and MFMA work (the loop is latency-bound otherwise:
  // every block streams all of W_gate).
  constexpr int PF = (NTW <= 2) ? 4 : 2;
  const int kend = kbeg + kq;
  g_bf16x8_t a[2][PF];
  g_f32x4_t w0[2][PF][NTW], w1[2][PF][NTW];
  auto load = [&](int buf, int k0) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const int kk = min(k0 + 16 * p, kend - 16);
      a[buf][p] = *reinterpret_cast<const g_bf16x8_t*>(xr + kk);
#pragma unroll
      for (int ni = 0; ni < NTW; ++ni) {
        w0[buf][p][ni] = *reinterpret_cast<const g_f32x4_t*>(wr[ni] + kk);
        w1[buf][p][ni] = *reinterpret_cast<const g_f32x4_t*>(wr[ni] + kk + 4);
      }
    }
  };
  auto compute = [&](int buf, int k0) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      if (k0 + 16 * p >= kend) break;
#pragma unroll
      for (int ni = 0; ni < NTW; ++ni) {
        if (ni >= ntw) break;
        g_bf16x8_t hi, mid, lo;
        split3(w0[buf][p][ni], w1[buf][p][ni], hi, mid, lo);
        acc[ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(lo, a[buf][p], acc[ni], 0, 0, 0);
        acc[ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(mid, a[buf][p], acc[ni], 0, 0, 0);
        acc[ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hi, a[buf][p], acc[ni], 0, 0, 0);
      }
    }
  };
  constexpr int CH = 16 * PF;
  load(0, kbeg);
  for (int k0 = kbeg; k0 < kend; k0 += 2 * CH) {
    if (k0 + CH < kend) load(1, k0 + CH);
    compute(0, k0);
    if (k0 + CH >= kend) break;
    if (k0 + 2 * CH < kend) load(0, k0 + 2 * CH);
    compute(1, k0 + CH);
  }
  // lane holds token m, experts ni*32 + 8*(r/4) + 4*(lane/32) + r%4
  float* pw = part + quarter * GM_TOK * LDP + m * LDP;
#pragma unroll
  for (int i = 0; i < NTW; ++i) {
    if (i >= ntw) break;
    const int ni = tfirst + i * TSTEP;
#pragma unroll
    for (int r = 0; r < 16; ++r) pw[ni * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)] = acc[i][r];
  }
  __syncthreads();
  const int ntok = min(GM_TOK, T - t0);
  for (int i = tid; i < GM_TOK * E; i += NTH) {
    const int t = i / E, e = i - t * E;
    const int o = t * LDP + e;
    const float v = ((part[o] + part[GM_TOK * LDP + o]) + part[2 * GM_TOK * LDP + o]) + part[3 * GM_TOK * LDP + o];
    part[o] = v;
    if (part_out) {
      if (t < ntok) part_out[((int64_t)split * T + t0 + t) * E + e] = v;
    } else if (out.logits && t < ntok) {
      out.logits[(int64_t)(t0 + t) * E + e] = v;
    }
  }
  if (part_out) return;
  __syncthreads();
  route_tokens(part, LDP, ntok, t0, bias_s, E, k, route_scale, DSMOE_BF16, out, out.counts ? hist : nullptr);
  __syncthreads();
  flush_hist(hist, E, out.counts);
}

// ------------------------------------------------------------------ SIMT logits (fp32 x) / given logits
// LDS layout (floats): xs[KC][TB+4] | ws[KC][EC+4] | lg[TB][E+1] | bias[E] | hist[E] (int) | routing scratch
template <typename XT, int EC, bool FROM_LOGITS>
__global__ __launch_bounds__(GATE_THREADS) void gate_kernel(const XT* __restrict__ x, const float* __restrict__ logits_in,
                                                            const float* __restrict__ gw, const float* __restrict__ bias,
                                                            int T, int D, int E, int k, float route_scale, int xdtype,
                                                            GateOut out) {
  constexpr int TX = EC / 4;                   // threads along experts
  constexpr int TB = (GATE_THREADS / TX) * 4;  // tokens per block
  extern __shared__ float smem[];
  float* xs = smem;                             // [KC][TB+4]
  float* ws = xs + GATE_KC * (TB + 4);          // [KC][EC+4]
  float* lg = ws + GATE_KC * (EC + 4);          // [TB][E+1]
  float* bias_s = lg + TB * (E + 1);            // [E]
  int* hist = reinterpret_cast<int*>(bias_s + E);  // [E]

  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * TB;
  const int ldl = E + 1;
  for (int e = tid; e < E; e += GATE_THREADS) {
    bias_s[e] = bias[e];
    hist[e] = 0;
  }

  if constexpr (FROM_LOGITS) {
    for (int i = tid; i < TB * E; i += GATE_THREADS) {
      int t = i / E, e = i - t * E;
      lg[t * ldl + e] = (t0 + t < T) ? logits_in[(int64_t)(t0 + t) * E + e] : 0.0f;
    }
  } else {
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
  }
  __syncthreads();
  const int ntok = min(TB, T - t0);
  if (!FROM_LOGITS && out.logits) {
    for (int i = tid; i < ntok * E; i += GATE_THREADS) {
      int t = i / E, e = i - t * E;
      out.logits[(int64_t)(t0 + t) * E + e] = lg[t * ldl + e];
    }
  }
  route_tokens(lg, ldl, ntok, t0, bias_s, E, k, route_scale, xdtype, out, out.counts ? hist : nullptr);
  __syncthreads();
  flush_hist(hist, E, out.counts);
}

__global__ void fill_i32_kernel(int32_t* p, int n, int32_t v) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// Routing after a K-split gate: logits = sum of the ks partial logits in
// split order (0, 1, ...), optionally written out, then route_tokens.
constexpr int RP_TOK = 1;        // tokens per block (one wave): small calls, spread over the CUs
__global__ __launch_bounds__(64) void route_partials_kernel(const float* __restrict__ part, int ks,
                                                             const float* __restrict__ bias, int T, int E, int k,
                                                             float route_scale, int xdtype, GateOut out) {
  extern __shared__ float rsm[];
  const int ldl = E + 1;
  float* lg = rsm;                               // [RP_TOK][E + 1]
  float* bias_s = lg + RP_TOK * ldl;             // [E]
  int* hist = reinterpret_cast<int*>(bias_s + E);
  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * RP_TOK;
  const int ntok = min(RP_TOK, T - t0);
  for (int e = tid; e < E; e += blockDim.x) {
    bias_s[e] = bias[e];
    hist[e] = 0;
  }
  for (int i = tid; i < ntok * E; i += blockDim.x) {
    const int t = i / E, e = i - t * E;
    const float* p = part + (int64_t)(t0 + t) * E + e;
    // every split's load is issued before the adds (one memory latency)
    float pv[GATE_KS_MAX];
#pragma unroll
    for (int sp = 0; sp < GATE_KS_MAX; ++sp) pv[sp] = sp < ks ? p[(int64_t)sp * T * E] : 0.0f;
    float v = pv[0];
#pragma unroll
    for (int sp = 1; sp < GATE_KS_MAX; ++sp)
      if (sp < ks) v += pv[sp];
    lg[t * ldl + e] = v;
    if (out.logits) out.logits[(int64_t)(t0 + t) * E + e] = v;
  }
  __syncthreads();
  route_tokens<1, 1>(lg, ldl, ntok, t0, bias_s, E, k, route_scale, xdtype, out, out.counts ? hist : nullptr);
  __syncthreads();
  flush_hist(hist, E, out.counts);
}

static int set_lds(const void* kern, size_t lds) {
  if (lds > 64 * 1024 &&
      hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
    return fail(DSMOE_ERR_HIP, "gate: cannot raise LDS limit");
  return DSMOE_OK;
}

template <typename XT, int EC, bool FROM_LOGITS>
static int launch_gate_t(const void* x, const float* logits_in, const float* gw, const float* bias, const dsmoe_dims& d,
                         const GateOut& out, hipStream_t st) {
  constexpr int TX = EC / 4;
  constexpr int TB = (GATE_THREADS / TX) * 4;
  const size_t lds = sizeof(float) * (GATE_KC * (TB + 4) + GATE_KC * (EC + 4) + TB * (d.E + 1) + d.E) +
                     sizeof(int) * d.E + 16;
  auto kern = gate_kernel<XT, EC, FROM_LOGITS>;
  int rc = set_lds((const void*)kern, lds);
  if (rc) return rc;
  int blocks = (int)cdiv(d.T, TB);
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(GATE_THREADS), lds, st, static_cast<const XT*>(x), logits_in, gw, bias,
                     d.T, d.D, d.E, d.k, d.route_scale, d.dtype, out);
  return check_launch("gate");
}

template <int NT>
static int launch_gate_mfma(const void* x, const float* gw, const float* bias, const dsmoe_dims& d, const GateOut& out,
                            float* part, int ks, hipStream_t st, const PtrChunk* tables, const void** tab_dst) {
  PtrChunk none;
  none.n = 0;
  none.off = 0;
  const size_t lds = sizeof(float) * (4 * GM_TOK * (NT * 32 + 1) + d.E) + sizeof(int) * ((d.E + 3) & ~3);
  auto kern = gate_mfma_kernel<NT>;
  int rc = set_lds((const void*)kern, lds);
  if (rc) return rc;
  const int64_t blocks = cdiv(d.T, GM_TOK) * (part ? ks : 1);
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(gm_waves(NT) * 64), lds, st, static_cast<const bf16_t*>(x), gw,
                     bias, d.T, d.D, d.E, d.k, d.route_scale, out, part, ks, tables ? *tables : none, tab_dst);
  rc = check_launch("gate_mfma");
  if (rc || !part) return rc;
  const size_t rlds = sizeof(float) * (RP_TOK * (d.E + 1) + d.E) + sizeof(int) * d.E;
  hipLaunchKernelGGL(route_partials_kernel, dim3((unsigned)cdiv(d.T, RP_TOK)), dim3(64), rlds, st, part, ks, bias,
                     d.T, d.E, d.k, d.route_scale, (int)DSMOE_BF16, out);
  return check_launch("route_partials");
}

int gate_k_splits(const dsmoe_dims& d) {
  const int64_t tiles = cdiv(d.T, GM_TOK);
  int ks = 1;
  while (ks < GATE_KS_MAX && tiles * ks * 2 <= 256) ks *= 2;   // fill the 256 CUs when there are few token tiles
  while (ks > 1 && d.D % (64 * ks) != 0) ks >>= 1;
  return ks;
}

size_t gate_part_floats(const dsmoe_dims& d) {
  const int ks = gate_k_splits(d);
  return ks > 1 ? (size_t)ks * d.T * d.E : 0;
}

static bool gate_mfma_ok(const void* x, const float* gw, const dsmoe_dims& d) {
  return d.dtype == DSMOE_BF16 && d.D % 64 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
         (reinterpret_cast<uintptr_t>(gw) & 15) == 0;
}

bool gate_uses_mfma(const void* x, const float* gw, const dsmoe_dims& d) { return d.T > 0 && gate_mfma_ok(x, gw, d); }

int launch_gate(const void* x, const float* logits_in, const float* gw, const float* bias, const dsmoe_dims& d,
                const GateOut& out, hipStream_t st, float* part, const PtrChunk* tables, const void** tab_dst) {
  if (tables && (logits_in || !gate_uses_mfma(x, gw, d)))
    return fail(DSMOE_ERR_INVALID, "gate: a pointer table rides only with the MFMA gate");
  if (out.counts) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)cdiv(d.E, 256)), dim3(256), 0, st, out.counts, d.E, 0);
  }
  if (d.T == 0) return check_launch("gate(fill)");
  if (logits_in) return launch_gate_t<float, 64, true>(nullptr, logits_in, gw, bias, d, out, st);
  const bool mfma = gate_mfma_ok(x, gw, d);
  if (mfma) {
    const int nt = (int)cdiv(d.E, 32);
    const int ks = part ? gate_k_splits(d) : 1;
    float* pp = ks > 1 ? part : nullptr;
    switch (nt) {
      case 1: return launch_gate_mfma<1>(x, gw, bias, d, out, pp, ks, st, tables, tab_dst);
      case 2: return launch_gate_mfma<2>(x, gw, bias, d, out, pp, ks, st, tables, tab_dst);
      case 3: return launch_gate_mfma<3>(x, gw, bias, d, out, pp, ks, st, tables, tab_dst);
      case 4: return launch_gate_mfma<4>(x, gw, bias, d, out, pp, ks, st, tables, tab_dst);
      default: return launch_gate_mfma<8>(x, gw, bias, d, out, pp, ks, st, tables, tab_dst);
    }
  }
  if (d.dtype == DSMOE_BF16) {
    if (d.E <= 16) return launch_gate_t<bf16_t, 16, false>(x, nullptr, gw, bias, d, out, st);
    if (d.E <= 32) return launch_gate_t<bf16_t, 32, false>(x, nullptr, gw, bias, d, out, st);
    return launch_gate_t<bf16_t, 64, false>(x, nullptr, gw, bias, d, out, st);
  }
  if (d.E <= 16) return launch_gate_t<float, 16, false>(x, nullptr, gw, bias, d, out, st);
  if (d.E <= 32) return launch_gate_t<float, 32, false>(x, nullptr, gw, bias, d, out, st);
  return launch_gate_t<float, 64, false>(x, nullptr, gw, bias, d, out, st);
}

void launch_fill_i32(int32_t* p, int n, int32_t v, hipStream_t st) {
  if (n > 0) hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, st, p, n, v);
}

}  // namespace dsmoe
