// (a) Fused gate: fp32 logits = x . W_gate^T, sigmoid, +bias, top-k,
// renormalisation, per-expert histogram.  Restates models/moe.py:29-37 and
// the bincount of models/moe.py:114 (see dsmoe.h for the tie rule).
#include "common.h"

namespace dsmoe {

constexpr int GATE_THREADS = 256;
constexpr int GATE_KC = 32;   // K chunk staged through LDS

// Top-k over one token's row of scores held in LDS.  Ties -> lower expert id.
__device__ __forceinline__ void topk_row(const float* sc, const float* bias_s, int E, int k, float* topv, int* topi) {
  int n = 0;
  for (int e = 0; e < E; ++e) {
    float b = sc[e] + bias_s[e];
    int pos = n;
    while (pos > 0 && topv[pos - 1] < b) --pos;
    if (pos >= k) continue;
    int last = n < k ? n : k - 1;
    for (int q = last; q > pos; --q) {
      topv[q] = topv[q - 1];
      topi[q] = topi[q - 1];
    }
    topv[pos] = b;
    topi[pos] = e;
    if (n < k) ++n;
  }
}

// LDS layout (floats): xs[KC][TB+4] | ws[KC][EC+4] | lg[TB][E+1] | bias[E] | hist[E] (int)
template <typename XT, int EC, bool FROM_LOGITS>
__global__ __launch_bounds__(GATE_THREADS) void gate_kernel(const XT* __restrict__ x, const float* __restrict__ logits_in,
                                                            const float* __restrict__ gw, const float* __restrict__ bias,
                                                            int T, int D, int E, int k, float route_scale, GateOut out) {
  constexpr int TX = EC / 4;                // threads along experts
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
          float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
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
  if (!FROM_LOGITS && out.logits) {
    for (int i = tid; i < TB * E; i += GATE_THREADS) {
      int t = i / E, e = i - t * E;
      if (t0 + t < T) out.logits[(int64_t)(t0 + t) * E + e] = lg[t * ldl + e];
    }
  }
  for (int i = tid; i < TB * E; i += GATE_THREADS) {
    int t = i / E, e = i - t * E;
    lg[t * ldl + e] = route_sigmoid(lg[t * ldl + e]);
  }
  __syncthreads();
  for (int t = tid; t < TB; t += GATE_THREADS) {
    if (t0 + t >= T) break;
    float topv[MAX_TOPK];
    int topi[MAX_TOPK];
    const float* row = lg + t * ldl;
    topk_row(row, bias_s, E, k, topv, topi);
    float sel[MAX_TOPK];
    float ssum = 0.0f;
    for (int j = 0; j < k; ++j) {
      sel[j] = row[topi[j]];
      ssum += sel[j];
    }
    const float den = ssum < 1e-10f ? 1e-10f : ssum;
    const int64_t o = (int64_t)(t0 + t) * k;
    for (int j = 0; j < k; ++j) {
      float w = sel[j] / den * route_scale;
      out.idx[o + j] = topi[j];
      if (out.idx64) out.idx64[o + j] = topi[j];
      out.weights[o + j] = w;
      if (out.weights_x) static_cast<XT*>(out.weights_x)[o + j] = from_f<XT>(w);
      if (out.sel_scores) out.sel_scores[o + j] = sel[j];
      atomicAdd(&hist[topi[j]], 1);
    }
  }
  __syncthreads();
  if (out.counts) {
    for (int e = tid; e < E; e += GATE_THREADS)
      if (hist[e]) atomicAdd(&out.counts[e], hist[e]);
  }
}

__global__ void fill_i32_kernel(int32_t* p, int n, int32_t v) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

template <typename XT, int EC, bool FROM_LOGITS>
static int launch_gate_t(const void* x, const float* logits_in, const float* gw, const float* bias, const dsmoe_dims& d,
                         const GateOut& out, hipStream_t st) {
  constexpr int TX = EC / 4;
  constexpr int TB = (GATE_THREADS / TX) * 4;
  size_t lds = sizeof(float) * (GATE_KC * (TB + 4) + GATE_KC * (EC + 4) + TB * (d.E + 1) + d.E) + sizeof(int) * d.E;
  auto kern = gate_kernel<XT, EC, FROM_LOGITS>;
  if (lds > 64 * 1024) {
    if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return fail(DSMOE_ERR_HIP, "gate: cannot raise LDS limit");
  }
  int blocks = (int)cdiv(d.T, TB);
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(GATE_THREADS), lds, st, static_cast<const XT*>(x), logits_in, gw, bias,
                     d.T, d.D, d.E, d.k, d.route_scale, out);
  return check_launch("gate");
}

int launch_gate(const void* x, const float* logits_in, const float* gw, const float* bias, const dsmoe_dims& d,
                const GateOut& out, hipStream_t st) {
  if (out.counts) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3((unsigned)cdiv(d.E, 256)), dim3(256), 0, st, out.counts, d.E, 0);
  }
  if (d.T == 0) return check_launch("gate(fill)");
  const bool fl = logits_in != nullptr;
  if (fl) {
    if (d.dtype == DSMOE_BF16) return launch_gate_t<bf16_t, 64, true>(nullptr, logits_in, gw, bias, d, out, st);
    return launch_gate_t<float, 64, true>(nullptr, logits_in, gw, bias, d, out, st);
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
