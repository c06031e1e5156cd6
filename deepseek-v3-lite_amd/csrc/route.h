// Token routing shared by the gate kernels and the small-call permute:
// sigmoid scores, bias, top-k selection, renormalised weights, histogram.
// Restates models/moe.py:32-36 (AuxLossFreeGate.forward after F.linear).
#pragma once

#include "common.h"

namespace dsmoe {

constexpr int MAX_EPL = 4;         // experts per lane in routing (E <= 256)

// Routes tokens [t0, t0 + ntok) whose fp32 logits sit in LDS rows lg[t*ldl].
// Wave w routes tokens in batches of route_ntok(EPL): w, w + nw, ... in batch
// units.  Lane l holds expert l (E <= 64) or
// experts l, l + 64, ... (E <= 256) in registers.
//
// Selection: k rounds of a wave arg-max over the biased scores under the
// order (value desc, id asc): a DPP max gives the round's value m, a ballot of
// the lanes holding m and its lowest set bit give the lowest expert id with
// that value, which takes slot j of the round and drops out.  This is the
// oracle's k rounds of arg-max with the same tie rule.  The renormalising sum
// runs over slots j = 0..k-1 in order, as in the oracle.
constexpr int route_ntok(int epl) { return epl == 1 ? 4 : 2; }

// Maximum over the 64 lanes (every lane gets it).  Row (16-lane) shifts, then
// the row broadcasts of lanes 15 and 31, leave the maximum in lane 63.
__device__ __forceinline__ float wave_max_f32(float v) {
  const int b = __float_as_int(v);
  float t;
  t = __int_as_float(__builtin_amdgcn_update_dpp(b, __float_as_int(v), 0x111, 0xf, 0xf, false));  // row_shr:1
  v = fmaxf(v, t);
  t = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x112, 0xf, 0xf, false));
  v = fmaxf(v, t);
  t = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x114, 0xf, 0xf, false));
  v = fmaxf(v, t);
  t = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x118, 0xf, 0xf, false));
  v = fmaxf(v, t);
  t = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x142, 0xa, 0xf, false));  // row_bcast:15
  v = fmaxf(v, t);
  t = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x143, 0xc, 0xf, false));  // row_bcast:31
  v = fmaxf(v, t);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// EPL: experts per lane (1 for E <= 64, MAX_EPL otherwise); NB: tokens a
// wave routes side by side (their sigmoid, max and ballot chains are
// independent, so their latencies overlap).
template <int EPL, int NB = route_ntok(EPL)>
__device__ __forceinline__ void route_tokens_t(const float* lg, int ldl, int ntok, int t0, const float* bias_s, int E,
                                               int k, float route_scale, int xdtype, const GateOut& out, int* hist) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  for (int tb = wave * NB; tb < ntok; tb += nw * NB) {
    float sv[NB][EPL], bv[NB][EPL];
    int slot[NB][EPL];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int q = 0; q < EPL; ++q) {
        const int e = lane + 64 * q;
        sv[b][q] = 0.0f;
        bv[b][q] = -INFINITY;
        slot[b][q] = -1;
        if (tb + b < ntok && e < E) {
          sv[b][q] = route_sigmoid(lg[(tb + b) * ldl + e]);
          bv[b][q] = sv[b][q] + bias_s[e];
        }
      }
    float ssum[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ssum[b] = 0.0f;
    for (int j = 0; j < k; ++j) {
      float m[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        float lm = bv[b][0];
#pragma unroll
        for (int q = 1; q < EPL; ++q) lm = fmaxf(lm, bv[b][q]);
        m[b] = wave_max_f32(lm);
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        int win = -1;
#pragma unroll
        for (int q = 0; q < EPL; ++q) {
          const uint64_t bl = __ballot(slot[b][q] < 0 && lane + 64 * q < E && bv[b][q] == m[b]);
          if (win < 0 && bl) win = __ffsll((unsigned long long)bl) - 1 + 64 * q;
        }
        if (win < 0) {
          // only NaN scores left: the lowest unselected expert id
#pragma unroll
          for (int q = 0; q < EPL; ++q) {
            const uint64_t bl = __ballot(slot[b][q] < 0 && lane + 64 * q < E);
            if (win < 0 && bl) win = __ffsll((unsigned long long)bl) - 1 + 64 * q;
          }
        }
        win = __builtin_amdgcn_readfirstlane(win);
        const int wl = win & 63, wq = win >> 6;
#pragma unroll
        for (int q = 0; q < EPL; ++q)
          if (q == wq) {
            ssum[b] += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sv[b][q]), wl));
            if (lane == wl) {
              slot[b][q] = j;
              bv[b][q] = -INFINITY;
            }
          }
      }
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if (tb + b >= ntok) break;   // padding tokens of the last batch write nothing
      const float den = ssum[b] < 1e-10f ? 1e-10f : ssum[b];
      const int64_t o = (int64_t)(t0 + tb + b) * k;
#pragma unroll
      for (int q = 0; q < EPL; ++q) {
        const int e = lane + 64 * q;
        if (slot[b][q] >= 0) {
          const int j = slot[b][q];
          const float w = sv[b][q] / den * route_scale;
          out.idx[o + j] = e;
          if (out.idx64) out.idx64[o + j] = e;
          out.weights[o + j] = w;
          if (out.weights_x) {
            if (xdtype == DSMOE_BF16)
              static_cast<bf16_t*>(out.weights_x)[o + j] = f2bf(w);
            else
              static_cast<float*>(out.weights_x)[o + j] = w;
          }
          if (out.sel_scores) out.sel_scores[o + j] = sv[b][q];
          if (hist) atomicAdd(&hist[e], 1);
        }
      }
    }
  }
}

template <int NB1 = route_ntok(1), int NB4 = route_ntok(MAX_EPL)>
__device__ __forceinline__ void route_tokens(const float* lg, int ldl, int ntok, int t0, const float* bias_s, int E,
                                             int k, float route_scale, int xdtype, const GateOut& out, int* hist) {
  if (E <= 64)
    route_tokens_t<1, NB1>(lg, ldl, ntok, t0, bias_s, E, k, route_scale, xdtype, out, hist);
  else
    route_tokens_t<MAX_EPL, NB4>(lg, ldl, ntok, t0, bias_s, E, k, route_scale, xdtype, out, hist);
}

__device__ __forceinline__ void flush_hist(const int* hist, int E, int32_t* counts) {
  if (!counts) return;
  for (int e = threadIdx.x; e < E; e += blockDim.x)
    if (hist[e]) atomicAdd(&counts[e], hist[e]);
}

}  // namespace dsmoe
