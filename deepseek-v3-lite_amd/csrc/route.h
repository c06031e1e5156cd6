// Token routing shared by the gate kernels and the small-call permute:
// sigmoid scores, bias, top-k selection, renormalised weights, histogram.
// Restates models/moe.py:32-36 (AuxLossFreeGate.forward after F.linear).
#pragma once

#include <stdint.h>

#include "common.h"

namespace dsmoe {

constexpr int MAX_EPL = 4;         // experts per lane in routing (E <= 256)

// Routes tokens [t0, t0 + ntok) whose fp32 logits sit in LDS rows lg[t*ldl].
// Wave w routes tokens in batches of NB: w, w + nw, ... in batch units.  Lane
// l holds expert l (E <= 64) or experts l, l + 64, ... (E <= 256) in
// registers.
//
// Selection: k rounds of a wave arg-max over the biased scores under the
// order (value desc, id asc).  Each score is held as an integer key with the
// same order (route_key), so a round is one integer DPP max (the round's key
// m) and a ballot of the lanes holding m, whose lowest set bit gives the
// lowest expert id with that key; that expert takes slot j and its key drops
// to INT32_MIN.  This is the oracle's k rounds of arg-max with the same tie
// rule.  The renormalising sum runs over slots j = 0..k-1 in order, as in
// the oracle.
constexpr int route_ntok(int epl) { return epl == 1 ? 4 : 2; }

// Order key of a biased score: a signed integer ordered like the score, with
// -0 folded into +0 (they compare equal) and NaN below every number (a NaN
// score is taken only when no number is left, lowest id first).  INT32_MIN
// marks lanes without an expert or already selected.
__device__ __forceinline__ int32_t route_key(float f) {
  int32_t b = __float_as_int(f);
  if (f != f) return INT32_MIN + 1;
  if (b == INT32_MIN) b = 0;
  return b >= 0 ? b : b ^ 0x7fffffff;
}

// Maximum over the 64 lanes (every lane gets it).  Row (16-lane) shifts, then
// the row broadcasts of lanes 15 and 31, leave the maximum in lane 63.
__device__ __forceinline__ int32_t wave_max_i32(int32_t v) {
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x111, 0xf, 0xf, false));  // row_shr:1
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x112, 0xf, 0xf, false));  // row_shr:2
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x114, 0xf, 0xf, false));  // row_shr:4
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x118, 0xf, 0xf, false));  // row_shr:8
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xa, 0xf, false));  // row_bcast:15
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return __builtin_amdgcn_readlane(v, 63);
}

// EPL: experts per lane (1 for E <= 64, MAX_EPL otherwise); NB: tokens a
// wave routes side by side (their sigmoid, max and ballot chains are
// independent, so their latencies overlap).
// sel (optional, LDS): sel[t * k + j] = the expert of slot j of token t0 + t.
template <int EPL, int NB = route_ntok(EPL)>
__device__ __forceinline__ void route_tokens_t(const float* lg, int ldl, int ntok, int t0, const float* bias_s, int E,
                                               int k, float route_scale, int xdtype, const GateOut& out, int* hist,
                                               int32_t* sel = nullptr) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  for (int tb = wave * NB; tb < ntok; tb += nw * NB) {
    float sv[NB][EPL];
    int32_t key[NB][EPL];
    int slot[NB][EPL];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int q = 0; q < EPL; ++q) {
        const int e = lane + 64 * q;
        sv[b][q] = 0.0f;
        key[b][q] = INT32_MIN;
        slot[b][q] = -1;
        if (tb + b < ntok && e < E) {
          sv[b][q] = route_sigmoid(lg[(tb + b) * ldl + e]);
          key[b][q] = route_key(sv[b][q] + bias_s[e]);
        }
      }
    float ssum[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) ssum[b] = 0.0f;
    for (int j = 0; j < k; ++j) {
      int32_t m[NB];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        int32_t lm = key[b][0];
#pragma unroll
        for (int q = 1; q < EPL; ++q) lm = max(lm, key[b][q]);
        m[b] = wave_max_i32(lm);
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        // the lowest expert id holding the round's key (a token past ntok
        // has no expert: its rounds pick lane 0 and write nothing)
        int win = -1;
#pragma unroll
        for (int q = 0; q < EPL; ++q) {
          const uint64_t bl = __ballot(key[b][q] == m[b]);
          if (win < 0 && bl) win = __ffsll((unsigned long long)bl) - 1 + 64 * q;
        }
        win = __builtin_amdgcn_readfirstlane(win);
        const int wl = win & 63, wq = win >> 6;
#pragma unroll
        for (int q = 0; q < EPL; ++q)
          if (q == wq) {
            ssum[b] += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sv[b][q]), wl));
            if (lane == wl) {
              slot[b][q] = j;
              key[b][q] = INT32_MIN;
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
          if (sel) sel[(tb + b) * k + j] = e;
        }
      }
    }
  }
}

// Maxima / minima over each 16-lane row of a wave (every lane gets its row's):
// rotations by 1, 2, 4, 8 within the row.
__device__ __forceinline__ int32_t row_max_i32(int32_t v) {
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x121, 0xf, 0xf, false));  // row_ror:1
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x122, 0xf, 0xf, false));  // row_ror:2
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x124, 0xf, 0xf, false));  // row_ror:4
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x128, 0xf, 0xf, false));  // row_ror:8
  return v;
}
__device__ __forceinline__ int32_t row_min_i32(int32_t v) {
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x121, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x122, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x124, 0xf, 0xf, false));
  v = min(v, __builtin_amdgcn_update_dpp(v, v, 0x128, 0xf, 0xf, false));
  return v;
}

// Writes slot j of token t0 + t (local index t): expert e, unbiased score sv,
// renormalising sum den.
__device__ __forceinline__ void route_emit(const GateOut& out, int t0, int t, int k, int j, int e, float sv, float den,
                                          float route_scale, int xdtype, int* hist, int32_t* sel) {
  const int64_t o = (int64_t)(t0 + t) * k + j;
  const float w = sv / den * route_scale;
  out.idx[o] = e;
  if (out.idx64) out.idx64[o] = e;
  out.weights[o] = w;
  if (out.weights_x) {
    if (xdtype == DSMOE_BF16)
      static_cast<bf16_t*>(out.weights_x)[o] = f2bf(w);
    else
      static_cast<float*>(out.weights_x)[o] = w;
  }
  if (out.sel_scores) out.sel_scores[o] = sv;
  if (hist) atomicAdd(&hist[e], 1);
  if (sel) sel[t * k + j] = e;
}

// Row (16-lane) sum, every lane gets its row's: rotations by 1, 2, 4, 8.
__device__ __forceinline__ int32_t row_sum_i32(int32_t v) {
  v += __builtin_amdgcn_update_dpp(v, v, 0x121, 0xf, 0xf, false);  // row_ror:1
  v += __builtin_amdgcn_update_dpp(v, v, 0x122, 0xf, 0xf, false);  // row_ror:2
  v += __builtin_amdgcn_update_dpp(v, v, 0x124, 0xf, 0xf, false);  // row_ror:4
  v += __builtin_amdgcn_update_dpp(v, v, 0x128, 0xf, 0xf, false);  // row_ror:8
  return v;
}

// Routing of E <= 64 experts with four tokens per wave: row r (16 lanes) holds
// token tb + r, lane c of the row experts c, c + 16, c + 32, c + 48.
//
// Exact rounds (route_batch_exact): the scores are the double-evaluated
// sigmoid; a round is a row max of the keys, a row min of the lowest expert id
// holding it (the tie rule), and a permute that hands the winner's unbiased
// score to the row for the renormalising sum (slot order, as in the oracle).
// Only the rows with `live` set write.
__device__ __forceinline__ void route_batch_exact(const float* lg, int ldl, int t, bool live, int t0,
                                                  const float* bias_s, int E, int k, float route_scale, int xdtype,
                                                  const GateOut& out, int* hist, int32_t* sel) {
  const int lane = threadIdx.x & 63;
  const int r = lane >> 4, c = lane & 15;
  float sv[4];
  int32_t key[4];
  int slot[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = c + 16 * q;
    sv[q] = 0.0f;
    key[q] = INT32_MIN;
    slot[q] = -1;
    if (live && e < E) {
      sv[q] = route_sigmoid(lg[t * ldl + e]);
      key[q] = route_key(sv[q] + bias_s[e]);
    }
  }
  float ssum = 0.0f;
  for (int j = 0; j < k; ++j) {
    const int32_t m = row_max_i32(max(max(key[0], key[1]), max(key[2], key[3])));
    int32_t cand = 255;
#pragma unroll
    for (int q = 3; q >= 0; --q)
      if (key[q] == m) cand = c + 16 * q;
    // a row without a live token has only INT32_MIN keys: its rounds pick
    // expert 0 and write nothing
    const int32_t win = row_min_i32(cand);
    const int wq = win >> 4;
    float wsv = sv[0];
#pragma unroll
    for (int q = 1; q < 4; ++q)
      if (q == wq) wsv = sv[q];
    ssum += __int_as_float(__builtin_amdgcn_ds_bpermute((r * 16 + (win & 15)) << 2, __float_as_int(wsv)));
    if (c == (win & 15)) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (q == wq) {
          slot[q] = j;
          key[q] = INT32_MIN;
        }
    }
  }
  if (!live) return;
  const float den = ssum < 1e-10f ? 1e-10f : ssum;
#pragma unroll
  for (int q = 0; q < 4; ++q)
    if (slot[q] >= 0) route_emit(out, t0, t, k, slot[q], c + 16 * q, sv[q], den, route_scale, xdtype, hist, sel);
}

// Screened rounds (route_batch_fast).  The exact score needs a
// double-precision exp and divide per expert; the selection only needs the
// order of the biased scores.  So the rounds run on a single-precision
// estimate sa = rcp(1 + exp2(-x log2 e)) (hardware exp2 and reciprocal, each
// within 1 ulp), whose error against the exact score is at most
// s(1-s)(|x|+1) 2^-23 + 1.5 s 2^-23 < 2^-22; ROUTE_SCREEN_DS takes twice that.
// Each biased estimate fl(sa + bias) is then within ROUTE_SCREEN_DS + 1 ulp of
// the exact biased score fl(s + bias).  The estimate keys are sorted within
// each lane (four per lane), and k + 1 rounds of a row max pick the k + 1
// largest; the winner of round j advances its list and records its expert.
// The result is the exact one when every pair of neighbouring round maxima
// m_j > m_{j+1} (j < k) is separated by more than twice that error bound: then
// the exact scores keep the same strict order among the k selected and stay
// strictly above every expert not selected, so neither the set, nor the slot
// order, nor the tie rule can differ.  A row passes when that holds, when
// every round had exactly one winner (no two equal estimates taken at once)
// and every estimate is finite; its k selected experts then get their exact
// scores (one double sigmoid per lane) for the weights.  Rows that fail are
// routed by the exact rounds.  `scr` is this wave's 64 ints of LDS.
constexpr float ROUTE_SCREEN_DS = 4.76837158203125e-7f;   // 2^-21
constexpr float ROUTE_ULP = 1.1920928955078125e-7f;       // 2^-23

__device__ __forceinline__ int32_t mono_key(float f) {
  const int32_t b = __float_as_int(f);
  return b ^ ((b >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float mono_val(int32_t v) { return __int_as_float(v ^ ((v >> 31) & 0x7fffffff)); }

template <int KR>
__device__ __forceinline__ void route_batch_fast(const float* lg, int ldl, int t, bool live, int t0,
                                                 const float* bias_s, const float (&bq)[4], int E, int k,
                                                 float route_scale, int xdtype, const GateOut& out, int* hist,
                                                 int32_t* sel, int32_t* scr) {
  const int lane = threadIdx.x & 63;
  const int r = lane >> 4, c = lane & 15;
  int32_t key[4];
  int id[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = c + 16 * q;
    key[q] = INT32_MIN;
    id[q] = e;
    if (live && e < E) {
      const float ea = __builtin_amdgcn_exp2f(lg[t * ldl + e] * -1.4426950408889634f);
      const float ka = __builtin_amdgcn_rcpf(1.0f + ea) + bq[q];
      // a non-finite estimate wins its row's first round and fails the margin
      key[q] = __builtin_isfinite(ka) ? mono_key(ka) : INT32_MAX;
    }
  }
  auto cx = [&](int a, int b) {
    if (key[b] > key[a]) {
      const int32_t tk = key[a];
      key[a] = key[b];
      key[b] = tk;
      const int ti = id[a];
      id[a] = id[b];
      id[b] = ti;
    }
  };
  cx(0, 1);
  cx(2, 3);
  cx(0, 2);
  cx(1, 3);
  cx(1, 2);
  int32_t mc = INT32_MIN, mc1 = INT32_MIN;   // lane c: round maxima m_c, m_{c+1}
  int nadv = 0, nround = 0;
#pragma unroll
  for (int j = 0; j < KR; ++j) {
    if (j <= k) {
      const int32_t m = row_max_i32(key[0]);
      if (c == j) mc = m;
      if (c + 1 == j) mc1 = m;
      if (m != INT32_MIN) {
        ++nround;
        if (key[0] == m) {
          scr[r * 16 + j] = id[0];
          key[0] = key[1];
          key[1] = key[2];
          key[2] = key[3];
          key[3] = INT32_MIN;
          id[0] = id[1];
          id[1] = id[2];
          id[2] = id[3];
          ++nadv;
        }
      }
    }
  }
  bool good = true;
  if (c < k) {
    if (mc == INT32_MIN || mc == INT32_MAX) {
      good = false;
    } else if (mc1 != INT32_MIN) {
      const float k1 = mono_val(mc), k2 = mono_val(mc1);
      const float th = fmaxf(fabsf(k1), fabsf(k2));
      good = k1 - k2 > 2.0f * (ROUTE_SCREEN_DS + th * ROUTE_ULP);
    }
  }
  // one winner per round with a key, and every margin held
  const bool pass = row_sum_i32(nadv + (good ? 0 : 256)) == nround;
  float s = 0.0f;
  int e = 0;
  if (live && pass && c < k) {
    e = scr[r * 16 + c];
    s = route_sigmoid(lg[t * ldl + e]);
  }
  float ssum = 0.0f;
#pragma unroll
  for (int j = 0; j < KR - 1; ++j)
    if (j < k) ssum += __int_as_float(__builtin_amdgcn_ds_bpermute((r * 16 + j) << 2, __float_as_int(s)));
  if (live && pass && c < k) {
    const float den = ssum < 1e-10f ? 1e-10f : ssum;
    route_emit(out, t0, t, k, c, e, s, den, route_scale, xdtype, hist, sel);
  }
  const bool redo = live && !pass;
  if (__builtin_amdgcn_ballot_w64(redo))
    route_batch_exact(lg, ldl, t, redo, t0, bias_s, E, k, route_scale, xdtype, out, hist, sel);
}

// Routes the block's tokens four per wave (rows); `scr` (LDS, 64 ints per
// wave) enables the screened rounds for k < 16.
__device__ __forceinline__ void route_tokens_rows(const float* lg, int ldl, int ntok, int t0, const float* bias_s,
                                                  int E, int k, float route_scale, int xdtype, const GateOut& out,
                                                  int* hist, int32_t* sel, int32_t* scr) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const int r = lane >> 4, c = lane & 15;
  float bq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) bq[q] = c + 16 * q < E ? bias_s[c + 16 * q] : 0.0f;
  int32_t* ws = scr ? scr + wave * 64 : nullptr;
  for (int tb = wave * 4; tb < ntok; tb += nw * 4) {
    const int t = tb + r;
    const bool live = t < ntok;
    if (ws && k < 8)
      route_batch_fast<8>(lg, ldl, t, live, t0, bias_s, bq, E, k, route_scale, xdtype, out, hist, sel, ws);
    else if (ws && k < 16)
      route_batch_fast<16>(lg, ldl, t, live, t0, bias_s, bq, E, k, route_scale, xdtype, out, hist, sel, ws);
    else
      route_batch_exact(lg, ldl, t, live, t0, bias_s, E, k, route_scale, xdtype, out, hist, sel);
  }
}

template <int NB4 = route_ntok(MAX_EPL)>
__device__ __forceinline__ void route_tokens(const float* lg, int ldl, int ntok, int t0, const float* bias_s, int E,
                                             int k, float route_scale, int xdtype, const GateOut& out, int* hist,
                                             int32_t* sel = nullptr, int32_t* scr = nullptr) {
  if (E <= 64)
    route_tokens_rows(lg, ldl, ntok, t0, bias_s, E, k, route_scale, xdtype, out, hist, sel, scr);
  else
    route_tokens_t<MAX_EPL, NB4>(lg, ldl, ntok, t0, bias_s, E, k, route_scale, xdtype, out, hist, sel);
}

__device__ __forceinline__ void flush_hist(const int* hist, int E, int32_t* counts) {
  if (!counts) return;
  for (int e = threadIdx.x; e < E; e += blockDim.x)
    if (hist[e]) atomicAdd(&counts[e], hist[e]);
}

}  // namespace dsmoe
