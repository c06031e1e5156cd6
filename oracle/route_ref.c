/* CPU restatement of the reference's routing arithmetic — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker.  The HIP product path never does.
 *
 * Functions and the reference lines they restate:
 *   oracle_route()   models/moe.py:32-36   sigmoid scores, +bias, top-k over the
 *                                           biased scores, gather of the unbiased
 *                                           scores, renormalisation * route_scale;
 *                    models/moe.py:114     per-expert counts (bincount).
 *   oracle_permute() models/moe.py:108-115 flat_idx -> stable argsort by expert,
 *                                           sorted token ids, offsets (E+1 form of
 *                                           models/moe_triton.py:33).
 *
 * Conventions fixed here (torch leaves them implementation-defined):
 *   - sigmoid is evaluated in double and rounded once to float
 *     (s = (float)(1 / (1 + exp(-(double)logit)))), i.e. correctly rounded
 *     except in cases rarer than 1 in 2^28;
 *   - top-k order is descending biased score; equal biased scores are ordered
 *     by ascending expert id;
 *   - the renormalising sum runs over j = 0..k-1 in that order, in float;
 *   - the permutation is the stable (expert, token) order.
 * Parity: pinned against torch.sigmoid/topk/argsort(stable)/bincount, the
 * reference docs' permutation example and golden vectors written by the
 * reference (tests/test_oracle.py).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

float oracle_sigmoid(float x) { return (float)(1.0 / (1.0 + exp(-(double)x))); }

/* logits (T,E) row-major fp32, bias (E) fp32.
 * Outputs: idx (T,k), weights (T,k) fp32, sel_scores (T,k) fp32 (unbiased
 * scores of the selected experts), counts (E).  Returns 0, or -1 on bad args. */
int oracle_route(const float* logits, const float* bias, int T, int E, int k, float route_scale,
                 int32_t* idx, float* weights, float* sel_scores, int32_t* counts) {
  if (T < 0 || E <= 0 || k <= 0 || k > E || k > 64) return -1;
  for (int e = 0; e < E; ++e) counts[e] = 0;
  for (int t = 0; t < T; ++t) {
    const float* row = logits + (int64_t)t * E;
    float topv[64];
    int topi[64];
    int n = 0;
    for (int e = 0; e < E; ++e) {
      float s = oracle_sigmoid(row[e]);
      float b = s + bias[e];
      /* insertion position: first slot whose value is strictly smaller */
      int pos = n;
      while (pos > 0 && topv[pos - 1] < b) --pos;
      if (pos >= k) continue;
      int last = n < k ? n : k - 1;
      for (int q = last; q > pos; --q) { topv[q] = topv[q - 1]; topi[q] = topi[q - 1]; }
      topv[pos] = b;
      topi[pos] = e;
      if (n < k) ++n;
    }
    float ssum = 0.0f;
    float sel[64];
    for (int j = 0; j < k; ++j) {
      sel[j] = oracle_sigmoid(row[topi[j]]);
      ssum += sel[j];
    }
    float den = ssum < 1e-10f ? 1e-10f : ssum;
    for (int j = 0; j < k; ++j) {
      idx[(int64_t)t * k + j] = topi[j];
      sel_scores[(int64_t)t * k + j] = sel[j];
      weights[(int64_t)t * k + j] = sel[j] / den * route_scale;
      counts[topi[j]] += 1;
    }
  }
  return 0;
}

/* idx (T,k) expert ids in [0,E).  Slot s = t*k + j.
 * Outputs: offsets (E+1), sorted_slot (N) slot id at each sorted position,
 * sorted_token (N) = sorted_slot / k, slot_pos (N) inverse of sorted_slot.
 * Stable counting sort: within one expert, slots keep ascending slot order,
 * which is ascending token order because a token selects an expert at most once. */
int oracle_permute(const int32_t* idx, int T, int k, int E, int32_t* offsets, int32_t* sorted_slot,
                   int32_t* sorted_token, int32_t* slot_pos) {
  if (T < 0 || k <= 0 || E <= 0) return -1;
  int64_t N = (int64_t)T * k;
  for (int e = 0; e <= E; ++e) offsets[e] = 0;
  for (int64_t s = 0; s < N; ++s) {
    int e = idx[s];
    if (e < 0 || e >= E) return -2;
    offsets[e + 1] += 1;
  }
  for (int e = 0; e < E; ++e) offsets[e + 1] += offsets[e];
  int32_t cursor[4096];
  if (E > 4096) return -1;
  for (int e = 0; e < E; ++e) cursor[e] = offsets[e];
  for (int64_t s = 0; s < N; ++s) {
    int e = idx[s];
    int32_t p = cursor[e]++;
    sorted_slot[p] = (int32_t)s;
    sorted_token[p] = (int32_t)(s / k);
    slot_pos[s] = p;
  }
  return 0;
}

/* Smallest gap between the k-th and (k+1)-th biased score over all tokens
 * (the "boundary margin"): a routing comparison is only meaningful when it
 * exceeds the sigmoid rounding differences between implementations. */
float oracle_min_margin(const float* logits, const float* bias, int T, int E, int k) {
  float best = INFINITY;
  if (k >= E) return best;
  for (int t = 0; t < T; ++t) {
    const float* row = logits + (int64_t)t * E;
    float topv[65];
    int n = 0;
    for (int e = 0; e < E; ++e) {
      float b = oracle_sigmoid(row[e]) + bias[e];
      int pos = n;
      while (pos > 0 && topv[pos - 1] < b) --pos;
      if (pos > k) continue;
      int last = n < k + 1 ? n : k;
      for (int q = last; q > pos; --q) topv[q] = topv[q - 1];
      topv[pos] = b;
      if (n < k + 1) ++n;
    }
    float gap = topv[k - 1] - topv[k];
    if (gap < best) best = gap;
  }
  return best;
}
