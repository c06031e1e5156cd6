// Slot ranking and placement shared by the permute kernels and the routing
// launch of the MFMA gate.  Restates the stable argsort of
// models/moe.py:107-117: sorted position of slot (t, j) routed to e =
// (slots of experts < e) + (tokens < t routed to e); a token holds an expert
// in at most one slot.
#pragma once

#include "common.h"

namespace dsmoe {

// Inclusive prefix sum over the 64 lanes of a wave (exact integer adds), on
// DPP: row (16-lane) shifts by 1, 2, 4, 8 (lanes without a source add 0),
// then the row broadcasts of lane 15 (into rows 1 and 3) and lane 31 (into
// rows 2 and 3).
__device__ __forceinline__ int32_t wave_incl_scan(int32_t x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}

// Lane 63's value in every lane.
__device__ __forceinline__ int32_t wave_last(int32_t x) { return __builtin_amdgcn_readlane(x, 63); }

// Ranks the slots of rank block b: tokens b * RANK_TOKENS + t for t < ntok,
// whose experts sit in sel[t * k + j] (LDS, -1 past ntok).  Lane t holds
// token t; wave w of nw takes experts w, w + nw, ...  A slot is ranked when
// its id lies in [0, E) and is the last occurrence of that id in its token;
// every other slot gets rank -1 (not placed).  hist[e] (LDS) receives the
// block's count of e.  Ranks go to rank_lds[t * k + j] when it is given (a
// call's only rank block), else to po.local_rank with the counts in
// po.blockhist[b * E + e].
template <int KB>
__device__ __forceinline__ void rank_block(const int32_t* sel, int ntok, int k, int E, int b, const PermuteOut& po,
                                           int32_t* hist, int32_t* rank_lds) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int t = lane;
  const int64_t s0 = ((int64_t)b * RANK_TOKENS + t) * k;
  int ex[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) ex[j] = (j < k && t < ntok) ? sel[t * k + j] : -1;
  if (wave == 0 && t < ntok) {
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      bool placed = (unsigned)ex[j] < (unsigned)E;
#pragma unroll
      for (int j2 = j + 1; j2 < KB; ++j2)
        if (ex[j2] == ex[j]) placed = false;
      if (j < k && !placed) {
        if (rank_lds)
          rank_lds[t * k + j] = -1;
        else
          po.local_rank[s0 + j] = -1;
      }
    }
  }
  const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
  for (int e = wave; e < E; e += nw) {
    int jsel = -1;
#pragma unroll
    for (int j = 0; j < KB; ++j)
      if (ex[j] == e) jsel = j;
    const uint64_t mask = __ballot(jsel >= 0);
    if (jsel >= 0) {
      const int32_t r = __popcll(mask & below);
      if (rank_lds)
        rank_lds[t * k + jsel] = r;
      else
        po.local_rank[s0 + jsel] = r;
    }
    if (lane == 0) {
      hist[e] = __popcll(mask);
      if (!rank_lds) po.blockhist[(int64_t)b * E + e] = __popcll(mask);
    }
  }
}

// Exclusive scans over the experts of cnt[] (LDS) by wave 0: off[e] (E + 1
// entries, off[E] = the total) and til[e], the first M tile of expert e in
// tiles of bm rows (til[E] = the tile count).
__device__ __forceinline__ void scan_experts(const int32_t* cnt, int E, int bm, int32_t* off, int32_t* til) {
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  int32_t co = 0, ct = 0;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    const int32_t c = e < E ? cnt[e] : 0;
    const int32_t tc = (c + bm - 1) / bm;
    const int32_t xo = wave_incl_scan(c), xt = wave_incl_scan(tc);
    if (e < E) {
      off[e] = co + xo - c;
      til[e] = ct + xt - tc;
    }
    co += wave_last(xo);
    ct += wave_last(xt);
  }
  if (lane == 0) {
    off[E] = co;
    til[E] = ct;
  }
}

// Counts, offsets, the schedule length and its M tiles, from the LDS scans.
__device__ __forceinline__ void write_offsets(const int32_t* cnt, const int32_t* off, const int32_t* til, int E,
                                              const PermuteOut& po) {
  for (int e = threadIdx.x; e <= E; e += blockDim.x) {
    po.offsets[e] = off[e];
    if (e < E && po.counts) po.counts[e] = cnt[e];
    if (e == E) *po.sched_count = til[E];
  }
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    const int32_t c = cnt[e], t0 = til[e];
    for (int i = 0; i * po.bm < c; ++i) {
      MTile m;
      m.group = e;
      m.row0 = off[e] + i * po.bm;
      m.rows = min(po.bm, c - i * po.bm);
      m.seq = mtile_seq(i, (c + po.bm - 1) / po.bm);
      po.sched[t0 + i] = m;
    }
  }
}

// Slot s (routed to e in [0, E)) at pos = off[e] + base + rank; a slot
// without a rank, or a position outside its expert's range, is not placed.
__device__ __forceinline__ void place_slot(int64_t s, int e, int32_t rank, int32_t base, const int32_t* off, int k,
                                           const PermuteOut& po) {
  if (rank < 0) return;
  const int32_t pos = off[e] + base + rank;
  if (pos < off[e] || pos >= off[e + 1]) return;
  po.sorted_slot[pos] = (int32_t)s;
  po.sorted_token[pos] = (int32_t)(s / k);
  po.slot_pos[s] = pos;
  if (po.sorted_w) po.sorted_w[pos] = po.w[s];
}

// The rest of the permute for a call whose tokens form one rank block (after
// rank_block with rank_lds): offsets and schedule from hist, then every slot.
__device__ __forceinline__ void finish_single_block(const int32_t* sel, const int32_t* rank_lds, int ntok, int k,
                                                    int E, const PermuteOut& po, const int32_t* hist, int32_t* off,
                                                    int32_t* til) {
  __syncthreads();
  scan_experts(hist, E, po.bm, off, til);
  __syncthreads();
  write_offsets(hist, off, til, E, po);
  for (int s = threadIdx.x; s < ntok * k; s += blockDim.x) {
    const int e = sel[s];
    if ((unsigned)e < (unsigned)E) place_slot(s, e, rank_lds[s], 0, off, k, po);
  }
}

}  // namespace dsmoe
