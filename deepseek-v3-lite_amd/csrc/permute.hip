// (b) Permute / dispatch: stable (expert, token) order without a host sync.
// Restates models/moe.py:107-117 (argsort, bincount, offsets) and the row
// gather flat[sorted_token_ids] of models/moe.py:127,150.
//
//   rank_kernel     one workgroup per 64 tokens (a rank block), its four waves
//                   splitting the experts: for each expert a wave ballot gives
//                   every slot its rank among the block's earlier tokens, and
//                   the block histogram (no atomics, deterministic).
//   scan_kernel     one block of 16 waves: per-expert exclusive scans over the
//                   block histograms (wave prefix sums, 64 blocks at a time),
//                   counts, offsets (E+1), and the M-tile schedule used by the
//                   grouped GEMMs (tiles of bm rows inside each expert).
//   scatter_kernel  pos = offsets[e] + blockbase[b][e] + rank; writes the
//                   sorted order, its inverse and optional weight gather.
//   permute_small_kernel  the three stages in one workgroup for calls of at
//                   most PERMUTE_SMALL_T tokens (decode), one launch.
//   gather_rows     x_sorted[p] = x[sorted_token[p]] with 16-byte accesses.
#include "common.h"

namespace dsmoe {

constexpr int RANK_TOKENS = 64;  // one wave64 per block, one token per lane
constexpr int MAX_K = 16;

// Ranks of the slots of rank block b (one wave, lane = token) for experts
// e0, e0 + estep, ...: for each expert a wave ballot gives every slot its rank
// among the block's earlier tokens, and the block's count of that expert.
template <int KB>  // bound on k (slots compared per expert)
__device__ __forceinline__ void rank_experts(const int32_t* __restrict__ idx, int T, int k, int E, int b, int e0,
                                             int estep, int32_t* __restrict__ blockhist,
                                             int32_t* __restrict__ local_rank) {
  const int lane = threadIdx.x & 63;
  const int t = b * RANK_TOKENS + lane;
  int ex[KB];
#pragma unroll
  for (int j = 0; j < KB; ++j) ex[j] = -1;
  if (t < T)
    for (int j = 0; j < k; ++j) ex[j] = idx[(int64_t)t * k + j];
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int e = e0; e < E; e += estep) {
    int jsel = -1;
#pragma unroll
    for (int j = 0; j < KB; ++j)
      if (ex[j] == e) jsel = j;
    const uint64_t mask = __ballot(jsel >= 0);
    if (jsel >= 0) local_rank[(int64_t)t * k + jsel] = __popcll(mask & below);
    if (lane == 0) blockhist[(int64_t)b * E + e] = __popcll(mask);
  }
}

// One rank block (64 tokens) per workgroup; its four waves split the experts.
template <int KB>
__global__ __launch_bounds__(256) void rank_kernel(const int32_t* __restrict__ idx, int T, int k, int E,
                                                   int32_t* __restrict__ blockhist, int32_t* __restrict__ local_rank) {
  rank_experts<KB>(idx, T, k, E, blockIdx.x, threadIdx.x >> 6, blockDim.x >> 6, blockhist, local_rank);
}

// Inclusive prefix sum over the 64 lanes of a wave (exact integer adds), on
// DPP: row (16-lane) shifts by 1, 2, 4, 8 (lanes without a source add 0),
// then the row broadcasts of lane 15 (into rows 1 and 3) and lane 31 (into
// rows 2 and 3).
__device__ __forceinline__ int32_t wave_incl_scan(int32_t x, int /*lane*/) {
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

// Scan over the block histograms by one workgroup.  LDS sh: cnt[E],
// off[E+1], tiles[E+1].  Wave w scans experts w, w + nw, ...: lane b holds
// block b's count of the expert, 64 blocks at a time, carried across chunks.
// Wave 0 then scans counts and tile counts over the experts, 64 at a time.
// Integer sums: the same values as a serial scan.
__device__ __forceinline__ void scan_body(const int32_t* __restrict__ blockhist, int nb, int E, int bm,
                                          int32_t* __restrict__ blockbase, int32_t* __restrict__ counts,
                                          int32_t* __restrict__ offsets, MTile* __restrict__ sched,
                                          int32_t* __restrict__ sched_count, int32_t* sh) {
  int32_t* cnt = sh;
  int32_t* off = sh + E;
  int32_t* til = off + E + 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const int epw = wave < E ? (E - wave + nw - 1) / nw : 0;   // experts of this wave
  const int nch = (nb + 63) / 64;                            // 64-block chunks per expert
  constexpr int PRE = 16;
  if (nch == 0) {
    for (int e = wave; e < E; e += nw)
      if (lane == 0) cnt[e] = 0;
  } else if (epw * nch <= PRE) {
    // every (expert, chunk) value of this wave is loaded before the scans, so
    // the global round trips overlap instead of following each other
    int32_t v[PRE];
#pragma unroll
    for (int i = 0; i < PRE; ++i) {
      v[i] = 0;
      if (i < epw * nch) {
        const int e = wave + (i / nch) * nw, b = (i % nch) * 64 + lane;
        if (b < nb) v[i] = blockhist[(int64_t)b * E + e];
      }
    }
    int32_t carry = 0;
#pragma unroll
    for (int i = 0; i < PRE; ++i) {
      if (i < epw * nch) {
        const int e = wave + (i / nch) * nw, c = i % nch, b = c * 64 + lane;
        if (c == 0) carry = 0;
        const int32_t x = wave_incl_scan(v[i], lane);
        if (b < nb) blockbase[(int64_t)b * E + e] = carry + x - v[i];
        carry += wave_last(x);
        if (c == nch - 1 && lane == 0) cnt[e] = carry;
      }
    }
  } else {
    for (int e = wave; e < E; e += nw) {
      int32_t carry = 0;
      for (int b0 = 0; b0 < nb; b0 += 64) {
        const int b = b0 + lane;
        const int32_t v = b < nb ? blockhist[(int64_t)b * E + e] : 0;
        const int32_t x = wave_incl_scan(v, lane);
        if (b < nb) blockbase[(int64_t)b * E + e] = carry + x - v;
        carry += wave_last(x);
      }
      if (lane == 0) cnt[e] = carry;
    }
  }
  __syncthreads();
  if (wave == 0) {
    int32_t co = 0, ct = 0;
    for (int e0 = 0; e0 < E; e0 += 64) {
      const int e = e0 + lane;
      const int32_t c = e < E ? cnt[e] : 0;
      const int32_t tc = (c + bm - 1) / bm;
      const int32_t xo = wave_incl_scan(c, lane), xt = wave_incl_scan(tc, lane);
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
      *sched_count = ct;
    }
  }
  __syncthreads();
  for (int e = tid; e <= E; e += blockDim.x) {
    offsets[e] = off[e];
    if (e < E && counts) counts[e] = cnt[e];
  }
  for (int e = tid; e < E; e += blockDim.x) {
    const int32_t c = cnt[e], base = til[e];
    for (int i = 0; i * bm < c; ++i) {
      MTile m;
      m.group = e;
      m.row0 = off[e] + i * bm;
      m.rows = min(bm, c - i * bm);
      m.pad = 0;
      sched[base + i] = m;
    }
  }
}

__global__ __launch_bounds__(1024) void scan_kernel(const int32_t* __restrict__ blockhist, int nb, int E, int bm,
                                                    int32_t* __restrict__ blockbase, int32_t* __restrict__ counts,
                                                    int32_t* __restrict__ offsets, MTile* __restrict__ sched,
                                                    int32_t* __restrict__ sched_count) {
  extern __shared__ int32_t sh[];
  scan_body(blockhist, nb, E, bm, blockbase, counts, offsets, sched, sched_count, sh);
}

// Slot s: pos = offsets[e] + blockbase[b][e] + rank; writes the sorted order,
// its inverse and the optional weight gather.
__device__ __forceinline__ void scatter_slot(int64_t s, const int32_t* __restrict__ idx,
                                             const int32_t* __restrict__ local_rank,
                                             const int32_t* __restrict__ blockbase,
                                             const int32_t* __restrict__ offsets, int k, int E,
                                             int32_t* __restrict__ sorted_slot, int32_t* __restrict__ sorted_token,
                                             int32_t* __restrict__ slot_pos, const float* __restrict__ w,
                                             float* __restrict__ sorted_w) {
  const int t = (int)(s / k);
  const int e = idx[s];
  // Invalid routing (an id outside [0, E), or an id repeated within a token,
  // whose earlier slots get no rank) is not placed: no write leaves the
  // expert's range of sorted positions.
  if ((unsigned)e >= (unsigned)E) return;
  const int b = t / RANK_TOKENS;
  const int32_t pos = offsets[e] + blockbase[(int64_t)b * E + e] + local_rank[s];
  if (pos < offsets[e] || pos >= offsets[e + 1]) return;
  sorted_slot[pos] = (int32_t)s;
  sorted_token[pos] = t;
  slot_pos[s] = pos;
  if (sorted_w) sorted_w[pos] = w[s];
}

__global__ void scatter_kernel(const int32_t* __restrict__ idx, const int32_t* __restrict__ local_rank,
                               const int32_t* __restrict__ blockbase, const int32_t* __restrict__ offsets, int T, int k,
                               int E, int32_t* __restrict__ sorted_slot, int32_t* __restrict__ sorted_token,
                               int32_t* __restrict__ slot_pos, const float* __restrict__ w, float* __restrict__ sorted_w) {
  const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (s >= (int64_t)T * k) return;
  scatter_slot(s, idx, local_rank, blockbase, offsets, k, E, sorted_slot, sorted_token, slot_pos, w, sorted_w);
}

// Small calls (decode): rank, scan and scatter in one workgroup of 16 waves,
// with workgroup barriers (which order the global scratch writes) between
// the stages.  The waves share out (rank block, expert phase) pairs.
template <int KB>
__global__ __launch_bounds__(1024) void permute_small_kernel(const int32_t* __restrict__ idx, int T, int k, int E,
                                                             int bm, int32_t* __restrict__ blockhist,
                                                             int32_t* __restrict__ local_rank,
                                                             int32_t* __restrict__ blockbase,
                                                             int32_t* __restrict__ counts,
                                                             int32_t* __restrict__ offsets, MTile* __restrict__ sched,
                                                             int32_t* __restrict__ sched_count,
                                                             int32_t* __restrict__ sorted_slot,
                                                             int32_t* __restrict__ sorted_token,
                                                             int32_t* __restrict__ slot_pos,
                                                             const float* __restrict__ w, float* __restrict__ sorted_w) {
  extern __shared__ int32_t sh[];
  const int nb = (T + RANK_TOKENS - 1) / RANK_TOKENS;
  const int nw = blockDim.x >> 6, wave = threadIdx.x >> 6;
  const int per_b = max(1, nw / max(nb, 1));
  for (int pr = wave; pr < nb * per_b; pr += nw)
    rank_experts<KB>(idx, T, k, E, pr / per_b, pr % per_b, per_b, blockhist, local_rank);
  __syncthreads();
  scan_body(blockhist, nb, E, bm, blockbase, counts, offsets, sched, sched_count, sh);
  __syncthreads();
  const int64_t N = (int64_t)T * k;
  for (int64_t s = threadIdx.x; s < N; s += blockDim.x)
    scatter_slot(s, idx, local_rank, blockbase, offsets, k, E, sorted_slot, sorted_token, slot_pos, w, sorted_w);
}

// Row gather with 16-byte vectors; row_bytes % 16 == 0.
// Row indices outside [0, src_rows) (left unset by an invalid routing) gather
// zero rows instead of reading out of bounds.
__global__ void gather_rows_kernel(const uint4* __restrict__ src, const int32_t* __restrict__ rows, int64_t nrows,
                                   int vec_per_row, int64_t src_rows, uint4* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nrows * vec_per_row) return;
  const int64_t r = i / vec_per_row;
  const int c = (int)(i - r * vec_per_row);
  const int32_t sr = rows[r];
  dst[i] = (sr >= 0 && sr < src_rows) ? src[(int64_t)sr * vec_per_row + c] : make_uint4(0, 0, 0, 0);
}

template <typename T>
__global__ void gather_rows_scalar_kernel(const T* __restrict__ src, const int32_t* __restrict__ rows, int64_t nrows,
                                          int D, int64_t src_rows, T* __restrict__ dst) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nrows * D) return;
  const int64_t r = i / D;
  const int c = (int)(i - r * D);
  const int32_t sr = rows[r];
  dst[i] = (sr >= 0 && sr < src_rows) ? src[(int64_t)sr * D + c] : T(0);
}

// Schedule from caller-provided int64 offsets (E+1) (grouped operator seam).
// Offsets that are not monotone, do not start at 0 or exceed `rows` yield an
// empty schedule (nothing is computed) instead of out-of-bounds accesses.
__global__ __launch_bounds__(256) void sched_from_offsets_kernel(const int64_t* __restrict__ offsets64, int E, int bm,
                                                                 int64_t rows, int32_t* __restrict__ offsets32,
                                                                 MTile* __restrict__ sched,
                                                                 int32_t* __restrict__ sched_count) {
  extern __shared__ int32_t til[];  // E+1, then one flag
  const int tid = threadIdx.x;
  if (tid == 0) {
    int32_t tl = 0;
    bool ok = offsets64[0] == 0 && offsets64[E] <= rows;
    for (int e = 0; e < E; ++e) {
      til[e] = tl;
      const int64_t c = offsets64[e + 1] - offsets64[e];
      if (c < 0) ok = false;
      tl += (int32_t)((c + bm - 1) / bm);
    }
    til[E] = tl;
    til[E + 1] = ok ? 1 : 0;
    *sched_count = ok ? tl : 0;
  }
  __syncthreads();
  if (!til[E + 1]) {
    // invalid offsets: every group is empty for the consumers of offsets32
    for (int e = tid; e <= E; e += blockDim.x) offsets32[e] = 0;
    return;
  }
  for (int e = tid; e <= E; e += blockDim.x) offsets32[e] = (int32_t)offsets64[e];
  for (int e = tid; e < E; e += blockDim.x) {
    const int32_t o = (int32_t)offsets64[e];
    const int32_t c = (int32_t)(offsets64[e + 1] - offsets64[e]);
    for (int i = 0; i * bm < c; ++i) {
      MTile m;
      m.group = e;
      m.row0 = o + i * bm;
      m.rows = min(bm, c - i * bm);
      m.pad = 0;
      sched[til[e] + i] = m;
    }
  }
}

// ---------------------------------------------------------------- host side
int64_t sched_bound(int64_t rows, int groups, int bm) { return rows / bm + groups + 1; }

size_t permute_scratch_carve(Carver& c, const dsmoe_dims& d, int bm, PermuteScratch* out) {
  const int64_t nb = cdiv(d.T, RANK_TOKENS);
  const int64_t N = (int64_t)d.T * d.k;
  PermuteScratch s;
  s.blockhist = c.take<int32_t>(nb * d.E);
  s.blockbase = c.take<int32_t>(nb * d.E);
  s.local_rank = c.take<int32_t>(N);
  s.sched = c.take<MTile>(sched_bound(N, d.E, bm));
  s.sched_count = c.take<int32_t>(1);
  if (out) *out = s;
  return c.used();
}

int launch_permute(const int32_t* idx, const dsmoe_dims& d, int bm, const PermuteScratch& s, int32_t* offsets,
                   int32_t* sorted_slot, int32_t* sorted_token, int32_t* slot_pos, int32_t* counts, const float* w,
                   float* sorted_w, hipStream_t st) {
  const int nb = (int)cdiv(d.T, RANK_TOKENS);
  const int64_t N = (int64_t)d.T * d.k;
  const size_t lds = sizeof(int32_t) * (3 * d.E + 2);
  if (d.T <= PERMUTE_SMALL_T) {
    if (d.k <= 8)
      hipLaunchKernelGGL(permute_small_kernel<8>, dim3(1), dim3(1024), lds, st, idx, d.T, d.k, d.E, bm, s.blockhist,
                         s.local_rank, s.blockbase, counts, offsets, s.sched, s.sched_count, sorted_slot, sorted_token,
                         slot_pos, w, sorted_w);
    else
      hipLaunchKernelGGL(permute_small_kernel<MAX_K>, dim3(1), dim3(1024), lds, st, idx, d.T, d.k, d.E, bm,
                         s.blockhist, s.local_rank, s.blockbase, counts, offsets, s.sched, s.sched_count, sorted_slot,
                         sorted_token, slot_pos, w, sorted_w);
    return check_launch("permute_small");
  }
  if (d.k <= 8)
    hipLaunchKernelGGL(rank_kernel<8>, dim3(nb), dim3(256), 0, st, idx, d.T, d.k, d.E, s.blockhist, s.local_rank);
  else
    hipLaunchKernelGGL(rank_kernel<MAX_K>, dim3(nb), dim3(256), 0, st, idx, d.T, d.k, d.E, s.blockhist, s.local_rank);
  hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(1024), lds, st, s.blockhist, nb, d.E, bm, s.blockbase, counts, offsets,
                     s.sched, s.sched_count);
  if (N > 0)
    hipLaunchKernelGGL(scatter_kernel, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, st, idx, s.local_rank, s.blockbase,
                       offsets, d.T, d.k, d.E, sorted_slot, sorted_token, slot_pos, w, sorted_w);
  return check_launch("permute");
}

int launch_gather_rows(const void* x, int64_t src_rows, const int32_t* rows, int64_t nrows, int D, int elem, void* dst,
                       hipStream_t st) {
  if (nrows == 0) return DSMOE_OK;
  const int64_t row_bytes = (int64_t)D * elem;
  if (row_bytes % 16 == 0 && ((uintptr_t)x % 16 == 0) && ((uintptr_t)dst % 16 == 0)) {
    const int vpr = (int)(row_bytes / 16);
    hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)cdiv(nrows * vpr, 256)), dim3(256), 0, st,
                       static_cast<const uint4*>(x), rows, nrows, vpr, src_rows, static_cast<uint4*>(dst));
  } else if (elem == 2) {
    hipLaunchKernelGGL(gather_rows_scalar_kernel<uint16_t>, dim3((unsigned)cdiv(nrows * D, 256)), dim3(256), 0, st,
                       static_cast<const uint16_t*>(x), rows, nrows, D, src_rows, static_cast<uint16_t*>(dst));
  } else {
    hipLaunchKernelGGL(gather_rows_scalar_kernel<float>, dim3((unsigned)cdiv(nrows * D, 256)), dim3(256), 0, st,
                       static_cast<const float*>(x), rows, nrows, D, src_rows, static_cast<float*>(dst));
  }
  return check_launch("gather_rows");
}

int launch_sched_from_offsets(const int64_t* offsets64, int E, int bm, int64_t rows, int32_t* offsets32, MTile* sched,
                              int32_t* sched_count, hipStream_t st) {
  hipLaunchKernelGGL(sched_from_offsets_kernel, dim3(1), dim3(256), sizeof(int32_t) * (E + 2), st, offsets64, E, bm,
                     rows, offsets32, sched, sched_count);
  return check_launch("sched_from_offsets");
}

}  // namespace dsmoe

