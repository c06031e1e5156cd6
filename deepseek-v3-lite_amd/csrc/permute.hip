// (b) Permute / dispatch: stable (expert, token) order without a host sync.
// Restates models/moe.py:107-117 (argsort, bincount, offsets) and the row
// gather flat[sorted_token_ids] of models/moe.py:127,150.
//
// Tokens are taken in rank blocks of RANK_TOKENS = 64 (one token per lane).
//   rank         for each expert a wave ballot over the block's tokens gives
//                every slot its rank among the block's earlier tokens routed
//                to that expert, and the block's count (blockhist).  Done by
//                rank_kernel here, or by the routing launch of the MFMA gate
//                for the tokens it has just routed (rank.h).
//   prefix_scatter_kernel  one workgroup per rank block (per run of rank
//                blocks when there are more than 256): it sums blockhist over
//                every block (expert totals, hence offsets) and over the
//                blocks before its own (its base inside each expert), and
//                places its slots at pos = offsets[e] + base[e] + rank.
//                Workgroup 0 also writes counts, offsets and the M-tile
//                schedule.  Each workgroup reads the whole histogram (nb x E
//                ints, cache-resident) instead of waiting on a separate scan.
//   A call of one rank block (T <= 64) is finished by its ranking workgroup:
//   one launch.
//   gather_rows  x_sorted[p] = x[sorted_token[p]] with 16-byte accesses.
//   scatter_rows the same copy from the token side: x_sorted[slot_pos[t k + j]]
//                = x[t], each row of x read once.
#include "rank.h"

namespace dsmoe {

// One rank block per workgroup (4 waves), idx read into LDS; a call of one
// rank block finishes its permute here.
// LDS: sel[64 k] | rank[64 k] | hist[E] | off[E + 1] | til[E + 1]
template <int KB>
__global__ __launch_bounds__(256) void rank_kernel(const int32_t* __restrict__ idx, int T, int k, int E, int nb,
                                                   PermuteOut po) {
  extern __shared__ int32_t rsh[];
  int32_t* sel = rsh;
  int32_t* rank_lds = sel + RANK_TOKENS * k;
  int32_t* hist = rank_lds + RANK_TOKENS * k;
  int32_t* off = hist + E;
  int32_t* til = off + E + 1;
  const int b = blockIdx.x;
  const int t0 = b * RANK_TOKENS;
  const int ntok = max(0, min(RANK_TOKENS, T - t0));
  for (int i = threadIdx.x; i < RANK_TOKENS * k; i += blockDim.x)
    sel[i] = i < ntok * k ? idx[(int64_t)t0 * k + i] : -1;
  __syncthreads();
  const bool single = nb <= 1;
  rank_block<KB>(sel, ntok, k, E, b, po, hist, single ? rank_lds : nullptr);
  if (single) finish_single_block(sel, rank_lds, ntok, k, E, po, hist, off, til);
}

// Expert totals and this workgroup's base from blockhist, then its slots.
// LDS: cnt[E] | base[E] | off[E + 1] | til[E + 1] | red[2][4][64]
__global__ __launch_bounds__(256) void prefix_scatter_kernel(const int32_t* __restrict__ idx, int T, int k, int E,
                                                             int nb, int G, PermuteOut po) {
  extern __shared__ int32_t psh[];
  int32_t* cnt = psh;
  int32_t* base = cnt + E;
  int32_t* off = base + E;
  int32_t* til = off + E + 1;
  int32_t* red = til + E + 1;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b0 = blockIdx.x * G, b1 = min(nb, b0 + G);
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    int32_t tot = 0, pre = 0;
    if (e < E) {
      // 16 loads in flight per lane: unconditional, from a clamped block
      // index, and those past nb are not added
      constexpr int U = 16;
      for (int b = wave; b < nb; b += 4 * U) {
        int32_t v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = po.blockhist[(int64_t)min(b + 4 * u, nb - 1) * E + e];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int bb = b + 4 * u;
          const int32_t w = bb < nb ? v[u] : 0;
          tot += w;
          pre += bb < b0 ? w : 0;
        }
      }
    }
    red[wave * 64 + lane] = tot;
    red[256 + wave * 64 + lane] = pre;
    __syncthreads();
    if (wave == 0 && e < E) {
      cnt[e] = ((red[lane] + red[64 + lane]) + red[128 + lane]) + red[192 + lane];
      base[e] = ((red[256 + lane] + red[320 + lane]) + red[384 + lane]) + red[448 + lane];
    }
    __syncthreads();
  }
  scan_experts(cnt, E, po.bm, off, til);
  __syncthreads();
  if (blockIdx.x == 0) write_offsets(cnt, off, til, E, po);
  for (int rb = b0; rb < b1; ++rb) {
    const int64_t s0 = (int64_t)rb * RANK_TOKENS * k;
    const int64_t s1 = min((int64_t)T * k, s0 + (int64_t)RANK_TOKENS * k);
    for (int64_t s = s0 + tid; s < s1; s += blockDim.x) {
      const int e = idx[s];
      if ((unsigned)e < (unsigned)E) place_slot(s, e, po.local_rank[s], base[e], off, k, po);
    }
    if (rb + 1 < b1) {
      __syncthreads();
      for (int e = tid; e < E; e += blockDim.x) base[e] += po.blockhist[(int64_t)rb * E + e];
      __syncthreads();
    }
  }
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

// Token-major copy of a permutation's rows, 16-byte vectors: workgroup t
// reads row t of src once and writes it to the k sorted rows slot_pos[t k + j]
// (uniform per workgroup: scalar loads, issued with the row's loads).  A slot
// position outside [0, nrows) (left unset by an invalid routing) is not
// written.
__global__ __launch_bounds__(256) void scatter_rows_kernel(const uint4* __restrict__ src,
                                                           const int32_t* __restrict__ slot_pos, int k, int vec_per_row,
                                                           int64_t nrows, uint4* __restrict__ dst) {
  const int64_t t = blockIdx.x;
  const int32_t* sp = slot_pos + t * k;
  for (int c = threadIdx.x; c < vec_per_row; c += blockDim.x) {
    const uint4 v = src[t * vec_per_row + c];
    for (int j = 0; j < k; ++j) {
      const int32_t p = sp[j];
      if (p >= 0 && p < nrows) dst[(int64_t)p * vec_per_row + c] = v;
    }
  }
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
      m.seq = mtile_seq(i, (c + bm - 1) / bm);
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
  s.local_rank = c.take<int32_t>(N);
  s.sched = c.take<MTile>(sched_bound(N, d.E, bm));
  s.sched_count = c.take<int32_t>(1);
  if (out) *out = s;
  return c.used();
}

PermuteOut permute_out(const PermuteScratch& s, int bm, int32_t* offsets, int32_t* sorted_slot, int32_t* sorted_token,
                       int32_t* slot_pos, int32_t* counts, const float* w, float* sorted_w) {
  PermuteOut po;
  po.offsets = offsets;
  po.sorted_slot = sorted_slot;
  po.sorted_token = sorted_token;
  po.slot_pos = slot_pos;
  po.counts = counts;
  po.w = w;
  po.sorted_w = sorted_w;
  po.sched = s.sched;
  po.sched_count = s.sched_count;
  po.bm = bm;
  po.blockhist = s.blockhist;
  po.local_rank = s.local_rank;
  return po;
}

int launch_permute(const int32_t* idx, const dsmoe_dims& d, const PermuteOut& po, bool ranked, hipStream_t st) {
  const int nb = (int)cdiv(d.T, RANK_TOKENS);
  if (!ranked) {
    const size_t lds = sizeof(int32_t) * (2 * RANK_TOKENS * d.k + 3 * d.E + 2);
    if (d.k <= 8)
      hipLaunchKernelGGL(rank_kernel<8>, dim3(max(nb, 1)), dim3(256), lds, st, idx, d.T, d.k, d.E, nb, po);
    else
      hipLaunchKernelGGL(rank_kernel<MAX_TOPK>, dim3(max(nb, 1)), dim3(256), lds, st, idx, d.T, d.k, d.E, nb, po);
    const int rc = check_launch("permute(rank)");
    if (rc) return rc;
  }
  if (nb <= 1) return DSMOE_OK;   // finished by the ranking workgroup
  const int G = (int)cdiv(nb, 256);
  const size_t lds = sizeof(int32_t) * (4 * d.E + 2 + 512);
  hipLaunchKernelGGL(prefix_scatter_kernel, dim3((unsigned)cdiv(nb, G)), dim3(256), lds, st, idx, d.T, d.k, d.E, nb,
                     G, po);
  return check_launch("permute(scatter)");
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

int launch_scatter_rows(const void* x, int64_t T, int k, const int32_t* slot_pos, const int32_t* sorted_token,
                        int D, int elem, void* dst, hipStream_t st) {
  const int64_t nrows = T * k;
  if (nrows == 0) return DSMOE_OK;
  const int64_t row_bytes = (int64_t)D * elem;
  if (row_bytes % 16 || (uintptr_t)x % 16 || (uintptr_t)dst % 16)
    return launch_gather_rows(x, T, sorted_token, nrows, D, elem, dst, st);
  const int vpr = (int)(row_bytes / 16);
  const unsigned threads = (unsigned)std::min<int64_t>(256, cdiv(vpr, 64) * 64);
  hipLaunchKernelGGL(scatter_rows_kernel, dim3((unsigned)T), dim3(threads), 0, st, static_cast<const uint4*>(x),
                     slot_pos, k, vpr, nrows, static_cast<uint4*>(dst));
  return check_launch("scatter_rows");
}

int launch_sched_from_offsets(const int64_t* offsets64, int E, int bm, int64_t rows, int32_t* offsets32, MTile* sched,
                              int32_t* sched_count, hipStream_t st) {
  hipLaunchKernelGGL(sched_from_offsets_kernel, dim3(1), dim3(256), sizeof(int32_t) * (E + 2), st, offsets64, E, bm,
                     rows, offsets32, sched, sched_count);
  return check_launch("sched_from_offsets");
}

}  // namespace dsmoe

