// Device helpers shared by the grouped GEMM kernels.
#pragma once

#include "common.h"

namespace dsmoe {

// Maps blockIdx.x to (group, first row, valid rows, N tile).  Tiles are
// enumerated M-major, N fastest; block b runs on XCD b % 8 and XCD x takes the
// x-th contiguous eighth of the tile list.  Returns false for surplus blocks.
template <int BM>
__device__ __forceinline__ bool tile_for_block(const GemmDesc& g, int n_tiles, int& grp, int& row0, int& rows,
                                               int& n_tile) {
  int64_t m_total;
  int tpg = 0;
  if (g.sched) {
    m_total = *g.sched_count;
  } else {
    tpg = (int)cdiv(g.dense_rows, BM);
    m_total = (int64_t)tpg * g.groups;
  }
  const int64_t total = m_total * n_tiles;
  const int64_t per_xcd = cdiv(total, 8);
  const int64_t j = blockIdx.x >> 3;
  if (j >= per_xcd) return false;
  const int64_t lin = (int64_t)(blockIdx.x & 7) * per_xcd + j;
  if (lin >= total) return false;
  const int64_t m_tile = lin / n_tiles;
  n_tile = (int)(lin - m_tile * n_tiles);
  if (g.sched) {
    const MTile t = g.sched[m_tile];
    grp = t.group;
    row0 = t.row0;
    rows = t.rows;
  } else {
    grp = (int)(m_tile / tpg);
    const int mt = (int)(m_tile - (int64_t)grp * tpg);
    row0 = mt * BM;
    rows = min(BM, g.dense_rows - row0);
  }
  return true;
}

// Tile lookup for two problems in one launch: gr (routed schedule or dense)
// and gd (dense, e.g. the shared experts over all tokens), both with output
// tiles BN wide.  Each XCD takes the x-th eighth of gd's tiles first, then the
// x-th eighth of gr's, so both problems are spread evenly over the XCDs and
// the dense tiles (the longer ones when gd has the larger K) start first.
// Surplus blocks return false.  which = 1 selects gd.
template <int BM>
__device__ __forceinline__ bool tile_for_block_pair(const GemmDesc& gr, const GemmDesc& gd, int bn, int& which,
                                                    int& grp, int& row0, int& rows, int& n_tile) {
  const int ntr = (int)cdiv(gr.N, bn), ntd = (int)cdiv(gd.N, bn);
  const int tpg_d = (int)cdiv(gd.dense_rows, BM);
  const int64_t td = (int64_t)tpg_d * gd.groups * ntd;
  int tpg_r = 0;
  int64_t mr;
  if (gr.sched) {
    mr = *gr.sched_count;
  } else {
    tpg_r = (int)cdiv(gr.dense_rows, BM);
    mr = (int64_t)tpg_r * gr.groups;
  }
  const int64_t tr = mr * ntr;
  const int64_t per_d = cdiv(td, 8), per_r = cdiv(tr, 8);
  const int64_t j = blockIdx.x >> 3, x = blockIdx.x & 7;
  int64_t lin;
  if (j < per_d) {
    which = 1;
    lin = x * per_d + j;
    if (lin >= td) return false;
    const int64_t m_tile = lin / ntd;
    n_tile = (int)(lin - m_tile * ntd);
    grp = (int)(m_tile / tpg_d);
    row0 = (int)(m_tile - (int64_t)grp * tpg_d) * BM;
    rows = min(BM, gd.dense_rows - row0);
    return true;
  }
  which = 0;
  if (j - per_d >= per_r) return false;
  lin = x * per_r + (j - per_d);
  if (lin >= tr) return false;
  const int64_t m_tile = lin / ntr;
  n_tile = (int)(lin - m_tile * ntr);
  if (gr.sched) {
    const MTile t = gr.sched[m_tile];
    grp = t.group;
    row0 = t.row0;
    rows = t.rows;
  } else {
    grp = (int)(m_tile / tpg_r);
    row0 = (int)(m_tile - (int64_t)grp * tpg_r) * BM;
    rows = min(BM, gr.dense_rows - row0);
  }
  return true;
}

// Backward GEMM tile lookup for the three XGemm schedules (same XCD-chunked
// enumeration as tile_for_block) of block blk, which runs on XCD blk mod 8.
// Returns false for surplus blocks.
//   XS_ROUTED  schedule entries of height bm, split into bm / BMK sub-tiles;
//   XS_DENSE   every group covers rows [0, dense_rows);
//   XS_WGRAD   M = weight rows per group; K range = k_off[grp] .. k_off[grp+1],
//              cut into ksplit parts of whole 64-row slabs (part index -> split).
template <int BMK, int BNK>
__device__ __forceinline__ bool xtile_at(const XGemm& g, int64_t blk, int& grp, int& row0, int& rows, int& n_tile,
                                         int& kbeg, int& kend, int& split) {
  const int n_tiles = (int)cdiv(g.N, BNK);
  int64_t m_total;
  int sub = 1, tpg = 0;
  if (g.sched_mode == XS_ROUTED) {
    sub = g.bm / BMK;
    m_total = (int64_t)(*g.sched_count) * sub;
  } else if (g.sched_mode == XS_DENSE) {
    tpg = (int)cdiv(g.dense_rows, BMK);
    m_total = (int64_t)tpg * g.groups;
  } else {
    tpg = (int)cdiv(g.M, BMK);
    m_total = (int64_t)tpg * g.groups * max(g.ksplit, 1);
  }
  const int64_t total = m_total * n_tiles;
  const int64_t per_xcd = cdiv(total, 8);
  const int64_t j = blk >> 3;
  if (j >= per_xcd) return false;
  const int64_t lin = (blk & 7) * per_xcd + j;
  if (lin >= total) return false;
  const int64_t mt = lin / n_tiles;
  n_tile = (int)(lin - mt * n_tiles);
  kbeg = 0;
  kend = g.K;
  split = 0;
  if (g.sched_mode == XS_ROUTED) {
    const MTile t = g.sched[mt / sub];
    const int s = (int)(mt % sub);
    grp = t.group;
    row0 = t.row0 + s * BMK;
    rows = min(BMK, t.rows - s * BMK);
    if (rows <= 0) return false;
  } else {
    const int ks = (g.sched_mode == XS_WGRAD) ? max(g.ksplit, 1) : 1;
    const int gs = (int)(mt / tpg);  // (group, split) in group-major order
    grp = gs / ks;
    split = gs - grp * ks;
    const int m = (int)(mt - (int64_t)gs * tpg);
    row0 = m * BMK;
    rows = min(BMK, (g.sched_mode == XS_DENSE ? g.dense_rows : g.M) - row0);
    if (g.sched_mode == XS_WGRAD && g.k_off) {
      kbeg = g.k_off[grp];
      kend = g.k_off[grp + 1];
    }
    if (ks > 1) {
      const int len = kend - kbeg;
      const int chunk = (int)cdiv(cdiv(len, ks), 64) * 64;
      const int b = kbeg + split * chunk;
      kend = min(kend, b + chunk);
      kbeg = min(b, kend);
    }
  }
  return true;
}

template <int BMK, int BNK>
__device__ __forceinline__ bool xtile(const XGemm& g, int& grp, int& row0, int& rows, int& n_tile, int& kbeg, int& kend,
                                      int& split) {
  return xtile_at<BMK, BNK>(g, blockIdx.x, grp, row0, rows, n_tile, kbeg, kend, split);
}

}  // namespace dsmoe
