"""CPU model of the global-memory addresses the grouped GEMM kernels touch.

Restates, in numpy, the index arithmetic of the direct-load loaders and the
epilogue stores of

* ``gemm_qp_kernel``  (deepseek-v3-lite_amd/csrc/gemm_qp.hip, forward gemm1 / gemm2, persistent),
* ``gemm_sk_kernel``  (csrc/gemm_sk.hip, the decode few-row kernel),
* ``xgemm_q_kernel``  (csrc/gemm_xq.hip, backward dh, dx, dW13, dW2),

including the block -> tile enumeration (csrc/gemm_tile.h, and the persistent
workgroups' tile lists of gemm_qp.hip), the staged epilogues' LDS regions, the loads the
main loops issue past the last K slab (clamped to the last slab), and the
zero-block redirection of K-major rows past a weight-gradient range.  Every
access is returned as (buffer, first byte, last byte + 1) per lane, so a test
can assert that each one stays inside its allocation.  The model follows the
kernels statement by statement; a change to a loader's indexing must be
mirrored here.

Addresses are in bytes relative to the start of the buffer named.  Test
infrastructure only.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np


def cdiv(a, b):
    return -(-a // b)


# ---------------------------------------------------------------- descriptors
@dataclass
class Buf:
    """One allocation: its name and size in bytes."""
    name: str
    nbytes: int


@dataclass
class Gemm:
    """Forward GemmDesc (csrc/common.h) with buffers named instead of pointed to.

    B0 / B1: per (group * nseg + segment) a Buf of an (N x kseg) row-major block."""
    N: int
    K: int
    A: Buf
    lda: int
    a_rows: int
    B0: List[Buf]
    B1: Optional[List[Buf]]
    ldb: int
    kseg: int
    nseg: int
    C: Buf
    ldc: int
    sched: Optional[List[Tuple[int, int, int]]] = None   # routed: (group, row0, rows)
    dense_rows: int = 0
    groups: int = 0
    a_map: Optional[np.ndarray] = None
    c_map: Optional[np.ndarray] = None
    c_group_col: int = 0
    Gs: Optional[Buf] = None
    Us: Optional[Buf] = None
    m_tiles_bound: int = 0


class Violation(AssertionError):
    pass


class Recorder:
    """Collects per-buffer min / max byte extents and checks them."""

    def __init__(self):
        self.ext: Dict[str, List[int]] = {}
        self.size: Dict[str, int] = {}

    def touch(self, buf: Buf, lo, hi, what: str):
        lo = np.asarray(lo, dtype=np.int64)
        hi = np.asarray(hi, dtype=np.int64)
        if lo.size == 0:
            return
        mn, mx = int(lo.min()), int(hi.max())
        if mn < 0 or mx > buf.nbytes:
            raise Violation(f"{what}: {buf.name} accessed at [{mn}, {mx}) outside [0, {buf.nbytes})")
        e = self.ext.setdefault(buf.name, [mn, mx])
        e[0], e[1] = min(e[0], mn), max(e[1], mx)
        self.size[buf.name] = buf.nbytes

    def index(self, arr: np.ndarray, idx, what: str):
        idx = np.asarray(idx, dtype=np.int64)
        if idx.size and (idx.min() < 0 or idx.max() >= len(arr)):
            raise Violation(f"{what}: index [{idx.min()}, {idx.max()}] outside a table of {len(arr)}")
        return arr[idx]


# ---------------------------------------------------------------- tile enumeration (gemm_tile.h)
def _sched_tile(g: Gemm, m_tile: int, bm: int):
    if g.sched is not None:
        return g.sched[m_tile]
    tpg = cdiv(g.dense_rows, bm)
    grp = m_tile // tpg
    row0 = (m_tile - grp * tpg) * bm
    return grp, row0, min(bm, g.dense_rows - row0)


def tiles_single(g: Gemm, bm: int, bn: int, grid: int):
    """tile_for_block: blockIdx -> (grp, row0, rows, n_tile), XCD-chunked."""
    n_tiles = cdiv(g.N, bn)
    m_total = len(g.sched) if g.sched is not None else cdiv(g.dense_rows, bm) * g.groups
    total = m_total * n_tiles
    per_xcd = cdiv(total, 8)
    out = []
    for b in range(grid):
        j = b >> 3
        if j >= per_xcd:
            continue
        lin = (b & 7) * per_xcd + j
        if lin >= total:
            continue
        m_tile, n_tile = divmod(lin, n_tiles)
        grp, row0, rows = _sched_tile(g, m_tile, bm)
        out.append((0, grp, row0, rows, n_tile))
    return out


def tiles_pair(gr: Gemm, gd: Gemm, bm: int, bn: int, grid: int):
    """tile_for_block_pair: dense gd first on each XCD, then the routed gr."""
    ntr, ntd = cdiv(gr.N, bn), cdiv(gd.N, bn)
    tpg_d = cdiv(gd.dense_rows, bm)
    td = tpg_d * gd.groups * ntd
    mr = len(gr.sched) if gr.sched is not None else cdiv(gr.dense_rows, bm) * gr.groups
    tr = mr * ntr
    per_d, per_r = cdiv(td, 8), cdiv(tr, 8)
    out = []
    for b in range(grid):
        j, x = b >> 3, b & 7
        if j < per_d:
            lin = x * per_d + j
            if lin >= td:
                continue
            m_tile, n_tile = divmod(lin, ntd)
            grp = m_tile // tpg_d
            row0 = (m_tile - grp * tpg_d) * bm
            out.append((1, grp, row0, min(bm, gd.dense_rows - row0), n_tile))
            continue
        if j - per_d >= per_r:
            continue
        lin = x * per_r + (j - per_d)
        if lin >= tr:
            continue
        m_tile, n_tile = divmod(lin, ntr)
        grp, row0, rows = _sched_tile(gr, m_tile, bm)
        out.append((0, grp, row0, rows, n_tile))
    return out


def routed_schedule(counts, bm: int):
    """The scan kernel's M-tile list: per expert, tiles of bm rows over its range."""
    sched, off = [], 0
    for e, c in enumerate(counts):
        for r in range(0, int(c), bm):
            sched.append((e, off + r, min(bm, int(c) - r)))
        off += int(c)
    return sched


def sched_seq(sched):
    """MTile::seq of each entry (mtile_seq): its index among its group's M tiles and their count."""
    out, i = [], 0
    while i < len(sched):
        j = i
        while j < len(sched) and sched[j][0] == sched[i][0]:
            j += 1
        out += [(k, j - i) for k in range(j - i)]
        i = j
    return out


_SEQ_CACHE = {}


def routed_item(sched, lin: int, nt: int):
    """Item lin of a routed tile list (qp_tile): (M tile, N tile).  Inside a
    group of n M tiles with nt > n the items run N tile by N tile."""
    key = (id(sched), len(sched))
    if key not in _SEQ_CACHE:
        _SEQ_CACHE.clear()
        _SEQ_CACHE[key] = sched_seq(sched)
    mt, nb = divmod(lin, nt)
    i, n = _SEQ_CACHE[key][mt]
    if 1 < n < 65536 and nt > n:
        t0 = mt - i
        q = lin - t0 * nt
        mt, nb = t0 + q % n, q // n
    return mt, nb


def sched_bound(rows: int, groups: int, bm: int) -> int:
    return rows // bm + groups + 1


# ---------------------------------------------------------------- gemm_qp (forward persistent ping-pong kernel)
# Loading wave w (0..3) of group 0 loads A rows, wave w of group 1 the same B
# rows; a tile's loads cover its slabs 0 .. nk - 1 (the loaders then move on
# to the next tile of the workgroup).
QW_BM, QW_BK, QW_LD = 256, 64, 8
QP_STAGE = 8192   # bytes of a slot a wave may stage in (its own 8 KB)


def qp_ok(g: Gemm) -> bool:
    """gemm_qp_ok (alignment of real pointers is not modelled; callers align)."""
    lim = 1 << 31
    return (1 <= g.nseg <= 2 and g.K % QW_BK == 0 and g.kseg % QW_BK == 0 and g.a_rows * g.lda < lim
            and g.N * g.ldb < lim and g.N % 8 == 0 and g.ldc % 8 == 0 and g.c_group_col % 8 == 0)


def qp_lists(gr: Gemm, gd: Optional[Gemm], bm: int, bn: int, grid: int):
    """qp_list / qp_tile: per workgroup b, its tiles (which, grp, row0, rows, n_tile) in order."""
    ntr = cdiv(gr.N, bn)
    mr = len(gr.sched) if gr.sched is not None else cdiv(gr.dense_rows, bm) * gr.groups
    tr = mr * ntr
    per_r = cdiv(tr, 8)
    ntd, td, per_d = 1, 0, 0
    if gd is not None:
        ntd = cdiv(gd.N, bn)
        td = cdiv(gd.dense_rows, bm) * gd.groups * ntd
        per_d = cdiv(td, 8)
    nb = grid >> 3
    out = []
    for b in range(grid):
        x, j = b & 7, b >> 3
        r_base = x * per_r
        r_cnt = max(0, min(per_r, tr - r_base))
        d_base = x * per_d
        d_cnt = max(0, min(per_d, td - d_base)) if gd is not None else 0
        tot = d_cnt + r_cnt
        ntiles = cdiv(tot - j, nb) if tot > j else 0
        tiles = []
        for i in range(ntiles):
            li = j + i * nb
            assert li < tot
            if li < d_cnt:
                lin, nt, g, which = d_base + li, ntd, gd, 1
            else:
                lin, nt, g, which = r_base + (li - d_cnt), ntr, gr, 0
            if which == 0 and g.sched is not None:
                m_tile, n_tile = routed_item(g.sched, lin, nt)
            else:
                m_tile, n_tile = divmod(lin, nt)
            grp, row0, rows = _sched_tile(g, m_tile, bm)
            tiles.append((which, grp, row0, rows, n_tile))
        out.append(tiles)
    return out


def qp_loads(rec: Recorder, g: Gemm, swiglu: bool, grp: int, row0: int, rows: int, n_tile: int, what: str):
    """qpa_rows / qpa_step and qpb_set / qpb_step for one tile: slabs 0 .. nk - 1."""
    NB = 2 if swiglu else 1
    BN = 128 if swiglu else 256
    n0 = n_tile * BN
    nk = g.K // QW_BK
    wave = np.arange(4)[:, None, None]          # wave in its loading group
    lane = np.arange(64)[None, :, None]
    i = np.arange(QW_LD)[None, None, :]
    r = (wave * QW_LD + i) * 8 + (lane >> 3)
    c = (lane & 7) ^ ((r >> 1) & 7)
    ra = np.minimum(r, rows - 1)
    if g.a_map is not None:
        arow = rec.index(g.a_map, row0 + ra, what + " a_map")
    else:
        arow = row0 + ra
    offa = arow * (2 * g.lda) + c * 16
    if np.any(offa >= 1 << 32):
        raise Violation(f"{what}: A byte offset past 32 bits")
    bn = n0 + (r & 127) if NB == 2 else n0 + r
    offb = 2 * (np.minimum(bn, g.N - 1) * g.ldb + c * 8)
    for k0 in sorted({0, (nk - 1) * QW_BK}):
        rec.touch(g.A, offa + 2 * k0, offa + 2 * k0 + 16, what + " A")
        hi = k0 >= (g.kseg if g.nseg > 1 else 1 << 62)
        seg = g.nseg - 1 if hi else 0
        kin = k0 - g.kseg if hi else k0
        for w in range(4):
            tab = g.B1 if (NB == 2 and w >= 2) else g.B0
            blk = rec.index(np.array(tab, dtype=object), grp * g.nseg + seg, what + " B table")
            rec.touch(blk, offb[w] + 2 * kin, offb[w] + 2 * kin + 16, what + " B")
            seg_len = (g.K - g.kseg if hi else g.kseg) if g.nseg > 1 else g.K
            if kin + 64 > seg_len:
                raise Violation(f"{what}: K slab {kin} past the segment")


def _qp_swz(r, WB):
    return (((r >> 2) & 3) << 1) if WB == 64 else (((r >> 1) & 7) << 1)


_QP_STAGE_CHECKED = set()


def _qp_stage_check(swiglu: bool, rows: int):
    """The wave -> output-row mapping and the LDS staging of one tile height:
    staging stays inside the wave's own 8 KB, and the stored rows are exactly
    0 .. rows - 1, each once per column group (checked once per height)."""
    key = (swiglu, rows)
    if key in _QP_STAGE_CHECKED:
        return
    TN = 1 if swiglu else 2
    WB = 64 * TN
    LPR = WB // 16
    RPI = 64 // LPR
    passes = [(0, 4)] if swiglu else [(0, 2), (2, 2)]
    lane = np.arange(64)
    for G in (0, 1):
        for s in range(4):
            wm = s >> 1
            nmi = max(0, min(4, (cdiv(rows, 32) - wm + 1) >> 1))
            stored = []
            for j0, nj in passes:
                for j in range(j0, min(j0 + nj, nmi)):
                    r = (j - j0) * 32 + (lane & 31)
                    for ni in range(TN):
                        for q in range(4):
                            u = ni * 8 + 2 * q + (lane >> 5)
                            a = r * WB + ((u ^ _qp_swz(r, WB)) << 3)
                            if a.min() < 0 or (a + 8).max() > QP_STAGE:
                                raise Violation("staging write outside the wave's 8 KB")
                for it in range(nj * 32 // RPI):
                    j = j0 + (it * RPI) // 32
                    if j >= nmi:
                        break
                    r = it * RPI + lane // LPR
                    cc = lane % LPR
                    a = r * WB + (((2 * cc) ^ _qp_swz(r, WB)) << 3)
                    if a.min() < 0 or (a + 16).max() > QP_STAGE:
                        raise Violation("staging read outside the wave's 8 KB")
                    lr = (it * RPI) % 32 + lane // LPR
                    m = (2 * j + wm) * 32 + lr
                    stored += [int(v) for v, c in zip(m, cc) if v < rows and c == 0]
            want = [m for m in range(rows) if (m // 32) % 2 == wm]
            if sorted(stored) != want:
                raise Violation(f"wave (G{G}, s{s}) stores rows {sorted(set(stored))[:8]}.. not its {want[:8]}..")
    _QP_STAGE_CHECKED.add(key)


def qp_epilogue(rec: Recorder, g: Gemm, swiglu: bool, grp: int, row0: int, rows: int, n_tile: int, what: str):
    """qp_epilogue / qp_out_pass of every wave: rows 0 .. rows - 1 of the tile
    (mapping and LDS staging checked by _qp_stage_check), each row's 16-byte
    chunks of the tile's columns below N."""
    _qp_stage_check(swiglu, rows)
    BN = 128 if swiglu else 256
    n0 = n_tile * BN
    rr = np.arange(rows)
    crow = rec.index(g.c_map, row0 + rr, what + " c_map") if g.c_map is not None else row0 + rr
    n = n0 + np.arange(BN // 8) * 8
    n = n[n < g.N]
    off = 2 * (crow[:, None] * g.ldc + grp * g.c_group_col + n[None, :])
    rec.touch(g.C, off, off + 16, what + " C")
    for sv in (g.Gs, g.Us):
        if swiglu and sv is not None:
            rec.touch(sv, off, off + 16, what + " G/U")


def qp_launch(rec: Recorder, gr: Gemm, swiglu: bool, gd: Optional[Gemm] = None, what: str = "gemm_qp",
              grid: int = 256):
    """launch_gemm_qp / launch_gemm_qp_pair: one workgroup per CU, each through
    its tile list; every tile of the problem(s) exactly once."""
    bn = 128 if swiglu else 256
    lists = qp_lists(gr, gd, QW_BM, bn, grid)
    seen = set()
    n = 0
    for tiles in lists:
        for which, grp, row0, rows, n_tile in tiles:
            g = gd if which else gr
            if rows <= 0:
                raise Violation(f"{what}: empty tile")
            key = (which, grp, row0, n_tile)
            if key in seen:
                raise Violation(f"{what}: tile {key} in two workgroups' lists")
            seen.add(key)
            tag = f"{what}[{'dense' if which else 'routed'} g{grp} r{row0}]"
            qp_loads(rec, g, swiglu, grp, row0, rows, n_tile, tag)
            qp_epilogue(rec, g, swiglu, grp, row0, rows, n_tile, tag)
            n += 1
    mr = len(gr.sched) if gr.sched is not None else cdiv(gr.dense_rows, QW_BM) * gr.groups
    want = mr * cdiv(gr.N, bn) + (cdiv(gd.dense_rows, QW_BM) * gd.groups * cdiv(gd.N, bn) if gd is not None else 0)
    if n != want:
        raise Violation(f"{what}: {n} tiles covered of {want}")
    return n


# ---------------------------------------------------------------- gemm_sk (decode few-row kernel)
SK_BM, SK_KSTEP = 64, 32


def sk_ok(g: Gemm) -> bool:
    return (1 <= g.nseg <= 2 and g.K > 0 and g.K % (4 * SK_KSTEP) == 0 and g.kseg % SK_KSTEP == 0 and g.N % 8 == 0
            and g.lda % 8 == 0 and g.ldb % 8 == 0 and g.ldc % 8 == 0 and g.c_group_col % 8 == 0
            and g.Gs is None and g.Us is None)


def sk_tile(rec: Recorder, g: Gemm, swiglu: bool, grp: int, row0: int, rows: int, n_tile: int, what: str):
    BN = 32 if swiglu else 64
    n0 = n_tile * BN
    lane = np.arange(64)
    per = g.K // (4 * SK_KSTEP)
    MT = min(4, cdiv(rows, 16))
    for cg in range(4):
        w3 = swiglu and cg >= 2
        col = (n0 + 16 * (cg & 1) + (lane & 15)) if swiglu else (n0 + 16 * cg + (lane & 15))
        roff = np.minimum(col, g.N - 1) * g.ldb + (lane >> 4) * 8
        tab = g.B1 if w3 else g.B0
        for wave in range(4):
            for s in (0, per - 1):
                k0 = (wave * per + s) * SK_KSTEP
                hi = k0 >= (g.kseg if g.nseg > 1 else 1 << 62)
                kin = k0 - g.kseg if hi else k0
                blk = rec.index(np.array(tab, dtype=object), grp * g.nseg + (g.nseg - 1 if hi else 0), what + " B table")
                rec.touch(blk, 2 * (roff + kin), 2 * (roff + kin) + 16, what + " B")
    for mt in range(MT):
        r = np.minimum(16 * mt + (lane & 15), rows - 1)
        arow = rec.index(g.a_map, row0 + r, what + " a_map") if g.a_map is not None else row0 + r
        base = arow * g.lda + (lane >> 4) * 8
        for wave in range(4):
            for s in (0, per - 1):
                k0 = (wave * per + s) * SK_KSTEP
                rec.touch(g.A, 2 * (base + k0), 2 * (base + k0) + 16, what + " A")
    TPR = BN // 8
    rr = np.arange(rows)
    crow = rec.index(g.c_map, row0 + rr, what + " c_map") if g.c_map is not None else row0 + rr
    n = n0 + np.arange(TPR) * 8
    n = n[n < g.N]
    off = 2 * (crow[:, None] * g.ldc + grp * g.c_group_col + n[None, :])
    rec.touch(g.C, off, off + 16, what + " C")


def sk_launch(rec: Recorder, gr: Gemm, swiglu: bool, gd: Optional[Gemm] = None, what: str = "gemm_sk"):
    bn = 32 if swiglu else 64
    mt = lambda g: g.m_tiles_bound if g.sched is not None else cdiv(g.dense_rows, SK_BM) * g.groups
    if gd is None:
        grid = 8 * cdiv(mt(gr) * cdiv(gr.N, bn), 8)
        tl = tiles_single(gr, SK_BM, bn, grid)
    else:
        grid = 8 * (cdiv(mt(gd) * cdiv(gd.N, bn), 8) + cdiv(mt(gr) * cdiv(gr.N, bn), 8))
        tl = tiles_pair(gr, gd, SK_BM, bn, grid)
    for which, grp, row0, rows, n_tile in tl:
        if rows <= 0:
            continue
        sk_tile(rec, gd if which else gr, swiglu, grp, row0, rows, n_tile, what)
    return len(tl)


# ---------------------------------------------------------------- xgemm_q (backward quad-wave kernel)
XQ_BM = XQ_BN = 256
XQ_BK, XQ_LD = 64, 8
XS_ROUTED, XS_DENSE, XS_WGRAD = 0, 1, 2


@dataclass
class XGemm:
    """Backward XGemm (csrc/common.h) with named buffers."""
    mode: int                 # XS_*
    M: int
    N: int
    K: int
    a_km: bool                # XA_KMAJOR, else XA_ROWS
    A: Buf
    lda: int
    b_weights: bool           # XB_W_NN (weight table), else XB_ACT_KMAJOR
    Btab: Optional[List[Buf]] = None
    Bact: Optional[Buf] = None
    ldb: int = 0
    kseg: int = 0
    nseg: int = 1
    a_col: int = 0
    b_col: int = 0
    a_map: Optional[np.ndarray] = None
    sched: Optional[List[Tuple[int, int, int]]] = None
    bm: int = XQ_BM
    dense_rows: int = 0
    groups: int = 0
    k_off: Optional[np.ndarray] = None
    ksplit: int = 1
    # outputs
    C: Optional[Buf] = None
    ldc: int = 0
    c_map: Optional[np.ndarray] = None
    c_group_col: int = 0
    Ctab0: Optional[List[Buf]] = None
    Ctab1: Optional[List[Buf]] = None
    msplit: int = 0
    part: Optional[Buf] = None
    c_f32: bool = False       # XE_WGRAD output rows are fp32
    swiglu_bwd: bool = False
    Gs: Optional[Buf] = None
    Us: Optional[Buf] = None
    ld_gu: int = 0
    gu_group_col: int = 0
    du_off: int = 0


def xtiles(g: XGemm):
    """xtile<256, 256>: (grp, row0, rows, n_tile, kbeg, kend, split) per block."""
    n_tiles = cdiv(g.N, XQ_BN)
    if g.mode == XS_ROUTED:
        sub = g.bm // XQ_BM
        m_total = len(g.sched) * sub
    elif g.mode == XS_DENSE:
        tpg = cdiv(g.dense_rows, XQ_BM)
        m_total = tpg * g.groups
    else:
        tpg = cdiv(g.M, XQ_BM)
        m_total = tpg * g.groups * max(g.ksplit, 1)
    total = m_total * n_tiles
    per_xcd = cdiv(total, 8)
    grid = 8 * per_xcd
    out = []
    for b in range(grid):
        j = b >> 3
        if j >= per_xcd:
            continue
        lin = (b & 7) * per_xcd + j
        if lin >= total:
            continue
        mt, n_tile = divmod(lin, n_tiles)
        kbeg, kend, split = 0, g.K, 0
        if g.mode == XS_ROUTED:
            grp, r0, rws = g.sched[mt // sub]
            s = mt % sub
            row0, rows = r0 + s * XQ_BM, min(XQ_BM, rws - s * XQ_BM)
            if rows <= 0:
                continue
        else:
            ks = max(g.ksplit, 1) if g.mode == XS_WGRAD else 1
            gs = mt // tpg
            grp, split = divmod(gs, ks)
            m = mt - gs * tpg
            row0 = m * XQ_BM
            rows = min(XQ_BM, (g.dense_rows if g.mode == XS_DENSE else g.M) - row0)
            if g.mode == XS_WGRAD and g.k_off is not None:
                kbeg, kend = int(g.k_off[grp]), int(g.k_off[grp + 1])
            if ks > 1:
                ln = kend - kbeg
                chunk = cdiv(cdiv(ln, ks), 64) * 64
                b0 = kbeg + split * chunk
                kend = min(kend, b0 + chunk)
                kbeg = min(b0, kend)
        out.append((grp, row0, rows, n_tile, kbeg, kend, split))
    return out


def xq_tile(rec: Recorder, g: XGemm, grp, row0, rows, n_tile, kbeg, kend, split, what):
    n0 = n_tile * XQ_BN
    nk = cdiv(kend - kbeg, XQ_BK) if kend > kbeg else 0
    wave = np.arange(4)[:, None, None]
    lane = np.arange(64)[None, :, None]
    i = np.arange(XQ_LD)[None, None, :]
    if nk > 0:
        # slabs 0 .. nk + 1 (refills of kb + 2), clamped to nk - 1
        k0s = sorted({kbeg + min(ka, nk - 1) * XQ_BK for ka in (0, nk - 1, nk, nk + 1)})
        kr = wave * 16 + (lane >> 5)                           # KM k row of load 0
        if not g.a_km:
            r = (wave * XQ_LD + i) * 8 + (lane >> 3)
            c = (lane & 7) ^ ((r >> 1) & 7)
            ra = np.minimum(r, rows - 1)
            arow = rec.index(g.a_map, row0 + ra, what + " a_map") if g.a_map is not None else row0 + ra
            offa = arow * g.lda + c * 8
            for k0 in k0s:
                rec.touch(g.A, 2 * (offa + k0), 2 * (offa + k0) + 16, what + " A rows")
        else:
            cpar = [(lane & 31) ^ (((kr + 2 * par) & 3) << 2) for par in (0, 1)]
            mcol = [np.minimum(row0 + 8 * cp, g.M - 8) for cp in cpar]
            for k0 in k0s:
                krow = k0 + kr + 2 * i                                  # the row load i reads
                col = np.where((i & 1) == 0, mcol[0], mcol[1])
                live = krow < kend                                       # else the zero block
                off = krow * g.lda + grp * g.a_col + col
                rec.touch(g.A, 2 * off[live], 2 * off[live] + 16, what + " A KM")
                if (col + 8 > g.lda - grp * g.a_col).any():
                    raise Violation(f"{what}: A KM column past the row")
        # B (always K-major)
        cpar = [(lane & 31) ^ (((kr + 2 * par) & 3) << 2) for par in (0, 1)]
        ncol = [np.minimum(n0 + 8 * cp, g.N - 8) for cp in cpar]
        for k0 in k0s:
            krow = k0 + kr + 2 * i
            col = np.where((i & 1) == 0, ncol[0], ncol[1])
            if g.b_weights:
                hi = k0 >= (g.kseg if g.nseg > 1 else 1 << 62)
                seg = g.nseg - 1 if hi else 0
                kin = k0 - g.kseg if hi else k0
                blk = rec.index(np.array(g.Btab, dtype=object), grp * g.nseg + seg, what + " B table")
                off = (krow - k0 + kin) * g.ldb + col
                rec.touch(blk, 2 * off, 2 * off + 16, what + " B W")
            else:
                live = krow < kend
                off = krow * g.ldb + grp * g.b_col + col
                rec.touch(g.Bact, 2 * off[live], 2 * off[live] + 16, what + " B act")
    # epilogue
    if g.mode == XS_WGRAD and (g.ksplit > 1 or g.c_f32):
        # register-direct float4 stores: split-K partials, or fp32 gradient rows
        j = np.arange(4)[:, None, None, None]
        wm = (np.arange(4) >> 1)[None, :, None, None]
        wn = (np.arange(4) & 1)[None, :, None, None]
        ln = np.arange(64)[None, None, :, None]
        m = (2 * j + wm) * 32 + (ln & 31)
        nq = np.arange(16)[None, None, None, :]            # ni * 4 + q
        n = n0 + wn * 128 + (nq >> 2) * 32 + (nq & 3) * 8 + (ln >> 5) * 4
        ok = np.broadcast_to((m < rows) & (n < g.N), np.broadcast_shapes(m.shape, n.shape))
        if g.ksplit > 1:
            off = 4 * ((((split * g.groups + grp) * g.M + row0 + m) * g.N) + n)
            off = np.broadcast_to(off, ok.shape)
            rec.touch(g.part, off[ok], off[ok] + 16, what + " part")
            return
        r = np.broadcast_to(row0 + m, ok.shape)
        nn = np.broadcast_to(n, ok.shape)
        lo = r < g.msplit
        for sel, tab, rel in ((ok & lo, g.Ctab0, r), (ok & ~lo, g.Ctab1, r - g.msplit)):
            if sel.any():
                buf = rec.index(np.array(tab, dtype=object), grp, what + " Ctab")
                off = 4 * (rel[sel] * g.ldc + nn[sel])
                rec.touch(buf, off, off + 16, what + " C fp32")
        return
    rr = row0 + np.arange(rows)
    if g.mode == XS_WGRAD:
        # rows below msplit go to Ctab0[grp], the rest to Ctab1[grp]
        lo = rr < g.msplit
        tab0 = rec.index(np.array(g.Ctab0, dtype=object), grp, what + " Ctab0")
        tab1 = rec.index(np.array(g.Ctab1, dtype=object), grp, what + " Ctab1")
        targets = [(tab0, rr[lo] * g.ldc), (tab1, (rr[~lo] - g.msplit) * g.ldc)]
    else:
        crow = rec.index(g.c_map, rr, what + " c_map") if g.c_map is not None else rr
        targets = [(g.C, crow * g.ldc + grp * g.c_group_col)]
    if not g.swiglu_bwd:
        n = n0 + np.arange(32) * 8
        n = n[n < g.N]
        for buf, base in targets:
            off = 2 * (base[:, None] + n[None, :])
            rec.touch(buf, off, off + 16, what + " C")
        return
    # SwiGLU backward: dg at row + n, du at row + du_off + n; g, u reads
    n = n0 + np.concatenate([h * 128 + np.arange(16) * 8 for h in (0, 1)])
    n = n[n < g.N]
    crow = rec.index(g.c_map, rr, what + " c_map") if g.c_map is not None else rr
    base = crow * g.ldc + grp * g.c_group_col
    off = 2 * (base[:, None] + n[None, :])
    rec.touch(g.C, off, off + 16, what + " dg")
    rec.touch(g.C, off + 2 * g.du_off, off + 2 * g.du_off + 16, what + " du")
    ogu = 2 * (rr[:, None] * g.ld_gu + grp * g.gu_group_col + n[None, :])
    rec.touch(g.Gs, ogu, ogu + 16, what + " g")
    rec.touch(g.Us, ogu, ogu + 16, what + " u")


def xq_ok(g: XGemm) -> bool:
    lim = 1 << 31
    if g.N % 8 or g.N < 8:
        return False
    if not g.a_km:
        if g.lda % 8 or g.K % XQ_BK:
            return False
    else:
        if g.a_map is not None or g.lda % 8 or g.a_col % 8 or g.M % 8 or g.M < 8:
            return False
        if (XQ_BK + 1) * g.lda >= lim:
            return False
    if g.b_weights:
        if g.a_km or g.kseg % XQ_BK or g.ldb % 8 or not 1 <= g.nseg <= 2:
            return False
    else:
        if not g.a_km or g.ldb % 8 or g.b_col % 8:
            return False
    return XQ_BK * g.ldb < lim


def xq_launch(rec: Recorder, g: XGemm, what: str):
    tl = xtiles(g)
    keys = {(grp, row0, n_tile, split) for grp, row0, rows, n_tile, kbeg, kend, split in tl}
    if len(keys) != len(tl):
        raise Violation(f"{what}: a tile in two blocks")
    for grp, row0, rows, n_tile, kbeg, kend, split in tl:
        xq_tile(rec, g, grp, row0, rows, n_tile, kbeg, kend, split, f"{what}[g{grp} r{row0} n{n_tile} s{split}]")
    return len(tl)


XM_BM, XM_BN = 256, 256


def xgemm_tiles(M: int, N: int, groups: int) -> int:
    return cdiv(M, XM_BM) * cdiv(N, XM_BN) * groups


def xgemm_pick_ksplit(tiles: int, k_len: int) -> int:
    """gemm_xm.hip xgemm_pick_ksplit: the split of the shared-expert weight
    gradients' K range (parts of whole slabs) that best fills 256 CUs."""
    if tiles >= 1024 or k_len < 4 * 64:
        return 1
    best, best_cost = 1, cdiv(tiles, 256)
    ks = 2
    while ks <= 8 and k_len // ks >= 128:
        cost = cdiv(tiles * ks, 256) / ks + 0.02 * ks
        if cost < best_cost - 1e-9:
            best, best_cost = ks, cost
        ks += 1
    return best
