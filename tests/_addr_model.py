"""CPU model of the global-memory addresses the grouped GEMM kernels touch.

Restates, in numpy, the index arithmetic of the direct-load loaders and the
epilogue stores of

* ``gemm_qw_kernel``  (deepseek-v3-lite_amd/csrc/gemm_qw.hip, forward gemm1 / gemm2),
* ``gemm_sk_kernel``  (csrc/gemm_sk.hip, the decode few-row kernel),
* ``xgemm_q_kernel``  (csrc/gemm_xq.hip, backward dh, dx, dW13, dW2),

including the block -> tile enumeration (csrc/gemm_tile.h), the loads the
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


def sched_bound(rows: int, groups: int, bm: int) -> int:
    return rows // bm + groups + 1


# ---------------------------------------------------------------- gemm_qw (forward ping-pong kernel)
# Loading wave w (0..3) of group 0 loads A rows, wave w of group 1 the same B
# rows; slabs 0 .. nk - 1 (the model also covers the clamped reloads of the
# last slab, a superset).
QW_BM, QW_BK, QW_LD = 256, 64, 8


def qw_ok(g: Gemm) -> bool:
    """gemm_qw_ok (alignment of real pointers is not modelled; callers align)."""
    lim = 1 << 31
    return (1 <= g.nseg <= 2 and g.K % QW_BK == 0 and g.kseg % QW_BK == 0 and g.a_rows * g.lda < lim
            and g.N * g.ldb < lim and g.N % 8 == 0 and g.ldc % 8 == 0 and g.c_group_col % 8 == 0)


def qw_tile(rec: Recorder, g: Gemm, swiglu: bool, grp: int, row0: int, rows: int, n_tile: int, what: str):
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
    offa = 2 * (arow * g.lda + c * 8)
    bn = n0 + (r & 127) if NB == 2 else n0 + r
    offb = 2 * (np.minimum(bn, g.N - 1) * g.ldb + c * 8)
    # slabs loaded: 0 .. nk + 1 (the main loop refills slab kb + 2), clamped to nk - 1
    k0s = sorted({min(ka, nk - 1) * QW_BK for ka in (0, nk - 1, nk, nk + 1)})
    for k0 in k0s:
        rec.touch(g.A, offa + 2 * k0, offa + 2 * k0 + 16, what + " A")
        hi = k0 >= (g.kseg if g.nseg > 1 else 1 << 62)
        seg = g.nseg - 1 if hi else 0
        kin = k0 - g.kseg if hi else k0
        for w in range(4):
            tab = g.B1 if (NB == 2 and w >= 2) else g.B0
            blk = rec.index(np.array(tab, dtype=object), grp * g.nseg + seg, what + " B table")
            rec.touch(blk, offb[w] + 2 * kin, offb[w] + 2 * kin + 16, what + " B")
            # a slab never reads past its K segment within a row
            seg_len = (g.K - g.kseg if hi else g.kseg) if g.nseg > 1 else g.K
            if kin + 64 > seg_len:
                raise Violation(f"{what}: K slab {kin} past the segment")
    # epilogue: rows r < rows, 16-byte chunks of BN columns
    LPR = BN * 2 // 16
    rr = np.arange(rows)
    if g.c_map is not None:
        crow = rec.index(g.c_map, row0 + rr, what + " c_map")
    else:
        crow = row0 + rr
    ccol = grp * g.c_group_col
    n = n0 + np.arange(LPR) * 8
    n = n[n < g.N]
    off = 2 * ((crow[:, None] * g.ldc + ccol + n[None, :]))
    rec.touch(g.C, off, off + 16, what + " C")
    for sv in (g.Gs, g.Us):
        if swiglu and sv is not None:
            rec.touch(sv, off, off + 16, what + " G/U")


def qw_launch(rec: Recorder, gr: Gemm, swiglu: bool, gd: Optional[Gemm] = None, what: str = "gemm_qw"):
    """launch_gemm_qw / launch_gemm_qw_pair: grid from the host bounds, every block's tile."""
    bn = 128 if swiglu else 256
    mr = gr.m_tiles_bound if gr.sched is not None else cdiv(gr.dense_rows, QW_BM) * gr.groups
    if gd is None:
        grid = 8 * cdiv(mr * cdiv(gr.N, bn), 8)
        tl = tiles_single(gr, QW_BM, bn, grid)
    else:
        md = cdiv(gd.dense_rows, QW_BM) * gd.groups
        grid = 8 * (cdiv(md * cdiv(gd.N, bn), 8) + cdiv(mr * cdiv(gr.N, bn), 8))
        tl = tiles_pair(gr, gd, QW_BM, bn, grid)
    for which, grp, row0, rows, n_tile in tl:
        g = gd if which else gr
        if rows <= 0:
            raise Violation(f"{what}: empty tile")
        qw_tile(rec, g, swiglu, grp, row0, rows, n_tile, f"{what}[{'dense' if which else 'routed'} g{grp} r{row0}]")
    return len(tl)


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
