"""Index arithmetic of the MLA attention kernels (csrc/mla.hip), restated on
the CPU (no kernel launches): every work item is run exactly once, every
direct 16-byte load into LDS fills its tile exactly once at the position the
reads expect and reads inside its source rows, and the peeled tile loops
never leave their tile ranges and run unmasked only where every pair is
visible.  Each function below restates the named kernel's formula.
"""
import itertools

import pytest

QB, KB, QI, KW, KT = 128, 64, 64, 128, 64   # MLA_QB, MLA_KB, MLB_QI, MLB_KW, MLB_KT
SPREAD = 32                                 # MLA_SPREAD


def mla_item(blk, BH, nrank):
    """mla_item: block -> (batch-head pair, rank) or None."""
    x, j = blk & 7, blk >> 3
    if BH >= SPREAD:
        nh = (BH - x + 7) >> 3
        if j >= nh * nrank:
            return None
        rank = j // nh
        return x + 8 * (j - rank * nh), rank
    total = BH * nrank
    per = (total + 7) // 8
    item = x * per + j
    if j >= per or item >= total:
        return None
    return item // nrank, item % nrank


def mla_grid(BH, nrank):
    return 8 * ((BH + 7) // 8) * nrank


@pytest.mark.parametrize("BH", list(range(1, 40)) + [63, 64, 65, 96, 127, 128, 129, 512, 2049])
def test_work_items_are_run_exactly_once(BH):
    for nrank in (1, 2, 3, 16, 17, 64):
        seen = set()
        for blk in range(mla_grid(BH, nrank)):
            r = mla_item(blk, BH, nrank)
            if r is None:
                continue
            assert 0 <= r[0] < BH and 0 <= r[1] < nrank, (BH, nrank, blk, r)
            assert r not in seen, (BH, nrank, blk, r)
            seen.add(r)
        assert len(seen) == BH * nrank


def test_work_items_start_longest_first_per_xcd():
    # with enough pairs, an XCD's blocks take rank 0 of all its pairs before rank 1
    BH, nrank = 96, 16
    for x in range(8):
        ranks = [mla_item(blk, BH, nrank)[1] for blk in range(x, mla_grid(BH, nrank), 8)
                 if mla_item(blk, BH, nrank) is not None]
        assert ranks == sorted(ranks)
        pairs = {mla_item(blk, BH, nrank)[0] for blk in range(x, mla_grid(BH, nrank), 8)
                 if mla_item(blk, BH, nrank) is not None}
        assert pairs == set(range(x, BH, 8))


def _g(r):
    return ((r & 3) << 2) | ((r >> 2) & 3)


def mlb_off(r, c, rb):
    """mlb_off: byte offset of 16-byte chunk c of row r in the swizzled tile."""
    return r * rb + (((c & ~15) | ((c & 15) ^ _g(r))) << 4)


def mla_vswz(nv, k):
    return 0 if nv == 1 else (8 * ((k >> 1) & 1) if nv == 2 else 8 * (k & 3))


@pytest.mark.parametrize("nstep,nv", list(itertools.product((2, 4, 6, 8, 12, 16), (1, 2, 4, 8))))
def test_direct_loads_fill_the_swizzled_tiles(nstep, nv):
    # the backward kernels' issue() (Q / dO tiles of 64 rows, K / V tiles of
    # 64 keys) and the forward's K tile: lane l of the wave's 1 KB block u
    # writes LDS offset 16 l and loads logical chunk pc ^ g(row) of its row
    DQKp, DVp = 16 * nstep, 32 * nv
    for width in (DQKp, DVp):
        rb = (width + 127) // 128 * 256
        tile = 64 * rb
        per_wave = tile // 4096
        seen = set()
        for wave, u, lane in itertools.product(range(4), range(per_wave), range(64)):
            blk = wave * per_wave + u
            ofs = blk * 1024 + 16 * lane
            row, pc = ofs // rb, (ofs % rb) >> 4
            cl = (pc & ~15) | ((pc & 15) ^ _g(row))
            if cl >= width // 8:
                continue                       # padding chunk: not loaded, never read
            assert row * width * 2 + 16 * cl + 16 <= 64 * width * 2
            assert mlb_off(row, cl, rb) == ofs
            assert (row, cl) not in seen
            seen.add((row, cl))
        assert len(seen) == 64 * width // 8
    # the forward's V tile: rows of DVp * 2 bytes, 8-byte unit u at u ^ vswz
    rb = DVp * 2
    seen = set()
    for wave, u, lane in itertools.product(range(4), range(64 * rb // 4096), range(64)):
        blk = wave * (64 * rb // 4096) + u
        ofs = blk * 1024 + 16 * lane
        row, pc = ofs // rb, (ofs % rb) >> 4
        cl = pc ^ (mla_vswz(nv, row) >> 1)
        assert 0 <= cl < DVp // 8
        for half in (0, 1):
            assert row * rb + (((2 * cl + half) ^ mla_vswz(nv, row)) << 3) == ofs + 8 * half
        seen.add((row, cl))
    assert len(seen) == 64 * DVp // 8


@pytest.mark.parametrize("nstep", (2, 4, 6, 8, 12, 16))
def test_fragment_reads_use_per_lane_offsets_plus_immediates(nstep):
    # MlbLane keeps mlb_off of rows 0..31 and chunk groups 0..7 per lane and
    # adds R RB + 256 (st >> 3) as immediates: that equals mlb_off of the full
    # row and chunk only because the swizzle sees the low four bits of each
    DQKp = 16 * nstep
    rb = (DQKp + 127) // 128 * 256
    for lane in range(64):
        hi, l32 = lane >> 5, lane & 31
        f = [mlb_off(l32, 2 * st + hi, rb) for st in range(8)]
        for R, st in itertools.product(range(0, 64, 32), range(nstep)):
            assert f[st & 7] + R * rb + 256 * (st >> 3) == mlb_off(R + l32, 2 * st + hi, rb)
            assert 2 * st + hi < DQKp // 8                       # a chunk the loads fill
        gq, sl = lane >> 4, lane & 15
        r = 4 * (gq >> 1) + (sl >> 2)
        for r0, ct in itertools.product(range(0, 64, 16), range(DQKp // 32)):
            u = 8 * (ct & 3) + 4 * (gq & 1) + (sl & 3)
            t0 = mlb_off(r, u >> 1, rb) + ((u & 1) << 3)
            t1 = mlb_off(r + 8, u >> 1, rb) + ((u & 1) << 3)
            uf = 8 * ct + 4 * (gq & 1) + (sl & 3)                # the unit of the full column
            assert t0 + r0 * rb + 256 * (ct >> 2) == mlb_off(r0 + r, uf >> 1, rb) + ((uf & 1) << 3)
            assert t1 + r0 * rb + 256 * (ct >> 2) == mlb_off(r0 + r + 8, uf >> 1, rb) + ((uf & 1) << 3)
            assert (uf >> 1) < DQKp // 8
    # the transposing reads: lanes 0-31 take rows r0 + {0-3, 8-11}, lanes 32-63 r0 + {4-7, 12-15}
    for half in (0, 1):
        rows = {4 * ((lane >> 4) >> 1) + ((lane & 15) >> 2) + d
                for lane in range(32 * half, 32 * half + 32) for d in (0, 8)}
        assert rows == {4 * half + i + d for i in range(4) for d in (0, 8)}


def kv_kernel_bounds(S_q, S_kv, causal, q_start, k0):
    """mla_bwd_kv_kernel: query tiles and the unmasked range [i_lo, i_hi)."""
    qb = (max(0, k0 - q_start) // QI * QI) if causal else 0
    nqt = (S_q - qb + QI - 1) // QI if S_q > qb else 0
    i_lo = i_hi = 0
    if k0 + KW <= S_kv:
        i_lo = min(nqt, max(0, (k0 + KW - 1 - q_start - qb + QI - 1) // QI)) if causal else 0
        i_hi = max(i_lo, (S_q - qb) // QI)
    return qb, nqt, i_lo, i_hi


def q_kernel_bounds(S_q, S_kv, causal, q_start, q0):
    """mla_bwd_q_kernel: key tiles and the unmasked leading count kfull."""
    kend = min(S_kv, min(q0 + QB, S_q) - 1 + q_start + 1) if causal else S_kv
    nkb = (kend + KT - 1) // KT
    kfull = 0
    if q0 + QB <= S_q:
        kfull = min(nkb, (min(S_kv, q0 + q_start + 1) if causal else S_kv) // KT)
    return nkb, kfull


def test_peeled_loops_stay_in_range_and_unmask_only_visible_tiles():
    visible = lambda q, k, causal, q_start, S_q, S_kv: q < S_q and k < S_kv and (not causal or k <= q + q_start)
    for S_q, S_kv, q_start in itertools.product([1, 3, 40, 64, 65, 128, 129, 300, 2048],
                                                [1, 5, 64, 128, 129, 300, 777, 2048], [0, 2, 200, 776]):
        for causal in (False, True):
            S_qp = (S_q + 63) // 64 * 64
            for k0 in range(0, S_kv, KW):
                qb, nqt, i_lo, i_hi = kv_kernel_bounds(S_q, S_kv, causal, q_start, k0)
                assert 0 <= i_lo <= i_hi <= nqt
                assert nqt == 0 or qb + nqt * QI <= S_qp         # packed rows exist
                if causal and nqt:                               # no visible query before qb
                    assert not visible(qb - 1, k0 + KW - 1, causal, q_start, S_q, S_kv) or qb == 0
                for i in range(i_lo, i_hi):
                    qt = qb + i * QI
                    for q, k in itertools.product((qt, qt + QI - 1), (k0, k0 + KW - 1)):
                        assert visible(q, k, causal, q_start, S_q, S_kv)
            S_kvp = (S_kv + 63) // 64 * 64
            for q0 in range(0, S_q, QB):
                nkb, kfull = q_kernel_bounds(S_q, S_kv, causal, q_start, q0)
                assert 0 <= kfull <= nkb and nkb * KT <= S_kvp   # K, V rows exist
                for kb in range(kfull):
                    for q, k in itertools.product((q0, q0 + QB - 1), (kb * KT, kb * KT + KT - 1)):
                        assert visible(q, k, causal, q_start, S_q, S_kv)
                # every key a query of the block sees lies below nkb * 64
                last_q = min(q0 + QB, S_q) - 1
                top = min(S_kv - 1, last_q + q_start) if causal else S_kv - 1
                assert top < nkb * KT
