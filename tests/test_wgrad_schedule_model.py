"""Schedule of the persistent weight-gradient kernel (csrc/gemm_xq.hip,
xgemm_wgrad_p_kernel), restated on the CPU (no kernel launches): for every
workgroup, the tiles it walks, the ring slab each load fills and each slab
computes, the point where the loader switches to the next tile, and the
vector-memory waits.  Checked: every output tile is computed exactly once;
every ring slab a tile computes was loaded from that tile's own K slab; the
loads past the last tile re-read its last slab; and at every slab's barrier
this wave's loads of the next ring slab are complete under the kernel's
waits (wait_vm<N> leaves the N youngest operations of the wave pending;
loads complete in issue order, as the slab loop of xgemm_q_kernel assumes).
"""
import itertools
import random

import pytest

XQ_LD = 8   # direct loads per wave, operand and slab


def cdiv(a, b):
    return -(-a // b)


def xtile_at(M, N, groups, k_off, blk):
    """xtile_at (csrc/gemm_tile.h), XS_WGRAD without split-K."""
    n_tiles, tpg = cdiv(N, 256), cdiv(M, 256)
    total = tpg * groups * n_tiles
    per = cdiv(total, 8)
    j = blk >> 3
    if j >= per:
        return None
    lin = (blk & 7) * per + j
    if lin >= total:
        return None
    mt, n_tile = divmod(lin, n_tiles)
    grp = mt // tpg
    return dict(lin=lin, grp=grp, kbeg=k_off[grp], kend=k_off[grp + 1])


def nk_of(t):
    """xq_wgrad_nk: at least two slabs."""
    return max(2, cdiv(t["kend"] - t["kbeg"], 64) if t["kend"] > t["kbeg"] else 0)


class Wave:
    """One wave's vector-memory operations and what the waits guarantee."""

    def __init__(self):
        self.pending = []    # ring slab of each pending operation (None: store), oldest first
        self.issued = {}     # ring slab -> loads issued

    def load(self, operand, ring):
        self.pending.append(ring)
        self.issued[ring] = self.issued.get(ring, 0) + 1

    def store(self, n):
        self.pending += [None] * n

    def wait_vm(self, n):
        if len(self.pending) > n:
            self.pending = self.pending[len(self.pending) - n:]

    def complete(self, ring):
        return ring not in self.pending and self.issued.get(ring, 0) == 2 * XQ_LD


def run_workgroup(b, grid, M, N, groups, k_off, f32):
    """xgemm_wgrad_p_kernel for block b; returns {tile lin: (b, ring of slab 0)}."""
    G, vb = grid, b
    cur = xtile_at(M, N, groups, k_off, vb)
    if cur is None:
        return {}
    nxt = xtile_at(M, N, groups, k_off, vb + G)
    more = nxt is not None
    L = (cur, 0)                 # loader: (tile, ring index of its slab 0)
    loaded = {}                  # ring slab -> (tile lin, K slab, past the tile)
    w = Wave()

    def issue(operand, ring):
        t, g0 = L
        loc = ring - g0
        assert loc >= 0
        loaded.setdefault(ring, set()).add((t["lin"], min(loc, nk_of(t) - 1), loc >= nk_of(t)))
        for _ in range(XQ_LD):
            w.load(operand, ring)

    # prologue: A(0), B(0), A(1), B(1); wait_vm<0>; barrier
    for ring in (0, 1):
        issue("A", ring)
        issue("B", ring)
    w.wait_vm(0)
    assert w.complete(0)
    out = {}
    gs, kb = 0, 0
    while True:
        nk = nk_of(cur)

        def slab(kb, first):
            got = loaded[kb]
            assert got == {(cur["lin"], kb - gs, False)}, (b, kb, got)
            issue("B", kb + 2)                   # steps 0 and 1
            if not first:
                w.wait_vm(XQ_LD)
            assert w.complete(kb + 1), (b, kb, first)   # the barrier
            issue("A", kb + 2)                   # steps 2 and 3

        if more and nk == 2:
            L = (nxt, gs + nk)
        slab(kb, True)
        kb += 1
        while kb - gs < nk:
            if more and kb - gs == nk - 2:
                L = (nxt, gs + nk)
            slab(kb, False)
            kb += 1
        assert cur["lin"] not in out
        out[cur["lin"]] = (b, gs)
        nn = xtile_at(M, N, groups, k_off, vb + 2 * G) if more else None
        w.wait_vm(0)                             # before the epilogue's stores
        w.store(64 if f32 else 32)
        if not more:
            break
        gs, cur, nxt, more, vb = kb, nxt, nn, nn is not None, vb + G
    for ring in (kb, kb + 1):                    # loads past the last tile
        assert loaded[ring] == {(cur["lin"], nk_of(cur) - 1, True)}
    return out


def run(M, N, groups, k_off, ncu, f32=False):
    total = cdiv(M, 256) * groups * cdiv(N, 256)
    grid = min(8 * cdiv(total, 8), 8 * cdiv(ncu, 8))   # launch_xgemm_q
    seen = {}
    for b in range(grid):
        for lin, v in run_workgroup(b, grid, M, N, groups, k_off, f32).items():
            assert lin not in seen
            seen[lin] = v
    assert sorted(seen) == list(range(total))


SHAPES = [(2816, 2048, 64), (2048, 1408, 64), (384, 256, 8), (256, 384, 5), (640, 256, 3),
          (2048, 1024, 16), (1024, 512, 16), (8, 8, 1), (512, 2048, 2)]


@pytest.mark.parametrize("M,N,groups", SHAPES)
def test_every_tile_once_from_its_own_slabs_and_loads_waited(M, N, groups):
    rng = random.Random(M * 7 + N + groups)
    for trial in range(3):
        rows = [rng.choice([0, 1, 3, 63, 64, 65, 127, 128, 129, 700, 1536]) for _ in range(groups)]
        k_off = list(itertools.accumulate([0] + rows))
        for ncu, f32 in ((256, False), (80, True), (8, False)):
            run(M, N, groups, k_off, ncu, f32)


def test_c4_routing_shape():
    # C4 at 256 CUs: 64 experts of about 1536 rows, dW1 | dW3 and dW2
    rng = random.Random(4)
    rows = [1536 + rng.randint(-120, 120) for _ in range(64)]
    k_off = list(itertools.accumulate([0] + rows))
    run(2816, 2048, 64, k_off, 256)
    run(2048, 1408, 64, k_off, 256)
