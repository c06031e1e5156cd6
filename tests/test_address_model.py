"""Every global address the grouped GEMM kernels compute stays inside its
allocation (CPU only; tests/_addr_model.py restates the loaders' and
epilogues' index arithmetic).

The layer's descriptors are rebuilt the way csrc/api.hip builds them
(dsmoe_moe_fwd: gemm1 routed + shared, gemm2 routed + shared, the decode
few-row path; dsmoe_moe_bwd: dh, dx, dW1|dW3, dW2 and the shared-expert
versions), with routings drawn like the gate's (k distinct experts per token)
at every BASELINE config, the C2 skew, ragged and empty experts, a single
token, and inter widths that leave a partial column tile.  A loader that read
one row past its slab (the fault a K-major loader once had: its parity offset
counted twice) fails here.
"""
import numpy as np
import pytest

from tests import _addr_model as M


def _routing(T, E, k, skew=False, seed=0, empty=0):
    rng = np.random.default_rng(seed)
    live = E - empty
    idx = np.empty((T, k), np.int64)
    for t in range(T):
        if skew:
            rest = rng.permutation(np.arange(2, live))[:k - 2]
            idx[t] = np.concatenate([[0, 1], rest])
        else:
            idx[t] = rng.permutation(live)[:k]
    flat = idx.reshape(-1)
    order = np.argsort(flat, kind="stable")
    counts = np.bincount(flat, minlength=E)
    sorted_token = (order // k).astype(np.int64)
    sorted_slot = order.astype(np.int64)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    return counts, sorted_token, sorted_slot, offsets


def _bufs(prefix, n, nbytes):
    return [M.Buf(f"{prefix}[{i}]", nbytes) for i in range(n)]


def _forward(rec, T, D, E, k, I, S, I_s, training, counts, sorted_token, sorted_slot):
    """dsmoe_moe_fwd's two GEMM launches (csrc/api.hip)."""
    N = T * k
    x = M.Buf("x", T * D * 2)
    w1, w3, w2 = _bufs("w1", E, I * D * 2), _bufs("w3", E, I * D * 2), _bufs("w2", E, D * I * 2)
    s1, s3, s2 = _bufs("sw1", S, I_s * D * 2), _bufs("sw3", S, I_s * D * 2), _bufs("sw2", S, D * I_s * 2)
    h = M.Buf("h", N * I * 2)
    gs_ = M.Buf("g", N * I * 2) if training else None
    us_ = M.Buf("u", N * I * 2) if training else None
    hs = M.Buf("hs", T * S * I_s * 2)
    o_sorted = M.Buf("o_sorted", N * D * 2)
    shared_out = M.Buf("shared_out", T * D * 2)
    decode = not training and T <= M.SK_BM
    bm = M.SK_BM if decode else M.QW_BM
    sched = M.routed_schedule(counts, bm)
    bound = M.sched_bound(N, E, bm)
    assert len(sched) <= bound, "schedule longer than its workspace bound"
    g1 = M.Gemm(N=I, K=D, A=x, lda=D, a_rows=T, B0=w1, B1=w3, ldb=D, kseg=D, nseg=1, C=h, ldc=I, sched=sched,
                a_map=sorted_token, Gs=gs_, Us=us_, m_tiles_bound=bound)
    g2 = M.Gemm(N=D, K=I, A=h, lda=I, a_rows=N, B0=w2, B1=None, ldb=I, kseg=I, nseg=1, C=o_sorted, ldc=D,
                sched=sched, m_tiles_bound=bound)
    d1 = d2 = None
    if S:
        d1 = M.Gemm(N=I_s, K=D, A=x, lda=D, a_rows=T, B0=s1, B1=s3, ldb=D, kseg=D, nseg=1, C=hs, ldc=S * I_s,
                    dense_rows=T, groups=S, c_group_col=I_s,
                    Gs=M.Buf("gs", T * S * I_s * 2) if training else None,
                    Us=M.Buf("us", T * S * I_s * 2) if training else None)
        d2 = M.Gemm(N=D, K=S * I_s, A=hs, lda=S * I_s, a_rows=T, B0=s2, B1=None, ldb=I_s, kseg=I_s, nseg=S,
                    C=shared_out, ldc=D, dense_rows=T, groups=1)
    launched = 0
    for gr, gd, sw in ((g1, d1, True), (g2, d2, False)):
        if decode:
            gr_ = M.Gemm(**{**gr.__dict__, "Gs": None, "Us": None})
            assert M.sk_ok(gr_), "decode shapes take the few-row kernel"
            if gd is not None and M.sk_ok(gd):
                launched += M.sk_launch(rec, gr_, sw, gd)
            else:
                launched += M.sk_launch(rec, gr_, sw)
        elif M.qp_ok(gr):
            if gd is not None and M.qp_ok(gd):
                launched += M.qp_launch(rec, gr, sw, gd)
            else:
                launched += M.qp_launch(rec, gr, sw)
                if gd is not None and M.qp_ok(gd):
                    launched += M.qp_launch(rec, gd, sw)
    return launched


def _backward(rec, T, D, E, k, I, S, I_s, counts, sorted_token, sorted_slot, offsets, dw_f32=False):
    """dsmoe_moe_bwd's backward GEMMs that take xgemm_q_kernel (csrc/api.hip);
    dw_f32: dsmoe_moe_bwd_ex with fp32 weight gradients (4-byte dW buffers)."""
    N = T * k
    we = 4 if dw_f32 else 2
    dy = M.Buf("dy", T * D * 2)
    x = M.Buf("x", T * D * 2)
    w1, w3, w2 = _bufs("w1", E, I * D * 2), _bufs("w3", E, I * D * 2), _bufs("w2", E, D * I * 2)
    w13 = [b for e in range(E) for b in (w1[e], w3[e])]
    dw1, dw3, dw2 = _bufs("dw1", E, I * D * we), _bufs("dw3", E, I * D * we), _bufs("dw2", E, D * I * we)
    g_, u_, h = M.Buf("g", N * I * 2), M.Buf("u", N * I * 2), M.Buf("h", N * I * 2)
    x_sorted = M.Buf("x_sorted", N * D * 2)
    dgdu = M.Buf("dgdu", N * 2 * I * 2)
    dx_slots = M.Buf("dx_slots", N * D * 2)
    dy_w = M.Buf("dy_w", N * D * 2)
    sched = M.routed_schedule(counts, M.XQ_BM)
    gemms = [
        ("dh", M.XGemm(mode=M.XS_ROUTED, M=0, N=I, K=D, a_km=False, A=dy, lda=D, a_map=sorted_token,
                       b_weights=True, Btab=w2, ldb=I, kseg=D, sched=sched, C=dgdu, ldc=2 * I, du_off=I,
                       swiglu_bwd=True, Gs=g_, Us=u_, ld_gu=I)),
        ("dx", M.XGemm(mode=M.XS_ROUTED, M=0, N=D, K=2 * I, a_km=False, A=dgdu, lda=2 * I, b_weights=True,
                       Btab=w13, ldb=D, kseg=I, nseg=2, sched=sched, C=dx_slots, ldc=D, c_map=sorted_slot)),
        ("dW13", M.XGemm(mode=M.XS_WGRAD, M=2 * I, N=D, K=N, a_km=True, A=dgdu, lda=2 * I, b_weights=False,
                         Bact=x_sorted, ldb=D, groups=E, k_off=offsets, Ctab0=dw1, Ctab1=dw3, msplit=I, ldc=D,
                         c_f32=dw_f32)),
        ("dW2", M.XGemm(mode=M.XS_WGRAD, M=D, N=I, K=N, a_km=True, A=dy_w, lda=D, b_weights=False, Bact=h, ldb=I,
                        groups=E, k_off=offsets, Ctab0=dw2, Ctab1=dw2, msplit=D, ldc=I, c_f32=dw_f32)),
    ]
    if S:
        SIs = S * I_s
        sw1, sw3, sw2 = _bufs("sw1", S, I_s * D * 2), _bufs("sw3", S, I_s * D * 2), _bufs("sw2", S, D * I_s * 2)
        dsw1, dsw3, dsw2 = (_bufs("dsw1", S, I_s * D * we), _bufs("dsw3", S, I_s * D * we),
                            _bufs("dsw2", S, D * I_s * we))
        gs_, us_, hs = M.Buf("gs", T * SIs * 2), M.Buf("us", T * SIs * 2), M.Buf("hs", T * SIs * 2)
        dgdu_s = M.Buf("dgdu_s", T * 2 * SIs * 2)
        ks13 = M.xgemm_pick_ksplit(M.xgemm_tiles(2 * I_s, D, S), T)
        ks2 = M.xgemm_pick_ksplit(M.xgemm_tiles(D, I_s, S), T)
        part = M.Buf("part", 4 * max(ks13 * 2 * I_s if ks13 > 1 else 0, ks2 * I_s if ks2 > 1 else 0) * S * D)
        gemms += [
            ("dh_s", M.XGemm(mode=M.XS_DENSE, M=0, N=I_s, K=D, a_km=False, A=dy, lda=D, b_weights=True, Btab=sw2,
                             ldb=I_s, kseg=D, dense_rows=T, groups=S, C=dgdu_s, ldc=2 * SIs, c_group_col=2 * I_s,
                             du_off=I_s, swiglu_bwd=True, Gs=gs_, Us=us_, ld_gu=SIs, gu_group_col=I_s)),
            ("dW13_s", M.XGemm(mode=M.XS_WGRAD, M=2 * I_s, N=D, K=T, a_km=True, A=dgdu_s, lda=2 * SIs,
                               a_col=2 * I_s, b_weights=False, Bact=x, ldb=D, groups=S, Ctab0=dsw1, Ctab1=dsw3,
                               msplit=I_s, ldc=D, ksplit=ks13, part=part, c_f32=dw_f32)),
            ("dW2_s", M.XGemm(mode=M.XS_WGRAD, M=D, N=I_s, K=T, a_km=True, A=dy, lda=D, b_weights=False, Bact=hs,
                              ldb=SIs, b_col=I_s, groups=S, Ctab0=dsw2, Ctab1=dsw2, msplit=D, ldc=I_s,
                              ksplit=ks2, part=part, c_f32=dw_f32)),
        ]
        # the shared dx sums 2S K segments: two as they are, more through
        # the stacked copy of the W1 / W3 blocks (one segment)
        tab = ([b for s in range(S) for b in (sw1[s], sw3[s])] if S <= 1
               else [M.Buf("sw13_stack", 2 * SIs * D * 2)])
        gemms.append(("dx_s", M.XGemm(mode=M.XS_DENSE, M=0, N=D, K=2 * SIs, a_km=False, A=dgdu_s, lda=2 * SIs,
                                      b_weights=True, Btab=tab, ldb=D, kseg=I_s if S <= 1 else 2 * SIs,
                                      nseg=2 * S if S <= 1 else 1, dense_rows=T, groups=1,
                                      C=M.Buf("dx_shared", T * D * 2), ldc=D)))
    n = 0
    for name, g in gemms:
        if M.xq_ok(g):
            n += M.xq_launch(rec, g, name)
    return n


# name: T, D, E, k, I, S, I_s, routing
CONFIGS = {
    "c0_bf16": (1024, 64, 4, 2, 128, 1, 128, {}),
    "c1": (8192, 1024, 16, 4, 512, 1, 1024, {}),
    "c2_skew": (8192, 1024, 16, 4, 512, 1, 1024, {"skew": True}),
    "c3": (8192, 2048, 64, 6, 1408, 2, 1408, {}),
    "c3_decode": (64, 2048, 64, 6, 1408, 2, 1408, {}),
    "c4": (16384, 2048, 64, 6, 1408, 2, 1408, {}),
    "one_token": (1, 2048, 64, 6, 1408, 2, 1408, {}),
    "ragged_empty": (777, 512, 16, 3, 192, 1, 320, {"empty": 5}),
    "wide_e256": (3000, 256, 256, 8, 64, 0, 0, {}),
    "decode_skew": (37, 512, 8, 2, 256, 1, 384, {"skew": True}),
}


@pytest.mark.parametrize("name", sorted(CONFIGS))
@pytest.mark.parametrize("training", [False, True])
def test_forward_gemm_addresses_in_bounds(name, training):
    T, D, E, k, I, S, I_s, kw = CONFIGS[name]
    counts, st, ss, _ = _routing(T, E, k, seed=T + E, **kw)
    rec = M.Recorder()
    n = _forward(rec, T, D, E, k, I, S, I_s, training, counts, st, ss)
    assert n > 0
    # the tiles cover the routed rows: h (gemm1) and o_sorted (gemm2) are written up to their last row
    if not (not training and T <= M.SK_BM):
        assert rec.ext["h"][1] == T * k * I * 2
    assert rec.ext["o_sorted"][1] == T * k * D * 2


@pytest.mark.parametrize("name", ["c0_bf16", "c1", "c2_skew", "c3", "c4", "ragged_empty", "wide_e256", "one_token"])
@pytest.mark.parametrize("dw_f32", [False, True])
def test_backward_gemm_addresses_in_bounds(name, dw_f32):
    T, D, E, k, I, S, I_s, kw = CONFIGS[name]
    counts, st, ss, off = _routing(T, E, k, seed=T + E + 1, **kw)
    rec = M.Recorder()
    assert _backward(rec, T, D, E, k, I, S, I_s, counts, st, ss, off, dw_f32=dw_f32) > 0
    if dw_f32:   # every fp32 gradient row is written to its last byte
        assert rec.ext["dw1[0]"][1] == I * D * 4 and rec.ext["dw2[0]"][1] == D * I * 4


def test_model_catches_a_slab_overrun():
    """The model's own check, on the fault a K-major loader once had: the
    lane's base row already held the parity offset and the per-load stride
    added it again, so odd loads read two rows further; in an expert's last
    slab of W2 (the dh GEMM's weight operand, which has no zero-block
    redirect) that is past the allocation, and the model reports it."""
    T, D, E, k, I, S, I_s, kw = CONFIGS["c1"]
    counts, st, ss, off = _routing(T, E, k, seed=5)
    orig = M.xq_tile

    def faulty(rec, g, grp, row0, rows, n_tile, kbeg, kend, split, what):
        if g.b_weights and g.nseg == 1:
            i = np.arange(M.XQ_LD)[None, None, :]
            kr = np.arange(4)[:, None, None] * 16 + (np.arange(64)[None, :, None] >> 5)
            k0 = kbeg + (M.cdiv(kend - kbeg, M.XQ_BK) - 1) * M.XQ_BK
            krow = k0 + kr + 2 * i + 2 * (i & 1)            # the doubled parity offset
            blk = g.Btab[grp]
            rec.touch(blk, 2 * krow * g.ldb, 2 * krow * g.ldb + 16, what + " B W (planted)")
        return orig(rec, g, grp, row0, rows, n_tile, kbeg, kend, split, what)

    M.xq_tile = faulty
    try:
        with pytest.raises(M.Violation, match="planted"):
            _backward(M.Recorder(), T, D, E, k, I, S, I_s, counts, st, ss, off)
    finally:
        M.xq_tile = orig


def test_routed_item_order_is_a_permutation():
    """qp_tile's item order inside an expert's M tiles: every (M tile,
    N tile) once, N tile by N tile when the expert has fewer M tiles than
    there are N tiles, M tile by M tile otherwise."""
    sched = M.routed_schedule([600, 0, 40, 1300, 256], 256)  # 3, 0, 1, 6, 1 M tiles
    nt = 4
    items = [M.routed_item(sched, lin, nt) for lin in range(len(sched) * nt)]
    assert sorted(items) == [(m, n) for m in range(len(sched)) for n in range(nt)]
    # expert 0 (3 M tiles < 4 N tiles): N-major inside its item range
    assert items[:6] == [(0, 0), (1, 0), (2, 0), (0, 1), (1, 1), (2, 1)]
    # expert 3 (6 M tiles >= 4 N tiles): M-major, as enumerated
    first3 = 4 * 4  # items before expert 3: 3 + 1 M tiles
    assert items[first3:first3 + 5] == [(4, 0), (4, 1), (4, 2), (4, 3), (5, 0)]
