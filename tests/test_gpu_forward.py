"""GPU parity of the forward path against the CPU oracle (MI355X only).

Bars: routing indices / counts / permutation bit-exact given identical fp32
logits; fp32 outputs within 1e-5; bf16 outputs within rtol 2e-2 / atol 2e-2
the reference's own GPU tolerances (1e-3 fp32, 1e-2
bf16; tests/test_moe_triton.py:209,226) are tighter or equal on the operator.
"""
import numpy as np
import pytest
import torch

from oracle import moe_ref as R
from oracle import route as RC
from tests import _cases as CS

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _lib():
    import dsmoe._lib as L
    L.load()
    assert torch.cuda.is_available()
    yield


def _ops():
    from dsmoe import ops
    return ops


def _np(t):
    return t.detach().cpu().numpy()


# --------------------------------------------------------------------- gate
@pytest.mark.parametrize("case", [CS.C0, CS.C1.with_tokens(2048), CS.C2.with_tokens(2048), CS.C3.with_tokens(2048),
                                  CS.C3_DECODE], ids=lambda c: c.name)
def test_gate_logits_and_routing_bit_exact(case):
    x, p, _ = CS.make_inputs(case)
    out = _ops().gate_forward(x.to(DEV), p.gate_w.to(DEV), p.gate_bias.to(DEV), case.k, case.route_scale,
                              want_logits=True)
    torch.cuda.synchronize()
    lg = out["logits"].cpu()
    ref_lg = R.gate_logits_ref(x, p.gate_w)
    torch.testing.assert_close(lg, ref_lg, rtol=1e-5, atol=1e-5)
    # routing given identical fp32 logits: the C oracle on the GPU's logits
    idx, w, s, c = RC.route(lg.numpy(), p.gate_bias.numpy(), case.k, case.route_scale)
    assert np.array_equal(_np(out["idx"]), idx)
    assert np.array_equal(_np(out["idx64"]), idx.astype(np.int64))
    assert np.array_equal(_np(out["weights"]), w)
    assert np.array_equal(_np(out["sel_scores"]), s)
    assert np.array_equal(_np(out["counts"]), c)
    np.testing.assert_array_equal(_np(out["weights_x"].float()), torch.from_numpy(w).to(case.dtype).float().numpy())
    margin = RC.min_margin(lg.numpy(), p.gate_bias.numpy(), case.k)
    print(f"[{case.name}] min k/k+1 biased-score margin = {margin:.3e}")
    if case.bias == "skew":
        assert c[0] == case.T and c[1] == case.T


@pytest.mark.parametrize("T,E,k", [(1, 4, 2), (333, 16, 4), (4096, 64, 6), (100, 256, 8), (5, 3, 3)])
def test_route_from_logits_bit_exact(T, E, k):
    g = torch.Generator().manual_seed(T + E)
    logits = torch.randn(T, E, generator=g)
    logits[::7, 1] = logits[::7, 0]                 # planted exact ties
    bias = torch.randn(E, generator=g) * 0.01
    out = _ops().route_from_logits(logits.to(DEV), bias.to(DEV), k, 1.5)
    idx, w, s, c = RC.route(logits.numpy(), bias.numpy(), k, 1.5)
    assert np.array_equal(_np(out["idx"]), idx)
    assert np.array_equal(_np(out["weights"]), w)
    assert np.array_equal(_np(out["sel_scores"]), s)
    assert np.array_equal(_np(out["counts"]), c)


@pytest.mark.parametrize("T,E,k", [(1, 4, 2), (5, 64, 6), (333, 16, 4), (70, 256, 8)])
def test_route_writes_only_the_token_rows(T, E, k):
    """Tokens are routed in batches per wave; the padding slots of a partly
    filled batch must write nothing past row T of any output."""
    from dsmoe import _lib as L
    g = torch.Generator().manual_seed(5 * T + E)
    logits = torch.randn(T, E, generator=g).to(DEV)
    bias = (torch.randn(E, generator=g) * 0.01).to(DEV)
    pad = 8
    idx = torch.full((T + pad, k), -7, dtype=torch.int32, device=DEV)
    idx64 = torch.full((T + pad, k), -7, dtype=torch.int64, device=DEV)
    w = torch.full((T + pad, k), -7.0, device=DEV)
    wx = torch.full((T + pad, k), -7.0, device=DEV)
    sel = torch.full((T + pad, k), -7.0, device=DEV)
    counts = torch.zeros(E, dtype=torch.int32, device=DEV)
    d = L.make_dims(T, 1, E, k, 1, 0, 0, torch.float32, 1.0)
    rc = L.load().dsmoe_route_from_logits(L.ptr(logits), L.ptr(bias), d, L.ptr(idx), L.ptr(idx64), L.ptr(w),
                                          L.ptr(wx), L.ptr(sel), L.ptr(counts), L.stream_ptr(logits.device))
    L.check(rc, "dsmoe_route_from_logits")
    torch.cuda.synchronize()
    for t in (idx, idx64, w, wx, sel):
        assert (t[T:] == -7).all()
    assert int(counts.sum()) == T * k
    ridx, _, _, rc_ = RC.route(logits.cpu().numpy(), bias.cpu().numpy(), k, 1.0)
    assert np.array_equal(_np(idx[:T]), ridx) and np.array_equal(_np(counts), rc_)


# --------------------------------------------------------------------- permute
@pytest.mark.parametrize("T,E,k", [(1, 4, 2), (64, 4, 2), (65, 4, 2), (1000, 16, 4), (8192, 64, 6), (3000, 256, 8),
                                   (8192, 16, 4), (20000, 64, 6)])
def test_permute_bit_exact(T, E, k):
    rng = np.random.default_rng(T * 31 + E)
    if T == 8192 and E == 16:       # C2-like skew: experts 0 and 1 in every token
        idx = np.stack([np.concatenate([[0, 1], rng.permutation(np.arange(2, E))[:k - 2]]) for _ in range(T)])
    else:
        idx = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    idx = idx.astype(np.int32)
    x = torch.randn(T, 48, dtype=torch.bfloat16)
    w = torch.rand(T, k)
    out = _ops().permute(torch.from_numpy(idx).to(DEV), E, x=x.to(DEV), weights=w.to(DEV))
    off, ss, st, sp = RC.permute(idx, E)
    assert np.array_equal(_np(out["offsets"]), off)
    assert np.array_equal(_np(out["sorted_slot"]), ss)
    assert np.array_equal(_np(out["sorted_token"]), st)
    assert np.array_equal(_np(out["slot_pos"]), sp)
    assert np.array_equal(_np(out["counts"]), np.diff(off))
    assert torch.equal(out["x_sorted"].cpu(), x[torch.from_numpy(st).long()])
    assert torch.equal(out["sorted_w"].cpu(), w.reshape(-1)[torch.from_numpy(ss).long()])


@pytest.mark.parametrize("T", [40, 300])   # one rank block (one launch), and several
def test_permute_c_abi_skips_invalid_slots(T):
    """Through the C ABI (ops.permute rejects such ids before the call): a
    slot whose id lies outside [0, E), or repeats a later slot's id in its
    token, is not placed; every other slot lands where a stable (expert,
    token) sort of the placed slots puts it, and offsets and counts count only
    those."""
    import dsmoe._lib as L
    E, k = 8, 3
    rng = np.random.default_rng(T)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
    idx[3, 1] = E + 5
    idx[7, 0] = -2
    idx[11, 0] = idx[11, 2]
    placed = [(t, j) for t in range(T) for j in range(k)
              if 0 <= idx[t, j] < E and idx[t, j] not in idx[t, j + 1:]]
    order = sorted(placed, key=lambda tj: (idx[tj], tj[0]))
    counts = np.bincount([idx[tj] for tj in placed], minlength=E)
    P = len(placed)
    N = T * k
    d = L.make_dims(T, 1, E, k, 1, 0, 0, torch.float32, 1.0)
    lib = L.load()
    ws = torch.empty(lib.dsmoe_permute_workspace_size(d), dtype=torch.uint8, device=DEV)
    gi = torch.from_numpy(idx).to(DEV)
    off = torch.full((E + 1,), -7, dtype=torch.int32, device=DEV)
    ss, st, sp = (torch.full((N,), -7, dtype=torch.int32, device=DEV) for _ in range(3))
    cnt = torch.full((E,), -7, dtype=torch.int32, device=DEV)
    rc = lib.dsmoe_permute(L.ptr(gi), d, L.ptr(off), L.ptr(ss), L.ptr(st), L.ptr(sp), L.ptr(cnt), None, None, None,
                           None, L.ptr(ws), ws.numel(), L.stream_ptr(DEV))
    L.check(rc, "dsmoe_permute")
    assert np.array_equal(_np(off), np.concatenate([[0], np.cumsum(counts)]))
    assert np.array_equal(_np(cnt), counts)
    assert np.array_equal(_np(ss)[:P], [t * k + j for t, j in order])
    assert np.array_equal(_np(st)[:P], [t for t, _ in order])
    assert (_np(ss)[P:] == -7).all()
    spn = _np(sp)
    for pos, (t, j) in enumerate(order):
        assert spn[t * k + j] == pos
    for t, j in ((3, 1), (7, 0), (11, 0)):
        assert spn[t * k + j] == -7


# --------------------------------------------------------------------- grouped operator seam
@pytest.mark.parametrize("T,D,E,I,counts,dtype,tol", [
    (32, 32, 4, 16, [8, 6, 10, 8], torch.float32, 1e-5),        # tests/test_moe_triton.py:194-209 shape
    (64, 48, 4, 24, [16, 14, 18, 16], torch.bfloat16, 2e-2),    # :211-226 shape
    (24, 16, 4, 12, [6, 0, 8, 10], torch.bfloat16, 2e-2),       # :228-242 empty expert
    (8, 768, 20, 384, [0] * 18 + [4, 4], torch.bfloat16, 2e-2), # :244-258 422m shape (no 256 cap here)
    (300, 128, 4, 256, [130, 0, 1, 169], torch.bfloat16, 2e-2), # MFMA path, ragged tiles
    (520, 256, 3, 192, [257, 256, 7], torch.bfloat16, 2e-2),    # MFMA path, N tail (192 = 128 + 64)
])
def test_grouped_operator_vs_oracle(T, D, E, I, counts, dtype, tol):
    x, w1, w2, w3, off, gw = CS.grouped_case(T, D, E, I, counts, dtype, seed=T + D)
    from dsmoe import grouped_moe_dispatch
    with torch.no_grad():
        y = grouped_moe_dispatch(x.to(DEV), w1.to(DEV), w2.to(DEV), w3.to(DEV), gw.to(DEV), off.to(DEV)).cpu()
    ref = R.grouped_moe_ref(x.float(), w1.float(), w2.float(), w3.float(), off, gw.float())
    assert torch.isfinite(y.float()).all()
    torch.testing.assert_close(y.float(), ref, rtol=tol, atol=tol)


# --------------------------------------------------------------------- whole layer
def _golden(golden_dir, name):
    return dict(np.load(golden_dir / name, allow_pickle=False))


def test_layer_matches_reference_golden_c0_fp32(golden_dir):
    from dsmoe import moe_layer
    d = _golden(golden_dir, "c0_fp32.npz")
    t = lambda a: torch.from_numpy(a).to(DEV)
    x = t(d["x"]).reshape(-1, 64)
    with torch.no_grad():
        y, idx, wx, counts = moe_layer(x, t(d["gate_w"]), t(d["gate_bias"]), list(t(d["w1"]).unbind(0)),
                                       list(t(d["w2"]).unbind(0)), list(t(d["w3"]).unbind(0)),
                                       list(t(d["sw1"]).unbind(0)), list(t(d["sw2"]).unbind(0)),
                                       list(t(d["sw3"]).unbind(0)), k=2)
    torch.cuda.synchronize()
    assert np.array_equal(_np(idx), d["last_indices"].reshape(-1, 2))
    assert np.array_equal(_np(counts), d["counts"])
    np.testing.assert_allclose(_np(wx), d["last_weights"].reshape(-1, 2), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(_np(y), d["y"].reshape(-1, 64), rtol=1e-5, atol=1e-5)


def test_layer_matches_reference_golden_c0_bf16(golden_dir):
    from dsmoe import moe_layer
    d = _golden(golden_dir, "c0_bf16_fp32gate.npz")
    bf = lambda a: torch.from_numpy(a.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16).to(DEV)
    t = lambda a: torch.from_numpy(a).to(DEV)
    with torch.no_grad():
        y, idx, wx, counts = moe_layer(bf(d["x_bits"]), t(d["gate_w"]), t(d["gate_bias"]),
                                       list(bf(d["w1_bits"]).unbind(0)), list(bf(d["w2_bits"]).unbind(0)),
                                       list(bf(d["w3_bits"]).unbind(0)), list(bf(d["sw1_bits"]).unbind(0)),
                                       list(bf(d["sw2_bits"]).unbind(0)), list(bf(d["sw3_bits"]).unbind(0)), k=2)
    assert np.array_equal(_np(idx), d["last_indices"])
    y_ref = bf(d["y_bits"]).float().cpu()
    torch.testing.assert_close(y.float().cpu(), y_ref, rtol=2e-2, atol=2e-2)


def _run_layer(case, x, p):
    from dsmoe import moe_layer
    q = CS.params_to(p, DEV)
    with torch.no_grad():
        out = moe_layer(x.to(DEV), q.gate_w, q.gate_bias, q.w1, q.w2, q.w3, q.sw1, q.sw2, q.sw3, k=case.k,
                        route_scale=case.route_scale)
    torch.cuda.synchronize()
    return out


def _layer_raw(case, x, p, training=False):
    """dsmoe_moe_fwd through the C ABI with its fp32 logits output, then the
    layer's own routing buffers read out of its workspace
    (dsmoe_moe_fwd_workspace_offset)."""
    from dsmoe import _lib as L
    lib = L.load()
    q = CS.params_to(p, DEV)
    T, D, E, k = case.T, case.D, case.E, case.k
    d = L.make_dims(T, D, E, k, case.I, case.S, case.I_s, case.dtype, case.route_scale)
    ws = torch.empty(max(256, lib.dsmoe_moe_fwd_workspace_size(d, int(training))), dtype=torch.uint8, device=DEV)
    xd = x.to(DEV).contiguous()
    y = torch.empty(T, D, dtype=case.dtype, device=DEV)
    idx64 = torch.empty(T, k, dtype=torch.int64, device=DEV)
    wx = torch.empty(T, k, dtype=case.dtype, device=DEV)
    counts = torch.empty(E, dtype=torch.int32, device=DEV)
    logits = torch.empty(T, E, dtype=torch.float32, device=DEV)
    arrs = [L.ptr_array(ts) for ts in (q.w1, q.w2, q.w3, q.sw1, q.sw2, q.sw3)]
    print(f"[{case.name}] dsmoe_moe_fwd T={T} D={D} E={E} k={k} training={int(training)}", flush=True)
    rc = lib.dsmoe_moe_fwd(L.ptr(xd), L.ptr(q.gate_w), L.ptr(q.gate_bias), *[a[0] for a in arrs], d, int(training),
                           L.ptr(y), L.ptr(idx64), L.ptr(wx), L.ptr(counts), L.ptr(logits), L.ptr(ws), ws.numel(),
                           L.stream_ptr(DEV))
    L.check(rc, "dsmoe_moe_fwd")
    torch.cuda.synchronize()
    wsc = ws.cpu()

    def buf(which, n, dt):
        off = lib.dsmoe_moe_fwd_workspace_offset(d, int(training), which)
        nb = n * torch.empty((), dtype=dt).element_size()
        return wsc[off:off + nb].view(dt).numpy()

    N = T * k
    return {"y": y.cpu(), "idx64": _np(idx64), "wx": wx.cpu(), "counts": _np(counts), "logits": _np(logits),
            "idx": buf(L.WS_IDX, N, torch.int32).reshape(T, k), "weights": buf(L.WS_WEIGHTS, N, torch.float32).reshape(T, k),
            "sel": buf(L.WS_SEL_SCORES, N, torch.float32).reshape(T, k), "offsets": buf(L.WS_OFFSETS, E + 1, torch.int32),
            "sorted_slot": buf(L.WS_SORTED_SLOT, N, torch.int32), "sorted_token": buf(L.WS_SORTED_TOKEN, N, torch.int32),
            "slot_pos": buf(L.WS_SLOT_POS, N, torch.int32)}


@pytest.mark.parametrize("case,sample,training", [
    (CS.C0, None, False),
    (CS.C1, 512, False),
    (CS.C2, 512, False),
    (CS.C3.with_tokens(1024), None, False),
    (CS.C3, 192, False),
    (CS.C4, 128, True),
    (CS.C3_DECODE, None, False),
    # decode-size calls (few-row GEMM path): one token; a skewed routing that
    # sends every token to two experts (37-row tiles); no shared experts
    (CS.Case("dec_t1", 1, 2048, 64, 1408, 6, 2, 1408, torch.bfloat16), None, False),
    (CS.Case("dec_t37_skew", 37, 512, 8, 256, 2, 1, 384, torch.bfloat16, "skew"), None, False),
    (CS.Case("dec_t64_noshared", 64, 1024, 16, 512, 4, 0, 0, torch.bfloat16, "normal"), None, False),
    # three shared experts (the down projection sums three K segments) and
    # inter widths with N % 8 == 4: the register-staged MFMA kernel
    # (gemm_mfma_kernel) instead of the quad-wave one
    (CS.Case("s3_i132", 512, 256, 8, 132, 2, 3, 100, torch.bfloat16, "normal"), None, False),
    (CS.Case("s3_i132_train", 512, 256, 8, 132, 2, 3, 100, torch.bfloat16, "normal"), None, True),
], ids=lambda v: getattr(v, "name", str(v)))
def test_layer_forward_vs_oracle(case, sample, training):
    """Every config at full size.  The layer's own fp32 logits (K-split gate
    and routing kernel at T <= 4096, fused gate above) are within 1e-5 of the
    fp32 oracle; given those logits, the C oracle reproduces the layer's expert
    ids, fp32 weights, selected scores, counts and its sorted order (offsets,
    sorted slots and tokens, inverse) bit for bit.  The output is checked on a
    seeded token sample: each token's output depends only on that token's row
    and the weights (the layer is token-separable), so the oracle on the
    sampled rows is exact for them."""
    x, p, _ = CS.make_inputs(case)
    out = _layer_raw(case, x, p, training)
    lg = out["logits"]
    np.testing.assert_allclose(lg, R.gate_logits_ref(x, p.gate_w).numpy(), rtol=1e-5, atol=1e-5)
    ridx, rw, rs, rc = RC.route(lg, p.gate_bias.numpy(), case.k, case.route_scale)
    print(f"[{case.name}] min k/k+1 margin on the layer's logits {RC.min_margin(lg, p.gate_bias.numpy(), case.k):.3e}")
    assert np.array_equal(out["idx"], ridx)
    assert np.array_equal(out["idx64"], ridx.astype(np.int64))
    assert np.array_equal(out["weights"], rw)
    assert np.array_equal(out["sel"], rs)
    assert np.array_equal(out["counts"], rc)
    np.testing.assert_array_equal(out["wx"].float().numpy(), torch.from_numpy(rw).to(case.dtype).float().numpy())
    off, ss, st, sp = RC.permute(ridx, case.E)
    assert np.array_equal(out["offsets"], off)
    assert np.array_equal(out["sorted_slot"], ss)
    assert np.array_equal(out["sorted_token"], st)
    assert np.array_equal(out["slot_pos"], sp)
    rows = torch.arange(case.T) if sample is None else \
        torch.randperm(case.T, generator=torch.Generator().manual_seed(11))[:sample]
    y_ref = R.moe_forward_ref(x[rows], p, case.k, case.route_scale)
    tol = 1e-5 if case.dtype == torch.float32 else 2e-2
    torch.testing.assert_close(out["y"][rows].float(), y_ref.float(), rtol=tol, atol=tol)
    if case.bias == "skew":
        assert rc[0] == case.T and rc[1] == case.T and rc.sum() == case.N


def test_layer_forward_is_deterministic():
    case = CS.C1.with_tokens(2048)
    x, p, _ = CS.make_inputs(case)
    y1 = _run_layer(case, x, p)[0]
    y2 = _run_layer(case, x, p)[0]
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


def test_module_drop_in_forward_and_side_state():
    from dsmoe import DeepSeekMoE
    case = CS.C1.with_tokens(1024)
    x, p, _ = CS.make_inputs(case)
    m = CS.load_module(case, p, DEV, DeepSeekMoE)
    with torch.no_grad():
        y = m(x.to(DEV).view(4, 256, case.D))
    assert y.shape == (4, 256, case.D) and y.dtype == case.dtype
    y_ref, w_ref, i_ref = R.moe_forward_ref(x, p, case.k, return_routing=True)
    torch.testing.assert_close(y.reshape(-1, case.D).float().cpu(), y_ref.float(), rtol=2e-2, atol=2e-2)
    assert torch.equal(m._last_indices.cpu(), i_ref)
    assert m._last_weights.dtype == case.dtype
    bl = m.get_load_balance_loss()
    assert abs(bl.item() - R.balance_loss_ref(w_ref, i_ref, case.E).item()) < 1e-3
    counts = torch.bincount(i_ref.flatten(), minlength=case.E)
    b0 = m.gate.bias.detach().cpu().clone()
    m.update_gate_bias(speed=0.01)
    assert torch.equal(m.gate.bias.cpu(), R.update_bias_ref(b0, counts, 0.01))
    assert torch.equal(m._stacked_w1[3].cpu(), p.w1[3]) and torch.equal(m._shared_w1[0].cpu(), p.sw1[0])


@pytest.mark.parametrize("training", [False, True])
def test_dispatch_key_triton_grouped_equals_stacked(training):
    """models/_triton_dispatch.py:13-35 and models/moe.py:61,87-99: a layer
    built with moe_dispatch='triton_grouped' and one built with 'stacked' from
    the same state_dict give the same result (the reference's own check,
    tests/test_moe_triton.py:162-180, at atol 1e-5).  Here both keys run the
    same HIP kernels, so outputs, routing and gradients are bitwise equal, and
    both match the oracle; the config rewrite of enforce_triton_env_var leaves
    the layer's results unchanged either way."""
    from dsmoe import DeepSeekMoE, enforce_triton_env_var
    case = CS.C1.with_tokens(768)
    x, p, dy = CS.make_inputs(case, with_dy=True)
    stacked = CS.load_module(case, p, DEV, lambda cfg: DeepSeekMoE(dict(cfg, moe_dispatch="stacked")))
    triton = DeepSeekMoE(dict(case.config(), moe_dispatch="triton_grouped")).to(DEV, case.dtype)
    triton.gate.float()
    triton.load_state_dict(stacked.state_dict())
    mods = {"stacked": stacked, "triton_grouped": triton}
    for key, m in mods.items():
        assert m.moe_dispatch == key
    rewritten = dict(case.config(), moe_dispatch="triton_grouped")
    enforce_triton_env_var(rewritten, lambda _msg: None)
    outs = {}
    for key, m in mods.items():
        xin = x.clone().to(DEV).requires_grad_(training)
        with torch.set_grad_enabled(training):
            y = m(xin)
            if training:
                (y.float() * dy.to(DEV).float()).sum().backward()
        torch.cuda.synchronize()
        outs[key] = (y.detach(), m._last_indices.clone(), xin.grad if training else None,
                     {n: q.grad.clone() for n, q in m.named_parameters() if training})
    (ys, is_, gs, ps), (yt, it, gt, pt) = outs["stacked"], outs["triton_grouped"]
    assert torch.equal(ys.view(torch.int16), yt.view(torch.int16)) and torch.equal(is_, it)
    if training:
        assert torch.equal(gs, gt)
        for n in ps:
            assert torch.equal(ps[n], pt[n]), n
    y_ref, _, i_ref = R.moe_forward_ref(x, p, case.k, return_routing=True)
    assert torch.equal(is_.cpu(), i_ref)
    torch.testing.assert_close(ys.float().cpu(), y_ref.float(), rtol=2e-2, atol=2e-2)
    assert rewritten["moe_dispatch"] in ("stacked", "triton_grouped")


def test_module_update_bias_kats_on_device():
    """tests/test_models.py:325-345 and :760-777 on the device kernel."""
    from dsmoe import AuxLossFreeGate
    gate = AuxLossFreeGate({"dim": 8, "n_activated_experts": 2, "n_routed_experts": 4,
                            "bias_upper_threshold": 0.10, "bias_lower_threshold": 0.10}).to(DEV)
    gate.update_bias(torch.tensor([10, 5, 5, 0], device=DEV), speed=0.01)
    assert torch.equal(gate.bias.cpu(), torch.tensor([-0.01, 0.0, 0.0, 0.01]))
    gate.bias.zero_()
    gate.update_bias(torch.tensor([256, 0, 0, 0], device=DEV), speed=0.1)
    assert torch.equal(gate.bias.cpu(), torch.tensor([-0.1, 0.1, 0.1, 0.1]))


def test_grouped_operator_promotes_like_the_reference():
    """models/moe_triton.py:525 returns out * sorted_weights.unsqueeze(-1):
    fp32 gate weights over a bf16 expert output give an fp32 result (the
    product of the bf16-rounded output and the fp32 weight), with and without
    autograd."""
    from dsmoe import grouped_moe_dispatch
    x, w1, w2, w3, off, _ = CS.grouped_case(300, 128, 4, 256, [130, 0, 1, 169], torch.bfloat16, seed=5)
    gw = torch.rand(300, generator=torch.Generator().manual_seed(6)) * 0.1          # fp32
    d = lambda t: t.to(DEV)
    ones = torch.ones(300, dtype=torch.bfloat16)
    with torch.no_grad():
        y = grouped_moe_dispatch(d(x), d(w1), d(w2), d(w3), d(gw), d(off))
        out = grouped_moe_dispatch(d(x), d(w1), d(w2), d(w3), d(ones), d(off))   # unweighted, bf16
    assert y.dtype == torch.float32 and out.dtype == torch.bfloat16
    assert torch.equal(y, out.float() * d(gw).unsqueeze(-1))
    xl = d(x).requires_grad_(True)
    yg = grouped_moe_dispatch(xl, d(w1), d(w2), d(w3), d(gw), d(off))
    assert yg.dtype == torch.float32 and torch.equal(yg.detach(), y)
    ref = R.grouped_moe_ref(x.float(), w1.float(), w2.float(), w3.float(), off, gw)
    torch.testing.assert_close(y.cpu(), ref, rtol=2e-2, atol=2e-2)


def test_expert_module_forward():
    """Expert.forward (models/moe.py:40-49) as a one-group call of the grouped
    operator, against the SwiGLU on the oracle's arithmetic."""
    from dsmoe import Expert
    g = torch.Generator().manual_seed(21)
    m = Expert(256, 192)
    with torch.no_grad():
        for lin in (m.w1, m.w2, m.w3):
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=g) * 0.05)
    x = torch.randn(3, 70, 256, generator=g)
    m = m.to(DEV, torch.bfloat16)
    with torch.no_grad():
        y = m(x.to(DEV, torch.bfloat16))
    assert y.shape == x.shape and y.dtype == torch.bfloat16
    xb = x.to(torch.bfloat16).float().reshape(-1, 256)
    w1, w2, w3 = (lin.weight.detach().float().cpu() for lin in (m.w1, m.w2, m.w3))
    ref = (torch.nn.functional.silu(xb @ w1.t()) * (xb @ w3.t())) @ w2.t()
    torch.testing.assert_close(y.float().cpu().reshape(-1, 256), ref, rtol=2e-2, atol=2e-2)


def test_update_bias_with_fractional_counts():
    """Floating counts (e.g. averaged over steps) run the fp32 band rule of
    models/moe.py:21-27 without truncation."""
    from dsmoe import AuxLossFreeGate
    gate = AuxLossFreeGate({"dim": 8, "n_activated_experts": 2, "n_routed_experts": 6,
                            "bias_upper_threshold": 0.10, "bias_lower_threshold": 0.10}).to(DEV)
    counts = torch.tensor([0.9, 0.5, 0.6, 0.4, 0.7, 0.3])   # mean 0.5667; every count 1e-2 or more from a band edge
    b0 = torch.tensor([0.1, -0.2, 0.0, 0.05, 0.0, 0.3])
    gate.bias.copy_(b0.to(DEV))
    gate.update_bias(counts.to(DEV), speed=0.01)
    assert torch.equal(gate.bias.cpu(), R.update_bias_ref(b0, counts, 0.01))
    truncated = R.update_bias_ref(b0, counts.to(torch.int32), 0.01)
    assert not torch.equal(gate.bias.cpu(), truncated)             # integer truncation would differ
