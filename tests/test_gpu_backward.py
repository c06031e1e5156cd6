"""GPU parity of the backward pass (dx, dW_gate, dW of every expert).

fp32: against gradients written by the reference layer itself (golden
fixtures), tolerance 1e-5 relative to the gradient scale.

bf16: against the oracle's autograd in bf16 (the reference's own rounding
points) with rtol/atol 2e-2.  Gradients that are sums over tokens (dW_gate and
every expert dW) carry absolute rounding noise that grows with the sum, and
the bf16 reference itself misses an elementwise 2e-2 bound against an fp32 run
on those (hundreds of elements at C1/C3 shapes, mostly where terms cancel).
For them atol is 2e-2 times the tensor's max magnitude.  All bf16 results are
also held to an accuracy bar: their relative L2 error against the fp32 oracle
(same bf16-valued inputs, fp32 arithmetic) must not exceed twice the bf16
reference's own.  Full C4 size: token-separable dx on a token sample, slices
of the weight gradients of three routed and both shared experts against the
fp32 oracle on those experts' rows, finiteness; determinism at C3 shape.
"""
import numpy as np
import pytest
import torch

from oracle import moe_ref as R
from tests import _cases as CS

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _leaf(t):
    return t.detach().clone().to(DEV).requires_grad_(True)


def _run(x, gw, gb, w1, w2, w3, sw1, sw2, sw3, k, rs, dy):
    from dsmoe import moe_layer
    leaves = dict(x=_leaf(x), gw=_leaf(gw), w1=[_leaf(t) for t in w1], w2=[_leaf(t) for t in w2],
                  w3=[_leaf(t) for t in w3], sw1=[_leaf(t) for t in sw1], sw2=[_leaf(t) for t in sw2],
                  sw3=[_leaf(t) for t in sw3])
    y, idx, wx, counts = moe_layer(leaves["x"], leaves["gw"], gb.to(DEV), leaves["w1"], leaves["w2"], leaves["w3"],
                                   leaves["sw1"], leaves["sw2"], leaves["sw3"], k=k, route_scale=rs)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    g = lambda ts: [t.grad.detach().cpu() for t in ts]
    return {"y": y.detach().cpu(), "dx": leaves["x"].grad.cpu(), "dgate_w": leaves["gw"].grad.cpu(),
            "dw1": g(leaves["w1"]), "dw2": g(leaves["w2"]), "dw3": g(leaves["w3"]),
            "dsw1": g(leaves["sw1"]), "dsw2": g(leaves["sw2"]), "dsw3": g(leaves["sw3"]), "idx": idx.cpu()}


def _close(a, b, rtol, atol, what):
    a, b = a.float(), b.float()
    err = (a - b).abs().max().item()
    assert torch.allclose(a, b, rtol=rtol, atol=atol), f"{what}: max |diff| {err:.3e} (ref max {b.abs().max():.3e})"


@pytest.mark.parametrize("name,k,rs", [("c0_fp32.npz", 2, 1.0), ("noshared_scale.npz", 3, 2.5),
                                       ("e16_k4_fp32.npz", 4, 1.5)])
def test_backward_matches_reference_golden_fp32(golden_dir, name, k, rs):
    d = dict(np.load(golden_dir / name, allow_pickle=False))
    t = lambda key: torch.from_numpy(d[key])
    st = lambda key: list(t(key).unbind(0)) if key in d else []
    D = d["x"].shape[-1]
    out = _run(t("x").reshape(-1, D), t("gate_w"), t("gate_bias"), st("w1"), st("w2"), st("w3"), st("sw1"), st("sw2"),
               st("sw3"), k, rs, t("dy").reshape(-1, D))
    assert np.array_equal(out["idx"].numpy(), d["last_indices"].reshape(-1, k))
    scale = lambda key: float(np.abs(d[key]).max())
    _close(out["y"], t("y").reshape(-1, D), 1e-5, 1e-5 * scale("y"), "y")
    _close(out["dx"], t("dx").reshape(-1, D), 1e-5, 1e-5 * scale("dx"), "dx")
    _close(out["dgate_w"], t("dgate_w"), 1e-5, 1e-5 * scale("dgate_w"), "dgate_w")
    for nm in ("dw1", "dw2", "dw3", "dsw1", "dsw2", "dsw3"):
        if nm in d:
            _close(torch.stack(out[nm]), t(nm), 1e-5, 1e-5 * scale(nm), nm)


def _sum_close(a, b, what):
    """bf16 bar for gradients summed over tokens: rtol 2e-2, atol 2e-2 x max|b|."""
    _close(a, b, 2e-2, 2e-2 * max(1.0, b.float().abs().max().item()), what)


def _relerr(a, b):
    a, b = a.float(), b.float()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _oracle_case(case, seed=0):
    x, p, dy = CS.make_inputs(case, seed=seed, with_dy=True)
    ref = R.moe_forward_backward_ref(x, p, case.k, dy, route_scale=case.route_scale)
    f32 = R.moe_forward_backward_ref(x.float(), p.to(torch.float32), case.k, dy.float(),
                                     route_scale=case.route_scale)
    out = _run(x, p.gate_w, p.gate_bias, p.w1, p.w2, p.w3, p.sw1, p.sw2, p.sw3, case.k, case.route_scale, dy)
    return ref, f32, out


@pytest.mark.parametrize("case", [CS.C1.with_tokens(512), CS.C3.with_tokens(384),
                                  CS.Case("bf16_small", 300, 128, 8, 64, 3, 1, 96, torch.bfloat16, "normal", 1.5),
                                  # +3 bias on experts 0 and 1 with k=2: experts 2..7 get no rows
                                  CS.Case("bf16_skew_empty", 320, 256, 8, 128, 2, 1, 128, torch.bfloat16, "skew"),
                                  # a width that is not a multiple of 8: dY is read through the row map
                                  CS.Case("bf16_odd_d", 300, 100, 8, 64, 2, 1, 72, torch.bfloat16, "normal"),
                                  # three shared experts, inter widths with N % 8 == 4
                                  CS.Case("bf16_s3_i132", 320, 256, 8, 132, 2, 3, 100, torch.bfloat16, "normal")],
                         ids=lambda c: c.name)
def test_backward_bf16_vs_oracle(case):
    ref, f32, out = _oracle_case(case)
    assert torch.equal(out["idx"], ref["indices"])
    assert torch.equal(f32["indices"], ref["indices"])
    _close(out["y"], ref["y"], 2e-2, 2e-2, "y")
    _close(out["dx"], ref["dx"], 2e-2, 2e-2, "dx")
    _sum_close(out["dgate_w"], ref["dgate_w"], "dgate_w")
    pairs = [("y", out["y"], ref["y"], f32["y"]), ("dx", out["dx"], ref["dx"], f32["dx"]),
             ("dgate_w", out["dgate_w"], ref["dgate_w"], f32["dgate_w"])]
    for nm in ("dw1", "dw2", "dw3", "dsw1", "dsw2", "dsw3"):
        if ref[nm]:
            a, b = torch.stack(out[nm]), torch.stack(ref[nm])
            _sum_close(a, b, nm)
            pairs.append((nm, a, b, torch.stack(f32[nm])))
    for nm, a, b, truth in pairs:
        ours, theirs = _relerr(a, truth), _relerr(b, truth)
        assert ours <= max(2.0 * theirs, 1e-3), f"{nm}: rel L2 err vs fp32 {ours:.3e}, bf16 reference {theirs:.3e}"
    # experts that received no rows get exactly zero weight gradients
    counts = torch.bincount(out["idx"].flatten(), minlength=case.E)
    for e in torch.nonzero(counts == 0).flatten().tolist():
        for nm in ("dw1", "dw2", "dw3"):
            assert not out[nm][e].any(), f"{nm}[{e}] of an expert with no rows is not zero"


def test_backward_matches_reference_golden_bf16(golden_dir):
    """Against the reference layer's own bf16 forward and backward (fp32 gate,
    tests/golden/c0_bf16_fwd_bwd.npz): routing exact; y and dx within 2e-2;
    the token sums (dW_gate, every dW) within 2e-2 x their max magnitude."""
    d = dict(np.load(golden_dir / "c0_bf16_fwd_bwd.npz", allow_pickle=False))
    cv = lambda a: torch.from_numpy(a.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16)
    st = lambda key: list(cv(d[key]).unbind(0))
    out = _run(cv(d["x_bits"]), torch.from_numpy(d["gate_w"]), torch.from_numpy(d["gate_bias"]), st("w1_bits"),
               st("w2_bits"), st("w3_bits"), st("sw1_bits"), st("sw2_bits"), st("sw3_bits"), 2, 1.0, cv(d["dy_bits"]))
    assert np.array_equal(out["idx"].numpy(), d["last_indices"])
    _close(out["y"], cv(d["y_bits"]), 2e-2, 2e-2, "y")
    _close(out["dx"], cv(d["dx_bits"]), 2e-2, 2e-2, "dx")
    _sum_close(out["dgate_w"], torch.from_numpy(d["dgate_w"]), "dgate_w")
    for nm in ("dw1", "dw2", "dw3", "dsw1", "dsw2", "dsw3"):
        _sum_close(torch.stack(out[nm]), cv(d[nm + "_bits"]), nm)


def test_backward_is_deterministic():
    case = CS.C3.with_tokens(512)
    x, p, dy = CS.make_inputs(case, with_dy=True)
    a = _run(x, p.gate_w, p.gate_bias, p.w1, p.w2, p.w3, p.sw1, p.sw2, p.sw3, case.k, 1.0, dy)
    b = _run(x, p.gate_w, p.gate_bias, p.w1, p.w2, p.w3, p.sw1, p.sw2, p.sw3, case.k, 1.0, dy)
    for key in ("dx", "dgate_w"):
        assert torch.equal(a[key], b[key]), key
    for key in ("dw1", "dw2", "dw3", "dsw1", "dsw2", "dsw3"):
        assert all(torch.equal(u, v) for u, v in zip(a[key], b[key])), key


def test_backward_second_stream_matches_one_stream():
    """The layer backward runs the routed dW2, the shared experts' chain and
    dW_gate on a second stream of its own, joined before the dx sum; with stage
    timing on it runs everything on the caller's stream.  Both give the same
    gradients bit for bit (every GEMM owns its tiles and sums in a fixed order),
    at a shape with routed and shared experts, on a non-default caller stream."""
    from dsmoe import _lib as L
    case = CS.C3.with_tokens(1024)
    x, p, dy = CS.make_inputs(case, with_dy=True)
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        a = _run(x, p.gate_w, p.gate_bias, p.w1, p.w2, p.w3, p.sw1, p.sw2, p.sw3, case.k, 1.0, dy)
        L.timing_enable(True)
        try:
            b = _run(x, p.gate_w, p.gate_bias, p.w1, p.w2, p.w3, p.sw1, p.sw2, p.sw3, case.k, 1.0, dy)
        finally:
            L.timing_enable(False)
            L.timing_read()
    torch.cuda.synchronize()
    for key in ("dx", "dgate_w"):
        assert torch.equal(a[key], b[key]), key
    for key in ("dw1", "dw2", "dw3", "dsw1", "dsw2", "dsw3"):
        assert all(torch.equal(u, v) for u, v in zip(a[key], b[key])), key


def test_dgate_full_batches_vs_oracle():
    """dW_gate where the kernel's waves sum full batches of rows, not only the
    one-row tail: at T=2048 and C3 width an expert holds about 192 sorted rows,
    against the 113 that one full batch of 16 waves x 8 rows needs (the T <= 512
    cases above hold about 48).  Compared with the bf16 reference autograd
    (models/moe.py:29-37 under autograd) and bitwise equal on a second run."""
    case = CS.C3.with_tokens(2048)
    x, p, dy = CS.make_inputs(case, with_dy=True)
    print(f"[dgate] fwd+bwd T={case.T}", flush=True)
    a = _run(x, p.gate_w, p.gate_bias, p.w1, p.w2, p.w3, p.sw1, p.sw2, p.sw3, case.k, 1.0, dy)
    b = _run(x, p.gate_w, p.gate_bias, p.w1, p.w2, p.w3, p.sw1, p.sw2, p.sw3, case.k, 1.0, dy)
    assert torch.equal(a["dgate_w"], b["dgate_w"])
    counts = torch.bincount(a["idx"].flatten(), minlength=case.E)
    assert counts.min().item() >= 113, counts.min().item()
    ref = R.moe_forward_backward_ref(x, p, case.k, dy)
    assert torch.equal(a["idx"], ref["indices"])
    _sum_close(a["dgate_w"], ref["dgate_w"], "dgate_w")
    _close(a["dx"], ref["dx"], 2e-2, 2e-2, "dx")


def _slice_close(a, b, what):
    """bf16 layer against the fp32 oracle on the same bf16 inputs: relative L2
    error at most 1e-2, and elementwise within rtol 2e-2, atol 2e-2 x max|b|."""
    a, b = a.float(), b.float()
    rel = _relerr(a, b)
    err = (a - b).abs().max().item()
    print(f"  {what}: rel L2 {rel:.2e}, max |diff| {err:.2e} (ref max {b.abs().max():.2e})")
    assert rel <= 1e-2, f"{what}: rel L2 err {rel:.3e}"
    assert torch.allclose(a, b, rtol=2e-2, atol=2e-2 * b.abs().max().item()), f"{what}: max |diff| {err:.3e}"


def _rows_close_or_fp32(a, b, what, x, p, dy, idx, k):
    """Token-separable outputs (y, dx) over many rows: elementwise within
    rtol = atol = 2e-2 of the bf16 oracle; a row where some element misses
    that bar (over tens of millions of elements the two bf16 computations'
    rounding differences reach past it) is checked against the fp32 oracle on
    the same bf16 inputs and routing, and must be within the bar of it."""
    a, b = a.float(), b.float()
    miss = ~torch.isclose(a, b, rtol=2e-2, atol=2e-2)
    rows = torch.nonzero(miss.any(-1)).flatten()
    print(f"  {what}: {int(miss.sum())} of {miss.numel()} elements in {rows.numel()} rows miss the bar against "
          f"the bf16 oracle (max |diff| {(a - b).abs().max().item():.3e})", flush=True)
    assert rows.numel() <= max(16, a.shape[0] // 1000), rows.numel()
    if rows.numel() == 0:
        return
    f32 = R.moe_forward_backward_ref(x[rows].float(), p.to(torch.float32), k, dy[rows].float(), indices=idx[rows])
    _close(a[rows], f32[what], 2e-2, 2e-2, f"{what} rows against the fp32 oracle")


def test_c4_full_size_gradients():
    """C4 (T=16384) at full size.  dx is token-separable: the oracle on a token
    sample is exact for those rows.  Weight gradients are sums over each
    expert's rows: for three routed experts (about 1,500 rows each) and both
    shared experts (all 16,384 rows) a slice of 64 inter columns of dW1, dW2
    and dW3 is compared with the fp32 oracle on exactly those rows
    (expert_grad_slice_ref), with the layer's routing and its fp32 weights.
    Every gradient is finite; unrouted experts get exact zeros.  Then the
    whole layer against the bf16 oracle's autograd at full size."""
    case = CS.C4
    x, p, dy = CS.make_inputs(case, with_dy=True)
    print(f"[c4] fwd+bwd T={case.T}", flush=True)
    out = _run(x, p.gate_w, p.gate_bias, p.w1, p.w2, p.w3, p.sw1, p.sw2, p.sw3, case.k, 1.0, dy)
    for key in ("dx", "dgate_w"):
        assert torch.isfinite(out[key].float()).all(), key
    for key in ("dw1", "dw2", "dw3", "dsw1", "dsw2", "dsw3"):
        assert all(torch.isfinite(t.float()).all() for t in out[key]), key
    rows = torch.randperm(case.T, generator=torch.Generator().manual_seed(3))[:96]
    ref = R.moe_forward_backward_ref(x[rows], p, case.k, dy[rows])
    _close(out["dx"][rows], ref["dx"], 2e-2, 2e-2, "dx sample")
    idx = out["idx"]
    counts = torch.bincount(idx.flatten(), minlength=case.E)
    for e in range(case.E):
        if counts[e] == 0:
            assert not out["dw2"][e].any()
    # routing weights of the layer's ids from the fp32 logits (renormalised as models/moe.py:35-36)
    sel = R.gate_logits_ref(x, p.gate_w).sigmoid().gather(1, idx)
    w = sel / sel.sum(-1, keepdim=True).clamp(min=1e-10)
    i0, i1 = 640, 704
    for e in (0, 17, 42):
        t, j = torch.nonzero(idx == e, as_tuple=True)
        print(f"[c4] expert {e}: {len(t)} rows", flush=True)
        a, b, c = R.expert_grad_slice_ref(x[t], dy[t], w[t, j], p.w1[e], p.w2[e], p.w3[e], i0, i1)
        _slice_close(out["dw1"][e][i0:i1], a, f"dw1[{e}]")
        _slice_close(out["dw2"][e][:, i0:i1], b, f"dw2[{e}]")
        _slice_close(out["dw3"][e][i0:i1], c, f"dw3[{e}]")
    for si in range(case.S):
        a, b, c = R.expert_grad_slice_ref(x, dy, torch.ones(case.T), p.sw1[si], p.sw2[si], p.sw3[si], i0, i1)
        _slice_close(out["dsw1"][si][i0:i1], a, f"dsw1[{si}]")
        _slice_close(out["dsw2"][si][:, i0:i1], b, f"dsw2[{si}]")
        _slice_close(out["dsw3"][si][i0:i1], c, f"dsw3[{si}]")
    # the whole layer under the oracle's autograd at full size (about 20 s of
    # host time): routing, every row of dx, the full dW_gate (64 x 2048, each
    # element a sum over about 1,500 rows) and every expert's dW, with the bf16
    # bars of test_backward_bf16_vs_oracle
    print("[c4] oracle autograd at full size", flush=True)
    # Routing is bit-exact given the kernel's own fp32 logits (the layer
    # routing tests); torch's CPU logits differ from them in accumulation
    # order, so at 16,384 tokens a few tokens whose k-th and (k+1)-th biased
    # scores are closer than that difference may pick the other expert.  The
    # gradients are compared under the layer's routing, and each token whose
    # set differs must be such a near-tie.
    lg = R.gate_logits_ref(x, p.gate_w)
    _, own, _ = R.route_from_logits_ref(lg, p.gate_bias, case.k)
    differ = torch.nonzero((own.sort(-1)[0] != idx.sort(-1)[0]).any(-1)).flatten()
    biased = (lg.sigmoid() + p.gate_bias).sort(-1, descending=True)[0]
    gaps = (biased[differ, case.k - 1] - biased[differ, case.k]).abs()
    print(f"[c4] tokens whose oracle top-k set differs: {differ.numel()}, gaps {gaps.tolist()}", flush=True)
    assert differ.numel() <= 8 and (gaps < 1e-5).all()
    ref = R.moe_forward_backward_ref(x, p, case.k, dy, indices=idx)
    assert torch.equal(idx, ref["indices"])
    _rows_close_or_fp32(out["y"], ref["y"], "y", x, p, dy, idx, case.k)
    _rows_close_or_fp32(out["dx"], ref["dx"], "dx", x, p, dy, idx, case.k)
    _sum_close(out["dgate_w"], ref["dgate_w"], "dgate_w")
    rel = _relerr(out["dgate_w"], ref["dgate_w"])
    print(f"[c4] dgate_w rel L2 vs the bf16 oracle {rel:.2e}", flush=True)
    assert rel <= 2e-2, rel
    for nm in ("dw1", "dw2", "dw3", "dsw1", "dsw2", "dsw3"):
        _sum_close(torch.stack(out[nm]), torch.stack(ref[nm]), nm)


def test_module_training_step_all_params_get_grads():
    from dsmoe import DeepSeekMoE
    case = CS.Case("train_small", 256, 128, 8, 64, 2, 1, 64, torch.bfloat16, "zeros")
    x, p, dy = CS.make_inputs(case, with_dy=True)
    m = CS.load_module(case, p, DEV, DeepSeekMoE)
    xin = x.to(DEV).view(2, 128, case.D).requires_grad_(True)
    y = m(xin)
    (y.float() * dy.to(DEV).view_as(y).float()).sum().backward()
    for name, prm in m.named_parameters():
        assert prm.grad is not None, name
        assert torch.isfinite(prm.grad.float()).all(), name
    assert m.gate.bias.grad is None
    ref = R.moe_forward_backward_ref(x, p, case.k, dy)
    _close(xin.grad.view(-1, case.D).cpu(), ref["dx"], 2e-2, 2e-2, "dx")
    _sum_close(m.gate.weight.grad.cpu(), ref["dgate_w"], "dgate_w")


# --------------------------------------------------------------------- grouped operator seam backward
@pytest.mark.parametrize("T,D,E,I,counts,dtype", [
    (16, 16, 2, 16, [9, 7], torch.float32),                 # tests/test_moe_triton.py:296-327 bwd shape
    (24, 16, 4, 12, [6, 0, 8, 10], torch.float32),          # empty expert: its dW must be zero
    (300, 128, 4, 256, [130, 0, 1, 169], torch.bfloat16),   # MFMA path, ragged tiles
    (520, 256, 3, 192, [257, 256, 7], torch.bfloat16),      # MFMA path, N tail
])
def test_grouped_operator_backward_vs_oracle(T, D, E, I, counts, dtype):
    """_TritonGroupedMoeFunction.backward contract (models/moe_triton.py:438-501)
    through grouped_moe_dispatch: dx, dW1, dW2, dW3 and the gate-weight gradient
    against autograd of the oracle (grouped_moe_pytorch restated), fp64."""
    from dsmoe import grouped_moe_dispatch
    x, w1, w2, w3, off, gw = CS.grouped_case(T, D, E, I, counts, dtype, seed=7 * T + D)
    dy = (torch.randn(T, D, generator=torch.Generator().manual_seed(T)) * 0.1).to(dtype)
    dev = [_leaf(t) for t in (x, w1, w2, w3, gw)]
    y = grouped_moe_dispatch(dev[0], dev[1], dev[2], dev[3], dev[4], off.to(DEV))
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    got = [t.grad.detach().cpu() for t in dev]
    ref = [t.detach().double().requires_grad_(True) for t in (x, w1, w2, w3, gw)]
    y_ref = R.grouped_moe_ref(ref[0], ref[1], ref[2], ref[3], off, ref[4])
    y_ref.backward(dy.double())
    names = ("dx", "dw1", "dw2", "dw3", "dgate_w")
    for name, a, r in zip(names, got, ref):
        b = r.grad
        assert torch.isfinite(a.float()).all(), name
        if dtype == torch.float32:
            _close(a, b, 1e-5, 1e-5 * max(1e-30, b.abs().max().item()), name)
        elif name == "dx":
            _close(a, b, 2e-2, 2e-2, name)
        else:
            _sum_close(a, b, name)
    for e, c in enumerate(counts):
        if c == 0:
            for name, a in zip(names[1:4], got[1:4]):
                assert torch.count_nonzero(a[e]) == 0, f"{name}[{e}] of an expert without rows must be zero"
