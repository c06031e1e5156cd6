"""Pins the CPU oracle before it is trusted as the checker (CPU only).

* golden vectors written by the real reference layer (tests/golden/*.npz);
* the reference's own known-answer tests (tests/test_models.py:325-345,760-777);
* the reference docs' permutation example (docs/concepts/moe-mtp.md:679-691);
* closed forms: torch argsort(stable)/bincount, correctly rounded sigmoid,
  C2 skew counts, balance metric = 1 at perfect balance, SwiGLU width split;
* brute force per-token loops on tiny inputs.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe_ref as R
from oracle import route as RC


def _load(golden_dir, name):
    return dict(np.load(golden_dir / name, allow_pickle=False))


def _params_from(d, bf16=False):
    if bf16:
        cv = lambda a: torch.from_numpy(a.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16)
        st = lambda key: list(cv(d[key + "_bits"]).unbind(0)) if key + "_bits" in d else []
    else:
        st = lambda key: list(torch.from_numpy(d[key]).unbind(0)) if key in d else []
    return R.MoEParams(torch.from_numpy(d["gate_w"]), torch.from_numpy(d["gate_bias"]),
                       st("w1"), st("w2"), st("w3"), st("sw1"), st("sw2"), st("sw3"))


# ----------------------------------------------------------------------------
# Golden vectors from the reference
# ----------------------------------------------------------------------------
@pytest.mark.parametrize("name,k,rs", [("c0_fp32.npz", 2, 1.0), ("noshared_scale.npz", 3, 2.5),
                                       ("e16_k4_fp32.npz", 4, 1.5)])
def test_oracle_matches_reference_golden_fwd_bwd(golden_dir, name, k, rs):
    d = _load(golden_dir, name)
    p = _params_from(d)
    x = torch.from_numpy(d["x"])
    dy = torch.from_numpy(d["dy"])
    out = R.moe_forward_backward_ref(x, p, k, dy, route_scale=rs)
    assert torch.equal(out["indices"], torch.from_numpy(d["last_indices"]))
    torch.testing.assert_close(out["weights"], torch.from_numpy(d["last_weights"]), rtol=0, atol=1e-7)
    torch.testing.assert_close(out["y"], torch.from_numpy(d["y"]), rtol=1e-6, atol=1e-7)
    E = len(p.w1)
    counts = torch.bincount(out["indices"].flatten(), minlength=E)
    assert torch.equal(counts, torch.from_numpy(d["counts"]))
    bl = R.balance_loss_ref(out["weights"], out["indices"], E)
    assert abs(bl.item() - float(d["balance_loss"])) < 1e-6
    torch.testing.assert_close(out["dx"], torch.from_numpy(d["dx"]), rtol=1e-5, atol=1e-7)
    torch.testing.assert_close(out["dgate_w"], torch.from_numpy(d["dgate_w"]), rtol=1e-5, atol=1e-7)
    # weight gradients are sums over rows: fp32 summation order shows at 1e-7
    # of their magnitude
    for nm in ("w1", "w2", "w3"):
        for key in ("d" + nm, "ds" + nm):
            if key in d:
                ref = torch.from_numpy(d[key])
                torch.testing.assert_close(torch.stack(out[key]), ref, rtol=1e-5,
                                           atol=1e-6 * max(1.0, ref.abs().max().item()))


def test_oracle_matches_reference_golden_bf16_fp32_gate(golden_dir):
    d = _load(golden_dir, "c0_bf16_fp32gate.npz")
    p = _params_from(d, bf16=True)
    cv = lambda a: torch.from_numpy(a.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16)
    x = cv(d["x_bits"])
    y, w, idx = R.moe_forward_ref(x, p, 2, return_routing=True)
    assert y.dtype == torch.bfloat16 and w.dtype == torch.bfloat16
    assert torch.equal(idx, torch.from_numpy(d["last_indices"]))
    assert torch.equal(w.view(torch.int16), cv(d["last_weights_bits"]).view(torch.int16))
    assert torch.equal(y.view(torch.int16), cv(d["y_bits"]).view(torch.int16))


def test_oracle_matches_reference_golden_bf16_fwd_bwd(golden_dir):
    """The reference's own bf16 autograd (fp32 gate): forward, dx and dW_gate
    bit for bit; expert weight gradients to within one bf16 ulp (the reference
    sums each expert's gradient through its stacked weight tensor, the oracle
    through the per-expert ones)."""
    d = _load(golden_dir, "c0_bf16_fwd_bwd.npz")
    cv = lambda a: torch.from_numpy(a.astype(np.uint16).view(np.int16).copy()).view(torch.bfloat16)
    st = lambda key: list(cv(d[key]).unbind(0))
    p = R.MoEParams(torch.from_numpy(d["gate_w"]), torch.from_numpy(d["gate_bias"]), st("w1_bits"), st("w2_bits"),
                    st("w3_bits"), st("sw1_bits"), st("sw2_bits"), st("sw3_bits"))
    out = R.moe_forward_backward_ref(cv(d["x_bits"]), p, 2, cv(d["dy_bits"]))
    assert torch.equal(out["indices"], torch.from_numpy(d["last_indices"]))
    assert torch.equal(out["y"].view(torch.int16), cv(d["y_bits"]).view(torch.int16))
    assert torch.equal(out["dx"].view(torch.int16), cv(d["dx_bits"]).view(torch.int16))
    assert torch.equal(out["dgate_w"], torch.from_numpy(d["dgate_w"]))
    for nm in ("dw1", "dw2", "dw3", "dsw1", "dsw2", "dsw3"):
        a, b = torch.stack(out[nm]).float(), cv(d[nm + "_bits"]).float()
        assert ((a - b).abs() <= b.abs() * 2.0 ** -7 + 1e-30).all(), nm


def test_grouped_operator_matches_reference_golden(golden_dir):
    d = _load(golden_dir, "grouped_op.npz")
    t = {k: torch.from_numpy(v) for k, v in d.items()}
    y = R.grouped_moe_ref(t["x_sorted"], t["w1"], t["w2"], t["w3"], t["offsets"], t["sorted_weights"])
    torch.testing.assert_close(y, t["y_sorted"], rtol=0, atol=1e-7)


# ----------------------------------------------------------------------------
# Reference known-answer tests
# ----------------------------------------------------------------------------
def test_update_bias_sign_rule_kat():
    """tests/test_models.py:760-777: counts [10,5,5,0], speed 0.01 -> [-0.01, 0, 0, +0.01]."""
    b = R.update_bias_ref(torch.zeros(4), torch.tensor([10, 5, 5, 0]), 0.01)
    assert torch.equal(b, torch.tensor([-0.01, 0.0, 0.0, 0.01]))


def test_update_bias_all_to_expert0_kat():
    """tests/test_models.py:325-345: _last_indices == 0 (T=128, k=2, E=4), speed 0.1."""
    idx = torch.zeros(128, 2, dtype=torch.long)
    counts = torch.bincount(idx.flatten(), minlength=4)
    b = R.update_bias_ref(torch.zeros(4), counts, 0.1)
    assert torch.equal(b, torch.tensor([-0.1, 0.1, 0.1, 0.1]))


def test_permutation_docs_example():
    """docs/concepts/moe-mtp.md:679-691: flat_idx [1,3,1,2,0,1] (T=3,k=2,E=4)."""
    idx = np.array([[1, 3], [1, 2], [0, 1]], np.int32)
    off, ss, st, sp = RC.permute(idx, 4)
    assert off.tolist() == [0, 1, 4, 5, 6]
    assert st.tolist() == [2, 0, 1, 2, 1, 0]          # e0:{t2} e1:{t0,t1,t2} e2:{t1} e3:{t0}
    assert ss.tolist() == [4, 0, 2, 5, 3, 1]
    assert np.array_equal(ss[sp], np.arange(6))
    w = np.array([0.6, 0.4, 0.5, 0.5, 0.7, 0.3], np.float32)
    assert w[ss].tolist() == pytest.approx([0.7, 0.6, 0.5, 0.3, 0.5, 0.4])


# ----------------------------------------------------------------------------
# Closed forms for the C routing oracle
# ----------------------------------------------------------------------------
def test_sigmoid_is_correctly_rounded():
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.normal(0, 3, 20000), [0.0, -0.0, 1e-30, -88.0, 88.0, 20.0, -20.0]]).astype(np.float32)
    got = np.array([RC.sigmoid(float(v)) for v in xs], np.float32)
    ld = np.longdouble
    exact = (ld(1) / (ld(1) + np.exp(-xs.astype(ld)))).astype(np.float32)
    assert np.array_equal(got, exact)


@pytest.mark.parametrize("T,E,k,bias_std", [(1024, 4, 2, 0.0), (4096, 16, 4, 0.01), (2048, 64, 6, 0.0)])
def test_route_matches_torch_topk_away_from_ties(T, E, k, bias_std):
    g = torch.Generator().manual_seed(7)
    logits = torch.randn(T, E, generator=g) * 0.9
    bias = torch.randn(E, generator=g) * bias_std
    idx, w, s, c = RC.route(logits.numpy(), bias.numpy(), k)
    tw, tidx, scores = R.route_from_logits_ref(logits, bias, k)
    biased = (scores + bias).sort(dim=-1, descending=True).values
    margin = (biased[:, k - 1] - biased[:, k])
    safe = margin > 1e-6                            # >> sigmoid ulp differences (6e-8 at 0.5)
    assert safe.float().mean() > 0.99
    ti = tidx.numpy()
    assert np.array_equal(idx[safe.numpy()], ti[safe.numpy()]), "ordered top-k differs away from ties"
    np.testing.assert_allclose(w, tw.numpy(), rtol=2e-6, atol=1e-7)
    assert np.array_equal(c, np.bincount(idx.ravel(), minlength=E))
    # min margin helper agrees with the sorted-scores formula
    assert abs(RC.min_margin(logits.numpy(), bias.numpy(), k) - margin.min().item()) < 1e-6


def test_route_tie_rule_lower_expert_first():
    # biased scores [0.5,0.7,0.7,0.1,0.7] as logits of the same sigmoid values
    s = np.array([[0.5, 0.7, 0.7, 0.1, 0.7]], np.float32)
    logits = np.log(s / (1 - s)).astype(np.float32)
    idx, w, _, _ = RC.route(logits, np.zeros(5, np.float32), 2)
    assert idx.tolist() == [[1, 2]]
    idx, _, _, _ = RC.route(np.zeros((1, 8), np.float32), np.zeros(8, np.float32), 3)
    assert idx.tolist() == [[0, 1, 2]]


def test_route_invariants_and_route_scale():
    g = torch.Generator().manual_seed(3)
    logits = torch.randn(512, 16, generator=g)
    idx, w, s, c = RC.route(logits.numpy(), np.zeros(16, np.float32), 4, route_scale=2.5)
    assert idx.max() < 16 and idx.min() >= 0
    assert all(len(set(r)) == 4 for r in idx.tolist())
    np.testing.assert_allclose(w.sum(1), 2.5, rtol=1e-6)
    assert np.all(np.diff(s, axis=1) <= 0)        # bias 0: descending unbiased scores
    assert c.sum() == 512 * 4


def test_skew_closed_form_c2():
    """bias +3 on e0,e1: sigmoid < 1 < 3 so every token selects e0 and e1 first."""
    g = torch.Generator().manual_seed(0)
    T, E, k = 8192, 16, 4
    logits = torch.randn(T, E, generator=g) * 0.9
    bias = torch.zeros(E); bias[:2] = 3.0
    idx, w, s, c = RC.route(logits.numpy(), bias.numpy(), k)
    assert c[0] == T and c[1] == T and c.sum() == T * k
    assert set(idx[:, 0]) | set(idx[:, 1]) == {0, 1}


@pytest.mark.parametrize("T,k,E", [(3, 2, 4), (1000, 2, 4), (333, 6, 64), (5000, 4, 16), (1, 1, 1), (0, 2, 4)])
def test_permute_matches_stable_argsort(T, k, E):
    rng = np.random.default_rng(T + E)
    idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32) if T else np.zeros((0, k), np.int32)
    off, ss, st, sp = RC.permute(idx, E)
    flat = torch.from_numpy(idx.reshape(-1).astype(np.int64))
    order = torch.argsort(flat, stable=True).numpy()
    assert np.array_equal(ss, order)
    assert np.array_equal(st, order // k)
    counts = torch.bincount(flat, minlength=E).numpy()
    assert np.array_equal(np.diff(off), counts) and off[0] == 0
    assert np.array_equal(sp[ss], np.arange(T * k))


# ----------------------------------------------------------------------------
# Float path: brute force and identities
# ----------------------------------------------------------------------------
def _expert(x, w1, w2, w3):
    return F.linear(F.silu(F.linear(x, w1)) * F.linear(x, w3), w2)


def test_forward_matches_per_token_brute_force():
    D, E, I, S, k = 12, 5, 7, 2, 2
    p = R.make_params(D, E, I, S, seed=5, std=0.3, bias=torch.tensor([0.1, 0, -0.1, 0.05, 0]))
    x = torch.randn(9, D, generator=torch.Generator().manual_seed(6), dtype=torch.float64).float()
    y = R.moe_forward_ref(x, p, k)
    p64 = R.MoEParams(*[t if not isinstance(t, list) else [u.double() for u in t] for t in
                        (p.gate_w.double(), p.gate_bias.double(), p.w1, p.w2, p.w3, p.sw1, p.sw2, p.sw3)])
    for t in range(9):
        xt = x[t].double()
        sc = torch.sigmoid(p64.gate_w @ xt)
        sel = torch.argsort(sc + p64.gate_bias, descending=True, stable=True)[:k]
        ws = sc[sel] / sc[sel].sum()
        ref = sum(ws[j] * _expert(xt, p64.w1[e], p64.w2[e], p64.w3[e]) for j, e in enumerate(sel.tolist()))
        ref = ref + sum(_expert(xt, p64.sw1[s], p64.sw2[s], p64.sw3[s]) for s in range(S))
        torch.testing.assert_close(y[t].double(), ref, rtol=1e-5, atol=1e-6)


def test_shared_inter_split_identity():
    """One shared SwiGLU of inter 2m == two of inter m holding the W1/W3 row halves
    and the W2 column halves (C1's shared inter 1024 vs routed 512)."""
    g = torch.Generator().manual_seed(1)
    D, m = 32, 16
    w1 = torch.randn(2 * m, D, generator=g); w3 = torch.randn(2 * m, D, generator=g)
    w2 = torch.randn(D, 2 * m, generator=g)
    x = torch.randn(10, D, generator=g)
    one = R.shared_ref(x, [w1], [w2], [w3])
    two = R.shared_ref(x, [w1[:m], w1[m:]], [w2[:, :m], w2[:, m:]], [w3[:m], w3[m:]])
    torch.testing.assert_close(one, two, rtol=1e-5, atol=1e-5)


def test_balance_loss_is_one_at_perfect_balance():
    T, E, k = 64, 4, 2
    idx = torch.tensor([[(2 * t) % E, (2 * t + 1) % E] for t in range(T)])
    w = torch.rand(T, k)
    w = w / w.sum(1, keepdim=True)
    assert abs(R.balance_loss_ref(w, idx, E).item() - 1.0) < 1e-6


def test_grouped_ref_matches_naive_loop_reference_shape():
    """Shape and seed of tests/test_moe_triton.py:29-53."""
    torch.manual_seed(0)
    T, D, E, I = 24, 16, 5, 12
    x = torch.randn(T, D); w1 = torch.randn(E, I, D) * 0.1; w2 = torch.randn(E, D, I) * 0.1
    w3 = torch.randn(E, I, D) * 0.1
    off = torch.cat([torch.zeros(1, dtype=torch.int64), torch.tensor([6, 4, 5, 3, 6]).cumsum(0)])
    gw = torch.rand(T) * 0.2
    y = R.grouped_moe_ref(x, w1, w2, w3, off, gw)
    for e in range(E):
        s, t = off[e].item(), off[e + 1].item()
        ref = _expert(x[s:t].double(), w1[e].double(), w2[e].double(), w3[e].double()) * gw[s:t, None].double()
        torch.testing.assert_close(y[s:t].double(), ref, rtol=1e-5, atol=1e-6)


def test_grouped_ref_gradients_pass_gradcheck():
    """Pins the oracle's seam gradients (the expected values of the grouped
    backward test): autograd of grouped_moe_ref against central finite
    differences in fp64, with an empty expert, at a tiny shape."""
    torch.manual_seed(0)
    T, D, E, I = 7, 5, 3, 4
    x = torch.randn(T, D, dtype=torch.float64, requires_grad=True)
    w1 = (torch.randn(E, I, D, dtype=torch.float64) * 0.5).requires_grad_(True)
    w2 = (torch.randn(E, D, I, dtype=torch.float64) * 0.5).requires_grad_(True)
    w3 = (torch.randn(E, I, D, dtype=torch.float64) * 0.5).requires_grad_(True)
    gw = torch.rand(T, dtype=torch.float64, requires_grad=True)
    off = torch.tensor([0, 4, 4, 7])
    assert torch.autograd.gradcheck(lambda a, b, c, d, w: R.grouped_moe_ref(a, b, c, d, off, w),
                                    (x, w1, w2, w3, gw), eps=1e-6, atol=1e-7)


def test_expert_grad_slice_matches_full_layer_autograd():
    """expert_grad_slice_ref on one expert's rows gives exactly the slice of
    the full layer's weight gradients (autograd through moe_forward_ref, fp64),
    for a routed expert (rows and weights from the layer's routing) and for a
    shared expert (all rows, weight 1)."""
    g = torch.Generator().manual_seed(3)
    T, D, E, I, k, S = 96, 24, 6, 20, 2, 1
    p = R.make_params(D, E, I, S, seed=9).to(torch.float64)
    x = torch.randn(T, D, generator=g, dtype=torch.float64)
    dy = torch.randn(T, D, generator=g, dtype=torch.float64)
    full = R.moe_forward_backward_ref(x, p, k, dy)
    idx, w = full["indices"], full["weights"]
    for e in range(E):
        t, j = torch.nonzero(idx == e, as_tuple=True)
        if len(t) == 0:
            continue
        a, b, c = R.expert_grad_slice_ref(x[t].double(), dy[t], w[t, j], p.w1[e].double(), p.w2[e].double(),
                                          p.w3[e].double(), 5, 13)
        torch.testing.assert_close(a.double(), full["dw1"][e][5:13], rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(b.double(), full["dw2"][e][:, 5:13], rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(c.double(), full["dw3"][e][5:13], rtol=1e-5, atol=1e-6)
    a, b, c = R.expert_grad_slice_ref(x, dy, torch.ones(T, dtype=torch.float64), p.sw1[0], p.sw2[0], p.sw3[0], 0, I)
    torch.testing.assert_close(a.double(), full["dsw1"][0], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(b.double(), full["dsw2"][0], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(c.double(), full["dsw3"][0], rtol=1e-5, atol=1e-6)


def test_fixed_routing_option_reproduces_the_oracle_and_follows_a_given_set():
    """moe_forward_backward_ref(indices=...) with the oracle's own routing gives
    its results bit for bit; with one token's set changed, that token's
    weights are the gathered, renormalised scores of the given experts."""
    g = torch.Generator().manual_seed(9)
    T, D, E, I, k = 40, 32, 8, 16, 2
    x = torch.randn(T, D, generator=g)
    dy = torch.randn(T, D, generator=g)
    p = R.make_params(D, E, I, 1, seed=10)
    a = R.moe_forward_backward_ref(x, p, k, dy)
    b = R.moe_forward_backward_ref(x, p, k, dy, indices=a["indices"])
    for key in ("y", "dx", "dgate_w"):
        assert torch.equal(a[key], b[key]), key
    forced = a["indices"].clone()
    forced[3] = torch.tensor([e for e in range(E) if e not in forced[3].tolist()][:k])
    c = R.moe_forward_backward_ref(x, p, k, dy, indices=forced)
    assert torch.equal(c["indices"], forced)
    s = R.gate_logits_ref(x, p.gate_w).sigmoid()[3, forced[3]]
    assert torch.allclose(c["weights"][3], s / s.sum(), rtol=0, atol=1e-7)
    assert not torch.equal(c["y"][3], a["y"][3]) and torch.equal(c["y"][4], a["y"][4])
