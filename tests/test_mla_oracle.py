"""Pins oracle/mla_ref.py (the MLA attention oracle) on the CPU: torch's
scaled_dot_product_attention in float64, the absorbed formulation, closed forms
and the reference's own CPU test cases (models/mla_triton.py semantics)."""
import numpy as np
import pytest
import torch

from oracle.mla_ref import mla_attention_absorbed, mla_attention_oracle, mla_flops, mla_kv_oracle, mla_mask_oracle


def _tensors(B=2, H=3, S_q=7, S_kv=9, R=10, Dn=6, Dr=4, Dv=5, seed=0):
    g = torch.Generator().manual_seed(seed)
    rn = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)
    return (rn(B, H, S_q, Dn), rn(B, H, S_q, Dr), rn(B, S_kv, R), rn(B, S_kv, Dr), rn(H, Dn, R) * 0.3,
            rn(H, Dv, R) * 0.3, (Dn + Dr) ** -0.5)


@pytest.mark.parametrize("causal,q_start,S_q,S_kv", [(False, 0, 7, 9), (True, 0, 9, 9), (True, 2, 7, 9),
                                                    (True, 8, 1, 9), (False, 0, 1, 5)])
def test_oracle_matches_sdpa_float64(causal, q_start, S_q, S_kv):
    qn, qp, kv, pe, wk, wv, sc = _tensors(S_q=S_q, S_kv=S_kv)
    k, v = mla_kv_oracle(kv, pe, wk, wv)
    q = torch.cat([qn, qp], dim=-1)
    mask = torch.from_numpy(mla_mask_oracle(S_q, S_kv, causal, q_start))
    ref = torch.nn.functional.scaled_dot_product_attention(q, torch.from_numpy(k), torch.from_numpy(v),
                                                           attn_mask=mask, scale=sc)
    got = mla_attention_oracle(qn, qp, kv, pe, wk, wv, sc, is_causal=causal, q_start=q_start)
    np.testing.assert_allclose(got, ref.permute(0, 2, 1, 3).numpy(), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("causal,q_start", [(False, 0), (True, 0), (True, 3)])
def test_oracle_matches_absorbed_formulation(causal, q_start):
    qn, qp, kv, pe, wk, wv, sc = _tensors(S_q=6, S_kv=9)
    a = mla_attention_oracle(qn, qp, kv, pe, wk, wv, sc, is_causal=causal, q_start=q_start)
    b = mla_attention_absorbed(qn, qp, kv, pe, wk, wv, sc, is_causal=causal, q_start=q_start)
    np.testing.assert_allclose(a, b, rtol=1e-11, atol=1e-12)


def test_materialised_k_v_shapes_and_rope_columns():
    qn, qp, kv, pe, wk, wv, sc = _tensors()
    k, v = mla_kv_oracle(kv, pe, wk, wv)
    assert k.shape == (2, 3, 9, 10) and v.shape == (2, 3, 9, 5)
    # the rope part of K is ctx_pe itself, the same for every head
    for h in range(3):
        np.testing.assert_array_equal(k[:, h, :, 6:], pe.numpy())
    # K_nope = ctx_kv W_k^T for one element, summed by hand
    b, h, s, d = 1, 2, 4, 3
    assert abs(k[b, h, s, d] - sum(kv[b, s, r].item() * wk[h, d, r].item() for r in range(10))) < 1e-12


def test_single_key_gives_its_value_row():
    qn, qp, kv, pe, wk, wv, sc = _tensors(S_q=4, S_kv=1)
    out = mla_attention_oracle(qn, qp, kv, pe, wk, wv, sc)
    _, v = mla_kv_oracle(kv, pe, wk, wv)
    for qi in range(4):
        np.testing.assert_allclose(out[:, qi], v[:, :, 0], rtol=1e-13, atol=1e-13)


def test_equal_scores_give_prefix_means():
    qn, qp, kv, pe, wk, wv, sc = _tensors(S_q=5, S_kv=5)
    out = mla_attention_oracle(qn * 0, qp * 0, kv, pe, wk, wv, sc, is_causal=True)
    _, v = mla_kv_oracle(kv, pe, wk, wv)
    for qi in range(5):
        np.testing.assert_allclose(out[:, qi], v[:, :, : qi + 1].mean(axis=2), rtol=1e-12, atol=1e-13)


def test_reference_case_last_position_query_sees_all_keys():
    # tests/test_mla_triton.py:68-86: a single query at q_start = S_kv - 1
    qn, qp, kv, pe, wk, wv, sc = _tensors(B=1, H=2, S_q=1, S_kv=10, R=8, Dn=6, Dr=4, Dv=8)
    a = mla_attention_oracle(qn, qp, kv, pe, wk, wv, sc, is_causal=True, q_start=9)
    b = mla_attention_oracle(qn, qp, kv, pe, wk, wv, sc, is_causal=False)
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-14)


def test_reference_case_q_start_blocks_future_keys():
    # tests/test_mla_triton.py:88-110: a chunk at global positions [6, 12) over 12 keys
    qn, qp, kv, pe, wk, wv, sc = _tensors(B=1, H=2, S_q=6, S_kv=12, R=8, Dn=6, Dr=4, Dv=8)
    out = mla_attention_oracle(qn, qp, kv, pe, wk, wv, sc, is_causal=True, q_start=6)
    # changing the keys a query may not see leaves its output unchanged
    kv2, pe2 = kv.clone(), pe.clone()
    kv2[:, 7:] += 5.0
    pe2[:, 7:] -= 3.0
    out2 = mla_attention_oracle(qn, qp, kv2, pe2, wk, wv, sc, is_causal=True, q_start=6)
    np.testing.assert_allclose(out[:, 0], out2[:, 0], rtol=0, atol=1e-14)   # query 6 sees keys 0..6
    assert np.abs(out[:, 1] - out2[:, 1]).max() > 1e-3                     # query 7 sees key 7


def test_square_mask_flag_states_the_reference_function_difference():
    # mla_attention_reference masks a square non-causal call (models/mla_triton.py:52-57), the
    # fused kernel does not: the flag reproduces the former, equal to the causal output
    qn, qp, kv, pe, wk, wv, sc = _tensors(S_q=6, S_kv=6)
    sq = mla_attention_oracle(qn, qp, kv, pe, wk, wv, sc, square_mask=True)
    causal = mla_attention_oracle(qn, qp, kv, pe, wk, wv, sc, is_causal=True)
    plain = mla_attention_oracle(qn, qp, kv, pe, wk, wv, sc)
    np.testing.assert_allclose(sq, causal, rtol=0, atol=1e-14)
    assert np.abs(sq - plain).max() > 1e-3


def test_flop_count_pairs():
    f = mla_flops(1, 1, 4, 4, 8, 2, 2, 2, True)
    assert f["pairs"] == 10
    assert mla_flops(1, 1, 2, 6, 8, 2, 2, 2, True, q_start=4)["pairs"] == 5 + 6


@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_restatement_matches_the_oracle(causal):
    """The torch restatement of the reference's SDPA path (bench.py's CPU
    baseline for the attention) computes the oracle's attention: float64
    inputs, within 1e-10."""
    from oracle.mla_ref import mla_attention_sdpa_torch
    g = torch.Generator().manual_seed(4)
    B, H, S, R, Dn, Dr, Dv = 2, 3, 40, 24, 16, 8, 20
    ts = [torch.randn(*s, generator=g, dtype=torch.float64) for s in
          ((B, H, S, Dn), (B, H, S, Dr), (B, S, R), (B, S, Dr), (H, Dn, R), (H, Dv, R))]
    sc = (Dn + Dr) ** -0.5
    got = mla_attention_sdpa_torch(*ts, sc, is_causal=causal).numpy()
    ref = mla_attention_oracle(*ts, sc, is_causal=causal)
    assert got.shape == ref.shape == (B, S, H, Dv)
    assert np.abs(got - ref).max() < 1e-10


_GRAD_KEYS = ("q_nope", "q_pe", "ctx_kv", "ctx_pe", "wkv_b_k", "wkv_b_v")


@pytest.mark.parametrize("causal,q_start,S_q,S_kv", [(False, 0, 7, 9), (True, 0, 9, 9), (True, 2, 7, 9),
                                                    (True, 8, 1, 9), (False, 0, 9, 9)])
def test_backward_oracle_matches_float64_autograd(causal, q_start, S_q, S_kv):
    # the closed-form chain rule against torch autograd of SDPA on materialised K, V
    from oracle.mla_ref import mla_attention_bwd_oracle
    qn, qp, kv, pe, wk, wv, sc = _tensors(S_q=S_q, S_kv=S_kv, seed=3)
    g = torch.Generator().manual_seed(4)
    dout = torch.randn(2, S_q, 3, 5, generator=g, dtype=torch.float64)
    ins = [t.clone().requires_grad_() for t in (qn, qp, kv, pe, wk, wv)]
    a_qn, a_qp, a_kv, a_pe, a_wk, a_wv = ins
    k = torch.cat([torch.einsum("bsr,hdr->bhsd", a_kv, a_wk), a_pe[:, None].expand(2, 3, S_kv, 4)], dim=-1)
    v = torch.einsum("bsr,hdr->bhsd", a_kv, a_wv)
    mask = torch.from_numpy(mla_mask_oracle(S_q, S_kv, causal, q_start))
    o = torch.nn.functional.scaled_dot_product_attention(torch.cat([a_qn, a_qp], -1), k, v, attn_mask=mask, scale=sc)
    o.permute(0, 2, 1, 3).backward(dout)
    got = mla_attention_bwd_oracle(qn, qp, kv, pe, wk, wv, dout, sc, is_causal=causal, q_start=q_start)
    for key, t in zip(_GRAD_KEYS, ins):
        np.testing.assert_allclose(got[key], t.grad.numpy(), rtol=1e-10, atol=1e-11, err_msg=key)


def test_backward_oracle_matches_finite_differences():
    from oracle.mla_ref import mla_attention_bwd_oracle
    qn, qp, kv, pe, wk, wv, sc = _tensors(B=1, H=2, S_q=4, S_kv=5, R=3, Dn=2, Dr=2, Dv=3, seed=5)
    ins = [t.numpy().copy() for t in (qn, qp, kv, pe, wk, wv)]
    dout = np.random.default_rng(6).standard_normal((1, 4, 2, 3))
    got = mla_attention_bwd_oracle(*ins, dout, sc, is_causal=True, q_start=1)
    f = lambda xs: float((mla_attention_oracle(*xs, sc, is_causal=True, q_start=1) * dout).sum())
    h = 1e-6
    for key, x in zip(_GRAD_KEYS, range(6)):
        flat = ins[x].reshape(-1)
        num = np.empty(flat.size)
        for i in range(flat.size):
            keep = flat[i]
            flat[i] = keep + h
            up = f(ins)
            flat[i] = keep - h
            dn = f(ins)
            flat[i] = keep
            num[i] = (up - dn) / (2 * h)
        np.testing.assert_allclose(got[key].reshape(-1), num, rtol=1e-6, atol=1e-8, err_msg=key)


def test_backward_oracle_invariants():
    # each query's probabilities sum to one, so dV = P^T dO summed over keys
    # equals dO summed over queries
    from oracle.mla_ref import mla_attention_bwd_oracle
    qn, qp, kv, pe, wk, wv, sc = _tensors(S_q=6, S_kv=8, seed=7)
    dout = np.random.default_rng(8).standard_normal((2, 6, 3, 5))
    got = mla_attention_bwd_oracle(qn, qp, kv, pe, wk, wv, dout, sc, is_causal=True, q_start=2)
    np.testing.assert_allclose(got["dv"].sum(axis=2), dout.sum(axis=1), rtol=1e-12, atol=1e-12)
    # a key no query sees (causal, key > last query + q_start) gets no gradient
    got = mla_attention_bwd_oracle(qn, qp, kv, pe, wk, wv, dout, sc, is_causal=True, q_start=0)
    assert np.all(got["dk_nope"][:, :, 6:] == 0) and np.all(got["dv"][:, :, 6:] == 0)
