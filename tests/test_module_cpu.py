"""Host-side behaviour of the drop-in module (CPU only, no kernel launches):
constructor contract, state_dict keys, buffers, error on CPU forward, balance
metric and bias update from planted routings, config-compat helper.  Mirrors
the reference's tests/test_models.py:287-389,757-800 and tests/test_force_back.py."""
import pytest
import torch

from dsmoe import AuxLossFreeGate, DeepSeekMoE, Expert, enforce_triton_env_var, next_pow2
from oracle import moe_ref as R


def test_construction_and_state_dict_keys(small_cfg):
    moe = DeepSeekMoE(small_cfg)
    assert len(moe.experts) == 4 and len(moe.shared_experts) == 1
    assert isinstance(moe.gate, AuxLossFreeGate)
    keys = set(moe.state_dict())
    expect = {"gate.weight", "gate.bias"}
    for e in range(4):
        expect |= {f"experts.{e}.w1.weight", f"experts.{e}.w2.weight", f"experts.{e}.w3.weight"}
    expect |= {"shared_experts.0.w1.weight", "shared_experts.0.w2.weight", "shared_experts.0.w3.weight"}
    assert keys == expect
    assert moe.experts[0].w1.weight.shape == (64, 64) and moe.experts[0].w2.weight.shape == (64, 64)
    assert moe.moe_dispatch == "stacked"
    assert DeepSeekMoE(dict(small_cfg, moe_dispatch="triton_grouped")).moe_dispatch == "triton_grouped"


def test_shared_inter_dim_extension(small_cfg):
    moe = DeepSeekMoE(dict(small_cfg, shared_inter_dim=128))
    assert moe.shared_experts[0].w1.weight.shape == (128, 64)
    assert moe.experts[0].w1.weight.shape == (64, 64)


def test_gate_contract(small_cfg):
    gate = AuxLossFreeGate(small_cfg)
    assert gate.weight.shape == (4, 64) and gate.bias.shape == (4,) and gate.bias.dtype == torch.float32
    assert id(gate.bias) not in {id(p) for p in gate.parameters()}
    assert "bias" in gate.state_dict()
    assert gate.route_scale == 1.0 and gate.bias_upper == 0.10 and gate.bias_lower == 0.10


def test_forward_on_cpu_raises(small_cfg):
    moe = DeepSeekMoE(small_cfg)
    with pytest.raises(RuntimeError, match="ROCm"):
        moe(torch.randn(2, 8, 64))
    with pytest.raises(RuntimeError, match="ROCm"):
        moe.gate(torch.randn(8, 64))
    with pytest.raises(RuntimeError, match="ROCm"):
        Expert(64, 32)(torch.randn(3, 64))


def test_balance_loss_zero_before_forward(small_cfg):
    assert DeepSeekMoE(small_cfg).get_load_balance_loss().item() == 0.0


def test_balance_loss_from_planted_routing_matches_oracle(small_cfg):
    moe = DeepSeekMoE(small_cfg)
    g = torch.Generator().manual_seed(0)
    idx = torch.stack([torch.randperm(4, generator=g)[:2] for _ in range(128)])
    w = torch.rand(128, 2, generator=g)
    w = w / w.sum(1, keepdim=True)
    moe._last_indices, moe._last_weights = idx, w
    assert abs(moe.get_load_balance_loss().item() - R.balance_loss_ref(w, idx, 4).item()) < 1e-6


def test_update_gate_bias_kat_all_to_expert0(small_cfg):
    """tests/test_models.py:325-345."""
    moe = DeepSeekMoE(small_cfg)
    moe._last_indices = torch.zeros(128, 2, dtype=torch.long)
    moe._last_weights = torch.ones(128, 2) / 2
    moe.update_gate_bias(speed=0.1)
    assert torch.equal(moe.gate.bias, torch.tensor([-0.1, 0.1, 0.1, 0.1]))


def test_update_bias_sign_rule_kat():
    """tests/test_models.py:760-777."""
    gate = AuxLossFreeGate({"dim": 8, "n_activated_experts": 2, "n_routed_experts": 4,
                            "bias_upper_threshold": 0.10, "bias_lower_threshold": 0.10})
    gate.update_bias(torch.tensor([10, 5, 5, 0], dtype=torch.float32), speed=0.01)
    assert torch.equal(gate.bias, torch.tensor([-0.01, 0.0, 0.0, 0.01]))


def test_update_gate_bias_noop_without_routing(small_cfg):
    moe = DeepSeekMoE(small_cfg)
    moe.update_gate_bias(0.5)
    assert torch.equal(moe.gate.bias, torch.zeros(4))


def test_stacked_views_absent_before_forward(small_cfg):
    moe = DeepSeekMoE(small_cfg)
    assert moe._stacked_w1 is None and moe._shared_w1 is None


@pytest.mark.parametrize("env,cfg,expect,warned", [
    (None, {"moe_dispatch": "triton_grouped"}, "stacked", True),
    ("1", {"moe_dispatch": "triton_grouped"}, "triton_grouped", False),
    (None, {"moe_dispatch": "stacked"}, "stacked", False),
])
def test_enforce_triton_env_var_compat(monkeypatch, env, cfg, expect, warned):
    """tests/test_force_back.py:29-72 behaviour of models/_triton_dispatch.py."""
    if env is None:
        monkeypatch.delenv("ENABLE_TRITON_KERNELS", raising=False)
    else:
        monkeypatch.setenv("ENABLE_TRITON_KERNELS", env)
    log = []
    enforce_triton_env_var(cfg, log.append)
    assert cfg["moe_dispatch"] == expect
    assert bool(log) == warned


@pytest.mark.parametrize("env", [None, "0", "1"])
def test_enforce_triton_env_var_attention_key(monkeypatch, env):
    """Both of the reference's keys (models/_triton_dispatch.py:13-16): the
    attention selection is reset to 'sdpa' with the MoE one, in one log call."""
    if env is None:
        monkeypatch.delenv("ENABLE_TRITON_KERNELS", raising=False)
    else:
        monkeypatch.setenv("ENABLE_TRITON_KERNELS", env)
    cfg = {"attn_impl": "triton", "moe_dispatch": "triton_grouped", "dim": 64}
    log = []
    enforce_triton_env_var(cfg, log.append)
    if env == "1":
        assert cfg == {"attn_impl": "triton", "moe_dispatch": "triton_grouped", "dim": 64} and not log
    else:
        assert cfg == {"attn_impl": "sdpa", "moe_dispatch": "stacked", "dim": 64} and len(log) == 1


def test_next_pow2():
    assert [next_pow2(n) for n in (0, 1, 2, 3, 64, 65, 384)] == [1, 1, 2, 4, 64, 128, 512]


def test_planted_routing_replaces_the_forward_histogram(small_cfg):
    """A forward leaves the kernel histogram beside _last_indices; planting new
    indices (as the reference's tests do) must switch the counts to them."""
    moe = DeepSeekMoE(small_cfg)
    moe._last_indices = torch.zeros(8, 2, dtype=torch.long)
    moe._last_weights = torch.ones(8, 2) / 2
    moe._last_counts = torch.tensor([16, 0, 0, 0], dtype=torch.int32)
    moe._counts_of = moe._last_indices
    assert torch.equal(moe._counts(), torch.tensor([16, 0, 0, 0], dtype=torch.int32))
    moe._last_indices = torch.full((8, 2), 3, dtype=torch.long)
    assert torch.equal(moe._counts(), torch.tensor([0, 0, 0, 16]))


def test_checkpoint_manager_roundtrip(small_cfg, tmp_path):
    """utils/checkpoint.py:17-55,78-88: the state_dict is saved with
    safetensors after the manager's shared-storage de-duplication and loaded
    back with strict key checking.  Every key must survive the de-duplication
    (no two entries share storage) and load into a fresh layer unchanged."""
    from safetensors.torch import load_file, save_file
    src = DeepSeekMoE(small_cfg)
    with torch.no_grad():
        src.gate.bias.copy_(torch.tensor([0.5, -0.25, 0.0, 1.0]))
    state = src.state_dict()
    seen, kept = set(), {}
    for k, v in state.items():          # the manager's de-duplication by data_ptr
        if v.data_ptr() in seen:
            continue
        seen.add(v.data_ptr())
        kept[k] = v.contiguous()
    assert set(kept) == set(state)
    path = tmp_path / "model_step_1.safetensors"
    save_file(kept, str(path))
    dst = DeepSeekMoE(small_cfg)
    missing, unexpected = dst.load_state_dict(load_file(str(path)), strict=False)
    assert not missing and not unexpected
    for k, v in dst.state_dict().items():
        assert torch.equal(v, state[k]), k
    assert dst.gate.bias.dtype == torch.float32


def test_layer_operator_shapes_without_a_gpu():
    """The layer's torch.library operators (what torch.compile traces) give
    the real outputs' shapes and dtypes from their fake implementations."""
    import dsmoe.ops  # noqa: F401  (registers dsmoe::moe_fwd / dsmoe::moe_bwd)
    T, D, E, S, k, I, I_s = 96, 128, 8, 1, 2, 64, 96
    m = dict(device="meta", dtype=torch.bfloat16)
    x = torch.empty(T, D, **m)
    gw, gb = torch.empty(E, D, device="meta"), torch.empty(E, device="meta")
    ws = ([torch.empty(I, D, **m) for _ in range(E)] + [torch.empty(D, I, **m) for _ in range(E)] +
          [torch.empty(I, D, **m) for _ in range(E)] +
          [torch.empty(I_s, D, **m), torch.empty(D, I_s, **m), torch.empty(I_s, D, **m)])
    y, idx, wx, counts, work = torch.ops.dsmoe.moe_fwd(x, gw, gb, ws, [], E, S, k, I, I_s, 1.0, True)
    assert y.shape == (T, D) and y.dtype == torch.bfloat16
    assert idx.shape == (T, k) and idx.dtype == torch.int64
    assert wx.shape == (T, k) and wx.dtype == torch.bfloat16
    assert counts.shape == (E,) and counts.dtype == torch.int32
    assert work.dtype == torch.uint8 and work.numel() >= 256
    for dw_f32 in (False, True):   # weight gradients in the weights' dtype, or fp32 for fp32 masters
        g = torch.ops.dsmoe.moe_bwd(x, gw, ws, y, work, E, S, k, I, I_s, 1.0, dw_f32)
        assert len(g) == 2 + len(ws)
        assert g[0].shape == (T, D) and g[1].shape == (E, D) and g[1].dtype == torch.float32
        want = torch.float32 if dw_f32 else torch.bfloat16
        assert all(a.shape == w.shape and a.dtype == want for a, w in zip(g[2:], ws))


def _layer_args(D=16, E=4, I=8, S=1, I_s=8, dt=torch.bfloat16):
    x = torch.zeros(5, D, dtype=dt)
    gw, gb = torch.zeros(E, D), torch.zeros(E)
    w1 = [torch.zeros(I, D, dtype=dt) for _ in range(E)]
    w2 = [torch.zeros(D, I, dtype=dt) for _ in range(E)]
    w3 = [torch.zeros(I, D, dtype=dt) for _ in range(E)]
    s1 = [torch.zeros(I_s, D, dtype=dt) for _ in range(S)]
    s2 = [torch.zeros(D, I_s, dtype=dt) for _ in range(S)]
    s3 = [torch.zeros(I_s, D, dtype=dt) for _ in range(S)]
    return [x, gw, gb, w1, w2, w3, s1, s2, s3]


@pytest.mark.parametrize("edit,match", [
    (lambda a: a.__setitem__(1, a[1].bfloat16()), "gate weight must be float32"),      # model.bfloat16()
    (lambda a: a.__setitem__(1, torch.zeros(4, 8)), "gate weight must be float32"),    # (E, D) mismatch
    (lambda a: a.__setitem__(2, torch.zeros(4, dtype=torch.float64)), "gate bias"),
    (lambda a: a.__setitem__(2, torch.zeros(5)), "gate bias"),
    (lambda a: a[4].__setitem__(1, torch.zeros(8, 16, dtype=torch.bfloat16)), "w2"),  # w2[1] transposed
    (lambda a: a[3].__setitem__(2, torch.zeros(8, 16)), "dtype"),                      # fp32 expert in bf16 layer
    (lambda a: a[3].__setitem__(0, torch.zeros(12, 16, dtype=torch.bfloat16)), "w1/w3"),
    (lambda a: a[6].__setitem__(0, torch.zeros(8, 12, dtype=torch.bfloat16)), "shared expert"),
    (lambda a: a.__setitem__(8, []), "shared"),
    (lambda a: a.__setitem__(0, torch.zeros(5, 16, dtype=torch.float16)), "activation dtype"),
])
def test_moe_layer_rejects_bad_shapes_before_any_launch(edit, match):
    """The kernels trust the sizes they are given; moe_layer checks them first
    (CPU tensors: the check runs before the device check)."""
    from dsmoe import ops
    args = _layer_args()
    ops.check_layer_args(*args, k=2)                                   # the valid case passes
    edit(args)
    with pytest.raises(ValueError, match=match):
        ops.moe_layer(*args, k=2)


def test_moe_layer_rejects_bad_topk():
    from dsmoe import ops
    with pytest.raises(ValueError, match="n_activated_experts"):
        ops.moe_layer(*_layer_args(), k=5)


@pytest.mark.parametrize("idx,ok", [
    ([[0, 1], [3, 2]], True),
    ([[0, 4], [3, 2]], False),      # id == E
    ([[0, -1], [3, 2]], False),     # negative id
    ([[1, 1], [3, 2]], False),      # repeated within a token
    ([[0], [3]], True),
])
def test_check_routing(idx, ok):
    from dsmoe import ops
    t = torch.tensor(idx, dtype=torch.int32)
    if ok:
        ops.check_routing(t, 4)
    else:
        with pytest.raises(ValueError):
            ops.check_routing(t, 4)


def test_autocast_cast_cache_follows_parameter_updates(small_cfg):
    """The bf16 copy used under autocast is made once per parameter version:
    reused while the parameter is unchanged, remade after an in-place update,
    and the gradient reaches the fp32 parameter through it."""
    moe = DeepSeekMoE(small_cfg)
    w = moe.experts[1].w3.weight
    a = moe._cast(w, torch.bfloat16)
    b = moe._cast(w, torch.bfloat16)
    assert a.dtype == torch.bfloat16 and a.data_ptr() == b.data_ptr()
    assert torch.equal(a.float(), w.detach().bfloat16().float())
    (a.float() * 3.0).sum().backward()
    assert w.grad.dtype == torch.float32 and torch.equal(w.grad, torch.full_like(w, 3.0))
    with torch.no_grad():
        w.mul_(0.5)                                   # an optimizer step
    c = moe._cast(w, torch.bfloat16)
    assert torch.equal(c.float(), w.detach().bfloat16().float())
    assert moe._cast(w, torch.float32) is w
    moe.to(torch.float64)
    assert not moe._cast_cache


@pytest.mark.parametrize("fused", [True, False])
def test_cast_cache_follows_adamw_steps(small_cfg, fused):
    """A fused AdamW step (the reference trainer's optimizer on GPU,
    training/pretrain.py:197) rewrites the parameters without moving their
    version counters or storage; the cached bf16 copy must still follow it.
    Writes through ``param.data`` move nothing: ``invalidate_weight_casts``
    covers those."""
    from dsmoe import invalidate_weight_casts
    moe = DeepSeekMoE(small_cfg)
    w = moe.experts[0].w1.weight
    opt = torch.optim.AdamW(moe.parameters(), lr=1e-2, fused=fused, foreach=False if fused else None)
    stale = moe._cached_copy(w, torch.bfloat16)
    for p in moe.parameters():
        p.grad = torch.ones_like(p)
    version, ptr = w._version, w.data_ptr()
    opt.step()
    if fused:
        assert (w._version, w.data_ptr()) == (version, ptr)   # nothing on the tensor shows the update
    fresh = moe._cached_copy(w, torch.bfloat16)
    assert not torch.equal(fresh, stale)
    assert torch.equal(fresh, w.detach().to(torch.bfloat16))
    with torch.no_grad():
        w.data.add_(1.0)
    invalidate_weight_casts()
    assert torch.equal(moe._cached_copy(w, torch.bfloat16), w.detach().to(torch.bfloat16))


def test_mla_operator_rejects_host_tensors_and_bad_dims():
    # the MLA drop-in has no CPU implementation: host tensors raise before any
    # launch, and the reference's 256 cap per dimension raises ValueError
    # (models/mla_triton.py:186-196)
    import torch
    from dsmoe.mla import _check_mla_dim_limits, mla_attention, triton_mla_attention
    assert triton_mla_attention is mla_attention
    t = torch.zeros(1, 1, 4, 8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        mla_attention(t, t, torch.zeros(1, 4, 8, dtype=torch.bfloat16), torch.zeros(1, 4, 8, dtype=torch.bfloat16),
                      torch.zeros(1, 8, 8, dtype=torch.bfloat16), torch.zeros(1, 8, 8, dtype=torch.bfloat16), 0.3)
    with pytest.raises(ValueError, match="256"):
        _check_mla_dim_limits(300, 8, 8, 8)
