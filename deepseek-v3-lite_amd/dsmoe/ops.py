"""Torch-facing operators over the dsmoe C ABI (device tensors only).

* ``moe_layer``            whole-layer autograd op (DeepSeekMoE.forward, models/moe.py:74-103)
* ``grouped_moe_dispatch`` the operator seam of models/moe_triton.py:504-525
* ``gate_forward``, ``route_from_logits``, ``permute``, ``combine``:
  the individual stages, exposed for tests and for callers that compose them.

Every function requires ROCm device tensors and the built HIP library; there
is no CPU path.
"""
from __future__ import annotations

from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib as L


def _require_gpu(*ts: torch.Tensor) -> torch.device:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError("dsmoe: tensors must be on a ROCm GPU (the layer has no CPU implementation)")
    return ts[0].device


def _c(t: torch.Tensor) -> torch.Tensor:
    return t if t.is_contiguous() else t.contiguous()


def _ws(nbytes: int, device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------------------- stages
def gate_forward(x: torch.Tensor, gate_w: torch.Tensor, gate_bias: torch.Tensor, k: int, route_scale: float = 1.0,
                 want_logits: bool = False):
    """AuxLossFreeGate.forward (models/moe.py:29-37), fp32 logits.

    Returns dict: idx (T,k) int32, idx64 int64, weights fp32, weights_x (x dtype),
    sel_scores fp32, counts (E,) int32, logits (T,E) fp32 or None."""
    dev = _require_gpu(x, gate_w, gate_bias)
    x = _c(x)
    T, D = x.shape
    E = gate_w.shape[0]
    d = L.make_dims(T, D, E, k, 1, 0, 0, x.dtype, route_scale)
    out = {
        "idx": torch.empty(T, k, dtype=torch.int32, device=dev),
        "idx64": torch.empty(T, k, dtype=torch.int64, device=dev),
        "weights": torch.empty(T, k, dtype=torch.float32, device=dev),
        "weights_x": torch.empty(T, k, dtype=x.dtype, device=dev),
        "sel_scores": torch.empty(T, k, dtype=torch.float32, device=dev),
        "counts": torch.empty(E, dtype=torch.int32, device=dev),
        "logits": torch.empty(T, E, dtype=torch.float32, device=dev) if want_logits else None,
    }
    gw, gb = _c(gate_w.float()), _c(gate_bias.float())
    rc = L.load().dsmoe_gate_fwd(L.ptr(x), L.ptr(gw), L.ptr(gb), d, L.ptr(out["logits"]), L.ptr(out["idx"]),
                                 L.ptr(out["idx64"]), L.ptr(out["weights"]), L.ptr(out["weights_x"]),
                                 L.ptr(out["sel_scores"]), L.ptr(out["counts"]), L.stream_ptr(dev))
    L.check(rc, "dsmoe_gate_fwd")
    return out


def route_from_logits(logits: torch.Tensor, gate_bias: torch.Tensor, k: int, route_scale: float = 1.0,
                      x_dtype: torch.dtype = torch.float32):
    """models/moe.py:32-36 after F.linear, from given fp32 logits (T,E)."""
    dev = _require_gpu(logits, gate_bias)
    logits = _c(logits.float())
    T, E = logits.shape
    d = L.make_dims(T, 1, E, k, 1, 0, 0, x_dtype, route_scale)
    out = {
        "idx": torch.empty(T, k, dtype=torch.int32, device=dev),
        "idx64": torch.empty(T, k, dtype=torch.int64, device=dev),
        "weights": torch.empty(T, k, dtype=torch.float32, device=dev),
        "weights_x": torch.empty(T, k, dtype=x_dtype, device=dev),
        "sel_scores": torch.empty(T, k, dtype=torch.float32, device=dev),
        "counts": torch.empty(E, dtype=torch.int32, device=dev),
    }
    gb = _c(gate_bias.float())
    rc = L.load().dsmoe_route_from_logits(L.ptr(logits), L.ptr(gb), d, L.ptr(out["idx"]), L.ptr(out["idx64"]),
                                          L.ptr(out["weights"]), L.ptr(out["weights_x"]), L.ptr(out["sel_scores"]),
                                          L.ptr(out["counts"]), L.stream_ptr(dev))
    L.check(rc, "dsmoe_route_from_logits")
    return out


def check_routing(idx: torch.Tensor, E: int) -> None:
    """ValueError unless every row of idx (T, k) holds k distinct expert ids
    in [0, E), the routing the gate produces.  Reads the ids back (a host
    sync), so the layer itself never calls it."""
    if idx.dim() != 2:
        raise ValueError(f"dsmoe: routing indices must be (T, k), got shape {tuple(idx.shape)}")
    if idx.numel() == 0:
        return
    if bool(((idx < 0) | (idx >= E)).any()):
        raise ValueError(f"dsmoe: routing ids must lie in [0, {E})")
    if idx.shape[1] > 1:
        srt = torch.sort(idx, dim=1).values
        if bool((srt[:, 1:] == srt[:, :-1]).any()):
            raise ValueError("dsmoe: a token's routing ids must be distinct")


def permute(idx: torch.Tensor, E: int, x: Optional[torch.Tensor] = None, weights: Optional[torch.Tensor] = None):
    """Routing prep of models/moe.py:107-117 (+ optional row gather of :150).
    The ids are checked first (check_routing): ValueError on ids outside
    [0, E) or repeated within a token."""
    dev = _require_gpu(idx)
    check_routing(idx, E)
    idx = _c(idx.to(torch.int32))
    T, k = idx.shape
    N = T * k
    D = x.shape[1] if x is not None else 1
    dt = x.dtype if x is not None else torch.float32
    d = L.make_dims(T, D, E, k, 1, 0, 0, dt, 1.0)
    lib = L.load()
    ws = _ws(lib.dsmoe_permute_workspace_size(d), dev)
    out = {
        "offsets": torch.empty(E + 1, dtype=torch.int32, device=dev),
        "sorted_slot": torch.empty(N, dtype=torch.int32, device=dev),
        "sorted_token": torch.empty(N, dtype=torch.int32, device=dev),
        "slot_pos": torch.empty(N, dtype=torch.int32, device=dev),
        "counts": torch.empty(E, dtype=torch.int32, device=dev),
        "x_sorted": torch.empty(N, D, dtype=dt, device=dev) if x is not None else None,
        "sorted_w": torch.empty(N, dtype=torch.float32, device=dev) if weights is not None else None,
    }
    xc = _c(x) if x is not None else None
    wc = _c(weights.float()) if weights is not None else None
    rc = lib.dsmoe_permute(L.ptr(idx), d, L.ptr(out["offsets"]), L.ptr(out["sorted_slot"]), L.ptr(out["sorted_token"]),
                           L.ptr(out["slot_pos"]), L.ptr(out["counts"]), L.ptr(xc), L.ptr(out["x_sorted"]), L.ptr(wc),
                           L.ptr(out["sorted_w"]), L.ptr(ws), ws.numel(), L.stream_ptr(dev))
    L.check(rc, "dsmoe_permute")
    return out


def combine(o_slots: torch.Tensor, weights: torch.Tensor, idx: torch.Tensor, shared: Optional[torch.Tensor] = None):
    """Weighted combine of models/moe.py:132 plus the shared add of :100-102.
    o_slots (T*k, D) in slot order, weights (T,k) fp32, idx (T,k)."""
    dev = _require_gpu(o_slots, weights, idx)
    T, k = idx.shape
    D = o_slots.shape[1]
    d = L.make_dims(T, D, k, k, 1, 0, 0, o_slots.dtype, 1.0)  # the combine does not read E
    y = torch.empty(T, D, dtype=o_slots.dtype, device=dev)
    oc, wc, ic = _c(o_slots), _c(weights.float()), _c(idx.to(torch.int32))
    sc = _c(shared) if shared is not None else None
    rc = L.load().dsmoe_combine_fwd(L.ptr(oc), L.ptr(wc), L.ptr(ic), L.ptr(sc), d, L.ptr(y), L.stream_ptr(dev))
    L.check(rc, "dsmoe_combine_fwd")
    return y


def update_bias_(counts: torch.Tensor, bias: torch.Tensor, speed: float, upper: float, lower: float) -> None:
    """In-place f1 bias update on device (models/moe.py:21-27), no host sync.
    Integer counts (the gate histogram) run the int32 kernel; floating counts
    (averaged or accumulated, possibly fractional) run the fp32 one, as the
    reference compares ``counts.float()`` either way."""
    dev = _require_gpu(counts, bias)
    if bias.dtype != torch.float32 or not bias.is_contiguous():
        raise ValueError("dsmoe: gate bias must be a contiguous float32 tensor")
    if counts.numel() != bias.numel():
        raise ValueError(f"dsmoe: {counts.numel()} counts for {bias.numel()} experts")
    if counts.is_floating_point():
        c = _c(counts.float().reshape(-1))
        rc = L.load().dsmoe_update_bias_f32(L.ptr(c), L.ptr(bias), bias.numel(), float(speed), float(upper),
                                            float(lower), L.stream_ptr(dev))
        L.check(rc, "dsmoe_update_bias_f32")
        return
    c = _c(counts.to(torch.int32).reshape(-1))
    rc = L.load().dsmoe_update_bias(L.ptr(c), L.ptr(bias), bias.numel(), float(speed), float(upper), float(lower),
                                    L.stream_ptr(dev))
    L.check(rc, "dsmoe_update_bias")


# ---------------------------------------------------------------------------- whole layer
def _layer_weights(weights: Sequence[torch.Tensor], E: int, S: int):
    """Splits the flat weight list [w1 x E, w2 x E, w3 x E, sw1 x S, sw2 x S, sw3 x S]."""
    return (weights[:E], weights[E:2 * E], weights[2 * E:3 * E], weights[3 * E:3 * E + S],
            weights[3 * E + S:3 * E + 2 * S], weights[3 * E + 2 * S:])


def _fwd_ws_bytes(T: int, D: int, E: int, S: int, k: int, I: int, I_s: int, dtype, rs: float, training: bool) -> int:
    d = L.make_dims(T, D, E, k, I, S, I_s, dtype, rs)
    return max(int(L.load().dsmoe_moe_fwd_workspace_size(d, int(training))), 256)


# The layer is registered as two torch.library operators, so torch.compile
# traces it as one node (shapes from the fake implementations below) instead
# of breaking the graph at a ctypes call, and autograd (including activation
# checkpoint recompute) sees an ordinary differentiable op.  The forward
# returns its workspace (routing, sorted order, pre-activations, expert
# outputs) as a fifth output; the backward consumes it.  `masters`, when not
# empty, are fp32 master copies of `weights` (a bf16 computation under
# autocast): the forward reads only `weights`, and the expert weight
# gradients go to the masters, written as fp32 by the backward kernels.
@torch.library.custom_op("dsmoe::moe_fwd", mutates_args=(), device_types="cuda")
def moe_fwd_op(x: torch.Tensor, gate_w: torch.Tensor, gate_bias: torch.Tensor, weights: List[torch.Tensor],
               masters: List[torch.Tensor], E: int, S: int, k: int, I: int, I_s: int, route_scale: float,
               training: bool) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """dsmoe_moe_fwd: returns (y, idx64, weights_x, counts int32, workspace u8)."""
    dev = x.device
    T, D = x.shape
    d = L.make_dims(T, D, E, k, I, S, I_s, x.dtype, route_scale)
    lib = L.load()
    ws = _ws(_fwd_ws_bytes(T, D, E, S, k, I, I_s, x.dtype, route_scale, training), dev)
    y = torch.empty_like(x)
    idx64 = torch.empty(T, k, dtype=torch.int64, device=dev)
    wx = torch.empty(T, k, dtype=x.dtype, device=dev)
    counts = torch.empty(E, dtype=torch.int32, device=dev)
    w1, w2, w3, s1, s2, s3 = _layer_weights(weights, E, S)
    p1, k1 = L.ptr_array(w1); p2, k2 = L.ptr_array(w2); p3, k3 = L.ptr_array(w3)
    q1, j1 = L.ptr_array(s1); q2, j2 = L.ptr_array(s2); q3, j3 = L.ptr_array(s3)
    rc = lib.dsmoe_moe_fwd(L.ptr(x), L.ptr(gate_w), L.ptr(gate_bias), p1, p2, p3, q1, q2, q3, d, int(training),
                           L.ptr(y), L.ptr(idx64), L.ptr(wx), L.ptr(counts), None, L.ptr(ws), ws.numel(),
                           L.stream_ptr(dev))
    L.check(rc, "dsmoe_moe_fwd")
    return y, idx64, wx, counts, ws


@moe_fwd_op.register_fake
def _moe_fwd_fake(x, gate_w, gate_bias, weights, masters, E, S, k, I, I_s, route_scale, training):
    T, D = x.shape
    nbytes = _fwd_ws_bytes(int(T), int(D), int(E), int(S), int(k), int(I), int(I_s), x.dtype, route_scale, training)
    return (torch.empty_like(x), x.new_empty((T, k), dtype=torch.int64), x.new_empty((T, k)),
            x.new_empty((E,), dtype=torch.int32), x.new_empty((nbytes,), dtype=torch.uint8))


@torch.library.custom_op("dsmoe::moe_bwd", mutates_args=(), device_types="cuda")
def moe_bwd_op(x: torch.Tensor, gate_w: torch.Tensor, weights: List[torch.Tensor], dy: torch.Tensor,
               ws: torch.Tensor, E: int, S: int, k: int, I: int, I_s: int, route_scale: float,
               dw_f32: bool) -> List[torch.Tensor]:
    """dsmoe_moe_bwd_ex: returns [dx, dgate_w (fp32), dW for every entry of
    weights (fp32 with dw_f32, else the weights' dtype)]."""
    dev = x.device
    T, D = x.shape
    d = L.make_dims(T, D, E, k, I, S, I_s, x.dtype, route_scale)
    lib = L.load()
    bws = _ws(lib.dsmoe_moe_bwd_workspace_size(d), dev)
    dx = torch.empty_like(x)
    dgw = torch.empty(E, D, dtype=torch.float32, device=dev)
    dws = [torch.empty(w.shape, dtype=torch.float32 if dw_f32 else w.dtype, device=dev) for w in weights]
    arrs = [L.ptr_array(a) for a in (*_layer_weights(weights, E, S), *_layer_weights(dws, E, S))]
    rc = lib.dsmoe_moe_bwd_ex(L.ptr(x), L.ptr(gate_w), *[a[0] for a in arrs[:6]], d, L.ptr(dy), L.ptr(ws),
                              L.ptr(dx), L.ptr(dgw), *[a[0] for a in arrs[6:]],
                              L.DSMOE_F32 if dw_f32 else L.dtype_code(x.dtype), L.ptr(bws), bws.numel(),
                              L.stream_ptr(dev))
    L.check(rc, "dsmoe_moe_bwd_ex")
    return [dx, dgw, *dws]


@moe_bwd_op.register_fake
def _moe_bwd_fake(x, gate_w, weights, dy, ws, E, S, k, I, I_s, route_scale, dw_f32):
    return [torch.empty_like(x), gate_w.new_empty((E, x.shape[1]), dtype=torch.float32),
            *[w.new_empty(w.shape, dtype=torch.float32 if dw_f32 else w.dtype) for w in weights]]


def _moe_fwd_setup(ctx, inputs, output):
    x, gate_w, gate_bias, weights, masters, E, S, k, I, I_s, rs, training = inputs
    ctx.meta = (E, S, k, I, I_s, rs, training, len(masters))
    ctx.save_for_backward(x, gate_w, output[4], *weights)
    # only y carries a gradient; without this autograd would materialise zero
    # gradients for the other outputs, the workspace included (GBs per step)
    ctx.set_materialize_grads(False)


def _moe_fwd_backward(ctx, dy, _didx, _dwx, _dcounts, _dws):
    E, S, k, I, I_s, rs, training, n_masters = ctx.meta
    x, gate_w, ws, *weights = ctx.saved_tensors
    rest = (None,) * 7
    if dy is None:
        return (None, None, None, [None] * len(weights), [None] * n_masters) + rest
    if not training:
        raise RuntimeError("dsmoe: forward ran without saving activations for backward")
    g = moe_bwd_op(x, gate_w, list(weights), _c(dy), ws, E, S, k, I, I_s, rs, n_masters > 0)
    if n_masters:
        return (g[0], g[1], None, [None] * len(weights), list(g[2:])) + rest
    return (g[0], g[1], None, list(g[2:]), []) + rest


torch.library.register_autograd("dsmoe::moe_fwd", _moe_fwd_backward, setup_context=_moe_fwd_setup)


def check_layer_args(x: torch.Tensor, gate_w: torch.Tensor, gate_bias: torch.Tensor, w1: Sequence[torch.Tensor],
                     w2: Sequence[torch.Tensor], w3: Sequence[torch.Tensor], sw1: Sequence[torch.Tensor],
                     sw2: Sequence[torch.Tensor], sw3: Sequence[torch.Tensor], k: int) -> Tuple[int, int, int, int]:
    """Shapes and dtypes moe_layer's kernels read, checked before any launch:
    ValueError on a mismatch (the kernels trust these sizes).  -> (E, S, I, I_s)."""
    if x.dim() != 2:
        raise ValueError(f"dsmoe: x must be (T, dim), got shape {tuple(x.shape)}")
    if x.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"dsmoe: unsupported activation dtype {x.dtype} (float32 or bfloat16)")
    D = x.shape[1]
    E, S = len(w1), len(sw1)
    if E == 0 or len(w2) != E or len(w3) != E:
        raise ValueError(f"dsmoe: need the same number (>= 1) of w1, w2, w3 expert weights, got "
                         f"{len(w1)}, {len(w2)}, {len(w3)}")
    if len(sw2) != S or len(sw3) != S:
        raise ValueError(f"dsmoe: need the same number of shared w1, w2, w3 weights, got {S}, {len(sw2)}, {len(sw3)}")
    if gate_w.dtype != torch.float32 or tuple(gate_w.shape) != (E, D):
        raise ValueError(f"dsmoe: gate weight must be float32 ({E}, {D}), got {gate_w.dtype} {tuple(gate_w.shape)}")
    if gate_bias.dtype != torch.float32 or tuple(gate_bias.shape) != (E,):
        raise ValueError(f"dsmoe: gate bias must be float32 ({E},), got {gate_bias.dtype} {tuple(gate_bias.shape)}")
    if not 1 <= int(k) <= E:
        raise ValueError(f"dsmoe: need 1 <= n_activated_experts <= {E}, got {k}")

    def inter(ws1, ws2, ws3, what):
        dims = None
        for a, b, c in zip(ws1, ws2, ws3):
            for w in (a, b, c):
                if w.dtype != x.dtype:
                    raise ValueError(f"dsmoe: {what} weight dtype {w.dtype} differs from activation dtype {x.dtype}")
                if w.dim() != 2:
                    raise ValueError(f"dsmoe: {what} weights must be 2-D, got shape {tuple(w.shape)}")
            i = a.shape[0]
            if tuple(a.shape) != (i, D) or tuple(c.shape) != (i, D) or tuple(b.shape) != (D, i):
                raise ValueError(f"dsmoe: {what} w1/w3 must be (inter, {D}) and w2 ({D}, inter), got "
                                 f"{tuple(a.shape)}, {tuple(c.shape)}, {tuple(b.shape)}")
            if dims is not None and i != dims:
                raise ValueError(f"dsmoe: all {what} experts must share one inter dim ({dims} and {i})")
            dims = i
        return dims or 0

    I = inter(w1, w2, w3, "expert")
    I_s = inter(sw1, sw2, sw3, "shared expert")
    return E, S, I, I_s


def moe_layer(x: torch.Tensor, gate_w: torch.Tensor, gate_bias: torch.Tensor, w1: Sequence[torch.Tensor],
              w2: Sequence[torch.Tensor], w3: Sequence[torch.Tensor], sw1: Sequence[torch.Tensor] = (),
              sw2: Sequence[torch.Tensor] = (), sw3: Sequence[torch.Tensor] = (), *, k: int,
              route_scale: float = 1.0, training: Optional[bool] = None,
              master_weights: Optional[Sequence[torch.Tensor]] = None):
    """One DeepSeekMoE layer on (T, D) tokens.  Expert weights must be in
    x.dtype, w1/w3 (inter, D) and w2 (D, inter); gate_w (E, D) and gate_bias
    (E,) are fp32 (check_layer_args raises ValueError otherwise).
    master_weights (optional, bf16 x only): fp32 tensors of the same shapes in
    the order [*w1, *w2, *w3, *sw1, *sw2, *sw3], of which the expert weights
    are bf16 copies; the expert weight gradients then go to the masters, as
    fp32 (the gradients of autocast's casts, computed without a cast pass).
    Returns (y, idx64, weights_x, counts)."""
    E, S, I, I_s = check_layer_args(x, gate_w, gate_bias, w1, w2, w3, sw1, sw2, sw3, k)
    _require_gpu(x, gate_w, gate_bias, *w1)
    weights = [*w1, *w2, *w3, *sw1, *sw2, *sw3]
    masters = list(master_weights) if master_weights is not None else []
    if masters:
        if x.dtype != torch.bfloat16 or len(masters) != len(weights):
            raise ValueError("dsmoe: master_weights need bf16 activations and one fp32 master per expert weight")
        for m, w in zip(masters, weights):
            if m.dtype != torch.float32 or m.shape != w.shape:
                raise ValueError(f"dsmoe: a master weight must be float32 of its copy's shape {tuple(w.shape)}, got "
                                 f"{m.dtype} {tuple(m.shape)}")
    needs_grad = x.requires_grad or gate_w.requires_grad
    for w in (*weights, *masters):
        needs_grad = needs_grad or w.requires_grad
    if training is None:
        training = torch.is_grad_enabled() and needs_grad
    ws = [_c(w) for w in weights]
    y, idx64, wx, counts, _ = moe_fwd_op(_c(x), _c(gate_w), _c(gate_bias), ws, masters, E, S, int(k), int(I),
                                         int(I_s), float(route_scale), bool(training))
    return y, idx64, wx, counts


# ---------------------------------------------------------------------------- operator seam
class _GroupedSwiGLUFn(torch.autograd.Function):
    """_TritonGroupedMoeFunction's contract (models/moe_triton.py:390-501):
    unweighted y_sorted; backward (dsmoe_grouped_swiglu_bwd) recomputes the
    gate/up GEMM and gives dx and fp32-accumulated dW in the weight dtype,
    returning (dx, dw1, dw2, dw3, None, None) like the reference's
    (dx, dw1, dw2, dw3, None)."""

    @staticmethod
    def forward(ctx, x_sorted, w1, w2, w3, expert_offsets, sorted_w=None):
        dev = x_sorted.device
        N, D = x_sorted.shape
        E, I, _ = w1.shape
        d = L.make_dims(N, D, E, 1, I, 0, 0, x_sorted.dtype, 1.0)
        lib = L.load()
        ws = _ws(lib.dsmoe_grouped_swiglu_workspace_size(d), dev)
        y = torch.empty(N, D, dtype=x_sorted.dtype, device=dev)
        p1, k1 = L.ptr_array(list(w1.unbind(0))); p2, k2 = L.ptr_array(list(w2.unbind(0)))
        p3, k3 = L.ptr_array(list(w3.unbind(0)))
        off = _c(expert_offsets.to(torch.int64))
        rc = lib.dsmoe_grouped_swiglu_fwd(L.ptr(x_sorted), p1, p2, p3, L.ptr(sorted_w), L.ptr(off), d, L.ptr(y),
                                          L.ptr(ws), ws.numel(), L.stream_ptr(dev))
        L.check(rc, "dsmoe_grouped_swiglu_fwd")
        ctx.save_for_backward(x_sorted, w1, w2, w3, off)
        return y

    @staticmethod
    def backward(ctx, dy):
        x_sorted, w1, w2, w3, off = ctx.saved_tensors
        dev = x_sorted.device
        N, D = x_sorted.shape
        E, I, _ = w1.shape
        d = L.make_dims(N, D, E, 1, I, 0, 0, x_sorted.dtype, 1.0)
        lib = L.load()
        ws = _ws(lib.dsmoe_grouped_swiglu_bwd_workspace_size(d), dev)
        dx = torch.empty_like(x_sorted)
        dw1, dw2, dw3 = torch.empty_like(w1), torch.empty_like(w2), torch.empty_like(w3)
        arrs = [L.ptr_array(list(t.unbind(0))) for t in (w1, w2, w3, dw1, dw2, dw3)]
        rc = lib.dsmoe_grouped_swiglu_bwd(L.ptr(x_sorted), arrs[0][0], arrs[1][0], arrs[2][0], L.ptr(off),
                                          L.ptr(_c(dy)), d, L.ptr(dx), arrs[3][0], arrs[4][0], arrs[5][0], L.ptr(ws),
                                          ws.numel(), L.stream_ptr(dev))
        L.check(rc, "dsmoe_grouped_swiglu_bwd")
        return dx, dw1, dw2, dw3, None, None


def grouped_moe_dispatch(x_sorted: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, w3: torch.Tensor,
                         sorted_weights: torch.Tensor, expert_offsets: torch.Tensor) -> torch.Tensor:
    """Drop-in for triton_grouped_moe_dispatch (models/moe_triton.py:504-525):
    x_sorted (N,D), w1/w3 (E,I,D), w2 (E,D,I), sorted_weights (N,), expert_offsets
    (E+1,) int64.  The gate weight is applied outside the autograd Function so
    routing receives gradients, as in the reference; without grad it is fused
    into the down-projection epilogue."""
    _require_gpu(x_sorted, w1, w2, w3, expert_offsets)
    if w1.dim() != 3 or w2.dim() != 3 or w3.dim() != 3:
        raise ValueError("dsmoe: w1/w3 must be (E, I, D) and w2 (E, D, I)")
    if x_sorted.dtype != w1.dtype or w1.dtype != w2.dtype or w2.dtype != w3.dtype:
        raise ValueError("dsmoe: x_sorted and expert weights must share one dtype")
    xs, a, b, c = _c(x_sorted), _c(w1), _c(w2), _c(w3)
    needs_grad = torch.is_grad_enabled() and any(t.requires_grad for t in (x_sorted, w1, w2, w3, sorted_weights))
    # the reference returns out * sorted_weights.unsqueeze(-1) with torch's
    # type promotion (an fp32 weight over a bf16 out gives fp32)
    out_dtype = torch.result_type(x_sorted, sorted_weights)
    if not needs_grad and out_dtype == x_sorted.dtype:
        # weight fused into the down-projection epilogue (fp32 product, one rounding)
        sw = _c(sorted_weights.float())
        return _GroupedSwiGLUFn.forward(_NoCtx(), xs, a, b, c, expert_offsets, sw)
    if not needs_grad:
        out = _GroupedSwiGLUFn.forward(_NoCtx(), xs, a, b, c, expert_offsets, None)
    else:
        out = _GroupedSwiGLUFn.apply(xs, a, b, c, expert_offsets)
    return out * sorted_weights.unsqueeze(-1)


class _NoCtx:
    def save_for_backward(self, *a):
        pass
