"""dsmoe_permute_noalloc (static device scratch, no workspace) against
dsmoe_permute (caller workspace) through the C ABI: bit-exact on two calls in
a row, the second smaller than the first, so the second runs over scratch the
first left behind."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _routing(T, E, k, seed):
    rng = np.random.default_rng(seed)
    return np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)


def _permute(lib, L, noalloc, idx, E, x, w):
    T, k = idx.shape
    N = T * k
    d = L.make_dims(T, x.shape[1], E, k, 1, 0, 0, x.dtype, 1.0)
    out = {n: torch.full((N,), -7, dtype=torch.int32, device=DEV) for n in ("sorted_slot", "sorted_token", "slot_pos")}
    out["offsets"] = torch.full((E + 1,), -7, dtype=torch.int32, device=DEV)
    out["counts"] = torch.full((E,), -7, dtype=torch.int32, device=DEV)
    out["x_sorted"] = torch.zeros(N, x.shape[1], dtype=x.dtype, device=DEV)
    out["sorted_w"] = torch.zeros(N, dtype=torch.float32, device=DEV)
    gi = torch.from_numpy(idx).to(DEV)
    args = [L.ptr(gi), d, L.ptr(out["offsets"]), L.ptr(out["sorted_slot"]), L.ptr(out["sorted_token"]),
            L.ptr(out["slot_pos"]), L.ptr(out["counts"]), L.ptr(x), L.ptr(out["x_sorted"]), L.ptr(w),
            L.ptr(out["sorted_w"])]
    if noalloc:
        rc = lib.dsmoe_permute_noalloc(*args, L.stream_ptr(DEV))
    else:
        ws = torch.empty(lib.dsmoe_permute_workspace_size(d), dtype=torch.uint8, device=DEV)
        rc = lib.dsmoe_permute(*args, L.ptr(ws), ws.numel(), L.stream_ptr(DEV))
    L.check(rc, "permute_noalloc" if noalloc else "permute")
    torch.cuda.synchronize()
    return {n: t.cpu() for n, t in out.items()}


def test_permute_noalloc_matches_permute_on_two_calls():
    import dsmoe._lib as L
    lib = L.load()
    for T, E, k, D in ((8192, 64, 6, 64), (100, 16, 4, 48)):
        idx = _routing(T, E, k, seed=T + E)
        x = torch.randn(T, D, dtype=torch.bfloat16, device=DEV)
        w = torch.rand(T, k, dtype=torch.float32, device=DEV)
        ref = _permute(lib, L, False, idx, E, x, w)
        got = _permute(lib, L, True, idx, E, x, w)
        for name in ref:
            assert torch.equal(got[name], ref[name]), (T, E, k, name)
        # and both are the stable (expert, token) order
        order = sorted(range(T * k), key=lambda s: (idx.reshape(-1)[s], s))
        assert np.array_equal(got["sorted_slot"].numpy(), order)
