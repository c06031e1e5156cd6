"""The C ABI library loads and exports every function include/dsmoe.h declares
(CPU only: no call here reaches the GPU)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "dsmoe.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsmoe_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    import dsmoe._lib as L
    if not L.LIB_PATH.exists():
        from dsmoe import build
        build.build(verbose=False)
    return L.load()


def test_header_declares_the_boundary():
    names = _declared()
    for must in ("dsmoe_gate_fwd", "dsmoe_route_from_logits", "dsmoe_permute", "dsmoe_grouped_swiglu_fwd",
                 "dsmoe_grouped_swiglu_bwd", "dsmoe_combine_fwd", "dsmoe_moe_fwd", "dsmoe_moe_bwd",
                 "dsmoe_update_bias", "dsmoe_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_every_declared_symbol():
    import dsmoe._lib as L
    assert set(L.exported_symbols()) == set(_declared())


def test_dims_struct_matches_header_layout():
    import dsmoe._lib as L
    assert ctypes.sizeof(L.Dims) == 9 * 4
    assert [f[0] for f in L.Dims._fields_] == ["T", "D", "E", "k", "I", "S", "I_s", "dtype", "route_scale"]


def test_validation_errors_without_launch(lib):
    import dsmoe._lib as L
    d = L.Dims(16, 64, 4, 5, 32, 1, 32, L.DSMOE_F32, 1.0)          # k > E
    assert lib.dsmoe_moe_fwd_workspace_size(ctypes.byref(d), 0) == 0
    rc = lib.dsmoe_gate_fwd(None, None, None, ctypes.byref(d), None, None, None, None, None, None, None, None)
    assert rc == L.DSMOE_ERR_INVALID
    assert b"n_activated_experts" in lib.dsmoe_last_error()
    d = L.Dims(16, 64, 4, 2, 32, 1, 32, 7, 1.0)                      # bad dtype
    rc = lib.dsmoe_gate_fwd(None, None, None, ctypes.byref(d), None, None, None, None, None, None, None, None)
    assert rc == L.DSMOE_ERR_UNSUPPORTED
    d = L.Dims(16, 64, 4, 2, 32, 1, 32, L.DSMOE_BF16, 1.0)
    rc = lib.dsmoe_gate_fwd(None, None, None, ctypes.byref(d), None, None, None, None, None, None, None, None)
    assert rc == L.DSMOE_ERR_INVALID and b"NULL" in lib.dsmoe_last_error()
    with pytest.raises(ValueError, match="NULL"):
        L.check(rc, "dsmoe_gate_fwd")


def test_workspace_sizes_are_consistent(lib):
    import dsmoe._lib as L
    d = L.Dims(8192, 2048, 64, 6, 1408, 2, 1408, L.DSMOE_BF16, 1.0)
    inf = lib.dsmoe_moe_fwd_workspace_size(ctypes.byref(d), 0)
    trn = lib.dsmoe_moe_fwd_workspace_size(ctypes.byref(d), 1)
    N = 8192 * 6
    # at least h (N x I), o_slots (N x D), shared h and out; training adds g and u
    assert inf >= 2 * (N * 1408 + N * 2048 + 8192 * 2816 + 8192 * 2048)
    assert trn - inf >= 2 * 2 * (N * 1408 + 8192 * 2816)
    assert lib.dsmoe_permute_workspace_size(ctypes.byref(d)) > 0


def test_workspace_offsets_lie_inside_the_forward_workspace(lib):
    """dsmoe_moe_fwd_workspace_offset: every routing buffer lies inside the
    workspace, 256-byte aligned, without overlaps; unknown ids and bad dims
    give (size_t)-1."""
    import dsmoe._lib as L
    bad = ctypes.c_size_t(-1).value
    for T, train in ((8192, 0), (64, 0), (16384, 1)):
        d = L.Dims(T, 2048, 64, 6, 1408, 2, 1408, L.DSMOE_BF16, 1.0)
        total = lib.dsmoe_moe_fwd_workspace_size(ctypes.byref(d), train)
        N = T * 6
        sizes = {L.WS_IDX: 4 * N, L.WS_WEIGHTS: 4 * N, L.WS_SEL_SCORES: 4 * N, L.WS_OFFSETS: 4 * 65,
                 L.WS_SORTED_SLOT: 4 * N, L.WS_SORTED_TOKEN: 4 * N, L.WS_SLOT_POS: 4 * N}
        spans = []
        for buf, nbytes in sizes.items():
            off = lib.dsmoe_moe_fwd_workspace_offset(ctypes.byref(d), train, buf)
            assert off != bad and off % 256 == 0 and off + nbytes <= total
            spans.append((off, off + nbytes))
        spans.sort()
        assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))
        assert lib.dsmoe_moe_fwd_workspace_offset(ctypes.byref(d), train, 99) == bad
    d = L.Dims(16, 64, 4, 5, 32, 1, 32, L.DSMOE_F32, 1.0)          # k > E
    assert lib.dsmoe_moe_fwd_workspace_offset(ctypes.byref(d), 0, L.WS_IDX) == bad


def test_permute_noalloc_rejects_calls_beyond_its_static_scratch(lib):
    """dsmoe_permute_noalloc refuses (before any device call) a shape whose
    permute scratch exceeds DSMOE_PERMUTE_NOALLOC_BYTES, and names the limit."""
    import dsmoe._lib as L
    d = L.Dims(600000, 64, 64, 6, 32, 0, 32, L.DSMOE_BF16, 1.0)
    assert lib.dsmoe_permute_workspace_size(ctypes.byref(d)) > L.PERMUTE_NOALLOC_BYTES
    rc = lib.dsmoe_permute_noalloc(None, ctypes.byref(d), None, None, None, None, None, None, None, None, None, None)
    assert rc == L.DSMOE_ERR_UNSUPPORTED
    assert str(L.PERMUTE_NOALLOC_BYTES).encode() in lib.dsmoe_last_error()
    small = L.Dims(8192, 2048, 64, 6, 1408, 2, 1408, L.DSMOE_BF16, 1.0)
    assert lib.dsmoe_permute_workspace_size(ctypes.byref(small)) <= L.PERMUTE_NOALLOC_BYTES


def test_probe_is_measurement_tooling_outside_the_layer_abi(lib):
    """The traffic-counter probe (include/dsmoe_probe.h) lives in its own
    library; libdsmoe.so does not export it."""
    import dsmoe._lib as L
    assert not hasattr(lib, "dsmoe_probe_dma_read")
    probe = ctypes.CDLL(str(L.LIB_PATH.with_name("libdsmoe_probe.so")))
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "dsmoe_probe.h").read_text(), flags=re.S)
    for name in set(re.findall(r"\b(dsmoe_[a-z0-9_]+)\s*\(", text)):
        assert hasattr(probe, name), name
