"""ctypes binding of libdsmoe.so (the C ABI declared in include/dsmoe.h).

Loading fails with ImportError when the library has not been built; there is
no other backend.  Status codes map to exceptions the way the reference's
operator signals them (models/moe_triton.py:377-384,518-523): bad or
unsupported shapes raise ValueError, HIP errors raise RuntimeError.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Iterable, Sequence

import torch

LIB_PATH = Path(__file__).resolve().parent / "libdsmoe.so"

DSMOE_OK = 0
DSMOE_ERR_INVALID = -1
DSMOE_ERR_UNSUPPORTED = -2
DSMOE_ERR_WORKSPACE = -3
DSMOE_ERR_HIP = -4
DSMOE_F32 = 0
DSMOE_BF16 = 1
# forward-workspace buffer ids of dsmoe_moe_fwd_workspace_offset
WS_IDX, WS_WEIGHTS, WS_SEL_SCORES, WS_OFFSETS, WS_SORTED_SLOT, WS_SORTED_TOKEN, WS_SLOT_POS = range(7)
PERMUTE_NOALLOC_BYTES = 2 << 20   # include/dsmoe.h DSMOE_PERMUTE_NOALLOC_BYTES


class Dims(ctypes.Structure):
    """dsmoe_dims (include/dsmoe.h)."""
    _fields_ = [("T", ctypes.c_int32), ("D", ctypes.c_int32), ("E", ctypes.c_int32), ("k", ctypes.c_int32),
                ("I", ctypes.c_int32), ("S", ctypes.c_int32), ("I_s", ctypes.c_int32), ("dtype", ctypes.c_int32),
                ("route_scale", ctypes.c_float)]


class MlaDims(ctypes.Structure):
    """dsmoe_mla_dims (include/dsmoe.h)."""
    _fields_ = [("B", ctypes.c_int32), ("H", ctypes.c_int32), ("S_q", ctypes.c_int32), ("S_kv", ctypes.c_int32),
                ("R", ctypes.c_int32), ("D_nope", ctypes.c_int32), ("D_rope", ctypes.c_int32),
                ("D_v", ctypes.c_int32), ("dtype", ctypes.c_int32), ("is_causal", ctypes.c_int32),
                ("q_start", ctypes.c_int32), ("softmax_scale", ctypes.c_float)]


P = ctypes.c_void_p
PP = ctypes.POINTER(ctypes.c_void_p)
DIMS = ctypes.POINTER(Dims)
I32 = ctypes.c_int
F32 = ctypes.c_float
SZ = ctypes.c_size_t

_SIGNATURES = {
    "dsmoe_last_error": ([], ctypes.c_char_p),
    "dsmoe_version": ([], I32),
    "dsmoe_gate_fwd": ([P, P, P, DIMS, P, P, P, P, P, P, P, P], I32),
    "dsmoe_route_from_logits": ([P, P, DIMS, P, P, P, P, P, P, P], I32),
    "dsmoe_permute_workspace_size": ([DIMS], SZ),
    "dsmoe_permute": ([P, DIMS, P, P, P, P, P, P, P, P, P, P, SZ, P], I32),
    "dsmoe_permute_noalloc": ([P, DIMS, P, P, P, P, P, P, P, P, P, P], I32),
    "dsmoe_grouped_swiglu_workspace_size": ([DIMS], SZ),
    "dsmoe_grouped_swiglu_fwd": ([P, PP, PP, PP, P, P, DIMS, P, P, SZ, P], I32),
    "dsmoe_grouped_swiglu_bwd_workspace_size": ([DIMS], SZ),
    "dsmoe_grouped_swiglu_bwd": ([P, PP, PP, PP, P, P, DIMS, P, PP, PP, PP, P, SZ, P], I32),
    "dsmoe_combine_fwd": ([P, P, P, P, DIMS, P, P], I32),
    "dsmoe_moe_fwd_workspace_size": ([DIMS, I32], SZ),
    "dsmoe_moe_fwd": ([P, P, P, PP, PP, PP, PP, PP, PP, DIMS, I32, P, P, P, P, P, P, SZ, P], I32),
    "dsmoe_moe_bwd_workspace_size": ([DIMS], SZ),
    "dsmoe_moe_bwd_ex": ([P, P, PP, PP, PP, PP, PP, PP, DIMS, P, P, P, P, PP, PP, PP, PP, PP, PP, I32, P, SZ, P], I32),
    "dsmoe_moe_bwd": ([P, P, PP, PP, PP, PP, PP, PP, DIMS, P, P, P, P, PP, PP, PP, PP, PP, PP, P, SZ, P], I32),
    "dsmoe_update_bias": ([P, P, I32, F32, F32, F32, P], I32),
    "dsmoe_update_bias_f32": ([P, P, I32, F32, F32, F32, P], I32),
    "dsmoe_moe_fwd_workspace_offset": ([DIMS, I32, I32], SZ),
    "dsmoe_timing_enable": ([I32], I32),
    "dsmoe_timing_read": ([ctypes.POINTER(ctypes.c_double), I32, ctypes.POINTER(ctypes.c_int)], I32),
    "dsmoe_timing_stage_name": ([I32], ctypes.c_char_p),
    "dsmoe_mla_attn_workspace_size": ([ctypes.POINTER(MlaDims)], SZ),
    "dsmoe_mla_attn_fwd": ([P, P, P, P, P, P, ctypes.POINTER(MlaDims), P, P, SZ, P], I32),
    "dsmoe_mla_attn_fwd_lse": ([P, P, P, P, P, P, ctypes.POINTER(MlaDims), P, P, P, SZ, P], I32),
    "dsmoe_mla_attn_bwd_workspace_size": ([ctypes.POINTER(MlaDims)], SZ),
    "dsmoe_mla_attn_kv": ([P, P, P, P, ctypes.POINTER(MlaDims), P, SZ, P], I32),
    "dsmoe_mla_attn_bwd": ([P, P, ctypes.POINTER(MlaDims), P, SZ, P, P, P, P, P, P, P, P, SZ, P], I32),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libdsmoe.so once; ImportError if it is missing."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"dsmoe: {LIB_PATH} is not built; run __graft_entry__.build() "
                              "(or `python -m dsmoe.build` in deepseek-v3-lite_amd/)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


def exported_symbols() -> Sequence[str]:
    return tuple(_SIGNATURES)


def check(rc: int, what: str) -> None:
    if rc == DSMOE_OK:
        return
    msg = load().dsmoe_last_error().decode(errors="replace")
    if rc in (DSMOE_ERR_INVALID, DSMOE_ERR_UNSUPPORTED, DSMOE_ERR_WORKSPACE):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (status {rc})")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.bfloat16:
        return DSMOE_BF16
    if dtype == torch.float32:
        return DSMOE_F32
    raise ValueError(f"dsmoe: unsupported activation dtype {dtype} (float32 or bfloat16)")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def ptr_array(ts: Iterable[torch.Tensor]):
    ts = list(ts)
    arr = (ctypes.c_void_p * max(len(ts), 1))(*[t.data_ptr() for t in ts])
    return ctypes.cast(arr, PP), arr  # keep `arr` alive while the call runs


def stream_ptr(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def timing_enable(on: bool) -> None:
    load().dsmoe_timing_enable(1 if on else 0)


def timing_read() -> tuple:
    """-> ({stage name: total ms since enable}, number of recorded calls)."""
    lib = load()
    buf = (ctypes.c_double * 64)()
    n = ctypes.c_int(0)
    ns = lib.dsmoe_timing_read(buf, 64, ctypes.byref(n))
    if ns < 0:
        check(ns, "dsmoe_timing_read")
    names = [lib.dsmoe_timing_stage_name(i).decode() for i in range(ns)]
    return {nm: buf[i] for i, nm in enumerate(names) if buf[i] > 0.0}, n.value


def make_dims(T, D, E, k, I, S, I_s, dtype: torch.dtype, route_scale: float) -> Dims:
    return Dims(int(T), int(D), int(E), int(k), int(I), int(S), int(I_s), dtype_code(dtype), float(route_scale))
