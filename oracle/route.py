"""ctypes wrapper and builder for oracle/route_ref.c — TEST INFRASTRUCTURE ONLY.

See route_ref.c for the reference lines each function restates."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "route_ref.c"
LIB = HERE / "liboracle_route.so"

_lib = None


def build(force: bool = True) -> Path:
    """Compile route_ref.c with gcc into oracle/liboracle_route.so."""
    if force or not LIB.exists():
        tmp = LIB.with_suffix(".so.tmp")
        subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-std=c99", str(SRC), "-o", str(tmp), "-lm"],
                       check=True)
        tmp.replace(LIB)
    return LIB


def _load():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        lib = ctypes.CDLL(str(LIB))
        P = ctypes.c_void_p
        lib.oracle_route.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, P, P, P, P]
        lib.oracle_route.restype = ctypes.c_int
        lib.oracle_permute.argtypes = [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P]
        lib.oracle_permute.restype = ctypes.c_int
        lib.oracle_min_margin.argtypes = [P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        lib.oracle_min_margin.restype = ctypes.c_float
        lib.oracle_sigmoid.argtypes = [ctypes.c_float]
        lib.oracle_sigmoid.restype = ctypes.c_float
        _lib = lib
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def route(logits: np.ndarray, bias: np.ndarray, k: int, route_scale: float = 1.0):
    """-> (idx int32 (T,k), weights f32 (T,k), sel_scores f32 (T,k), counts int32 (E,))"""
    lib = _load()
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    bias = np.ascontiguousarray(bias, dtype=np.float32)
    T, E = logits.shape
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    s = np.empty((T, k), np.float32)
    c = np.empty((E,), np.int32)
    rc = lib.oracle_route(_p(logits), _p(bias), T, E, k, route_scale, _p(idx), _p(w), _p(s), _p(c))
    if rc != 0:
        raise ValueError(f"oracle_route failed ({rc})")
    return idx, w, s, c


def permute(idx: np.ndarray, E: int):
    """-> (offsets (E+1), sorted_slot (N), sorted_token (N), slot_pos (N)) int32"""
    lib = _load()
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    T, k = idx.shape
    N = T * k
    off = np.empty((E + 1,), np.int32)
    ss = np.empty((N,), np.int32)
    st = np.empty((N,), np.int32)
    sp = np.empty((N,), np.int32)
    rc = lib.oracle_permute(_p(idx), T, k, E, _p(off), _p(ss), _p(st), _p(sp))
    if rc != 0:
        raise ValueError(f"oracle_permute failed ({rc})")
    return off, ss, st, sp


def min_margin(logits: np.ndarray, bias: np.ndarray, k: int) -> float:
    lib = _load()
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    bias = np.ascontiguousarray(bias, dtype=np.float32)
    T, E = logits.shape
    return float(lib.oracle_min_margin(_p(logits), _p(bias), T, E, k))


def sigmoid(x: float) -> float:
    return float(_load().oracle_sigmoid(x))
