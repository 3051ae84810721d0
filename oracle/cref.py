"""ctypes wrapper of the C oracle (``combine_ref.c``) -- TEST INFRASTRUCTURE ONLY.

Inputs are numpy arrays on the host.  Expert buffers of bf16/f16 are passed as uint16 bit
patterns.  dtype codes: 0 = f32, 1 = bf16, 2 = f16 (include/fastmoe_amd.h).
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Sequence

import numpy as np

from . import build as _build

_LIB = None
F32, BF16, F16 = 0, 1, 2

_p = ctypes.c_void_p
_i64 = ctypes.c_int64


def lib():
    global _LIB
    if _LIB is None:
        path = _build.LIB
        if not path.exists():
            _build.build()
        l = ctypes.CDLL(str(path))
        l.oracle_combine_fwd.restype = _i64
        l.oracle_combine_fwd.argtypes = [_p, _p, _i64, ctypes.c_int, _p, _p, _i64, _i64, _p]
        l.oracle_combine_bwd.restype = None
        l.oracle_combine_bwd.argtypes = [_p, _p, _i64, ctypes.c_int, _p, _p, _i64, _i64, _p, _p, _p]
        l.oracle_plan.restype = None
        l.oracle_plan.argtypes = [_p, _i64, _i64, _p, _p]
        l.oracle_metadata.restype = _i64
        l.oracle_metadata.argtypes = [_p, _i64, _p, _p]
        l.oracle_round_f32.restype = None
        l.oracle_round_f32.argtypes = [_p, _i64, ctypes.c_int, _p]
        l.oracle_widen_f32.restype = None
        l.oracle_widen_f32.argtypes = [_p, _i64, ctypes.c_int, _p]
        l.oracle_permute.restype = _i64
        l.oracle_permute.argtypes = [_p, _i64, _i64, _i64, _p, _p, _p, _p]
        _LIB = l
    return _LIB


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _dtype_code(a: np.ndarray, code: int | None) -> int:
    if code is not None:
        return code
    if a.dtype == np.float32:
        return F32
    raise ValueError("16-bit buffers are uint16 bit patterns: pass the dtype code")


def metadata(rows: Sequence[int]):
    rows_a = np.ascontiguousarray(rows, dtype=np.int64)
    E = len(rows_a)
    off = np.zeros(E + 1, dtype=np.int64)
    mx = np.zeros(1, dtype=np.int64)
    lib().oracle_metadata(_ptr(rows_a), E, _ptr(off), _ptr(mx))
    return off, int(mx[0])


def combine_fwd(xs: Sequence[np.ndarray], idx: np.ndarray, w: np.ndarray, T: int, D: int,
                x_dtype: int | None = None, acc: np.ndarray | None = None):
    """fp32 accumulator [T, D] after the ordered combine; returns (acc, skipped_rows)."""
    xs = [np.ascontiguousarray(x) for x in xs]
    code = _dtype_code(xs[0], x_dtype)
    rows = np.array([x.shape[0] for x in xs], dtype=np.int64)
    ptrs = np.array([_ptr(x) for x in xs], dtype=np.uint64)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.zeros((T, D), dtype=np.float32) if acc is None else np.ascontiguousarray(acc, np.float32).copy()
    bad = lib().oracle_combine_fwd(_ptr(ptrs), _ptr(rows), len(xs), code, _ptr(idx), _ptr(w), T, D,
                                   _ptr(out))
    return out, int(bad)


def combine_bwd(xs: Sequence[np.ndarray], idx: np.ndarray, w: np.ndarray, T: int, D: int,
                grad_out: np.ndarray, x_dtype: int | None = None, want_x=True, want_w=True):
    """(grad_x [N, D] in the experts' storage dtype, grad_w [N] float64)."""
    xs = [np.ascontiguousarray(x) for x in xs]
    code = _dtype_code(xs[0], x_dtype)
    rows = np.array([x.shape[0] for x in xs], dtype=np.int64)
    ptrs = np.array([_ptr(x) for x in xs], dtype=np.uint64)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    w = np.ascontiguousarray(w, dtype=np.float32)
    go = np.ascontiguousarray(grad_out)
    N = int(rows.sum())
    gx = np.zeros((N, D), dtype=xs[0].dtype) if want_x else None
    gw = np.zeros(N, dtype=np.float64) if want_w else None
    lib().oracle_combine_bwd(_ptr(ptrs), _ptr(rows), len(xs), code, _ptr(idx), _ptr(w), T, D,
                             _ptr(go), _ptr(gx) if gx is not None else None,
                             _ptr(gw) if gw is not None else None)
    return gx, gw


def plan(idx: np.ndarray, T: int):
    """(row_ptr int32[T + 2], g_list int32[N]) of the token-major inverse."""
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    N = idx.shape[0]
    row_ptr = np.zeros(T + 2, dtype=np.int32)
    g_list = np.zeros(N, dtype=np.int32)
    lib().oracle_plan(_ptr(idx), N, T, _ptr(row_ptr), _ptr(g_list))
    return row_ptr, g_list


def round_to(a: np.ndarray, code: int) -> np.ndarray:
    """Round fp32 values to f32/bf16/f16 storage (bf16/f16 as uint16 bits), nearest-even."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.float32 if code == F32 else np.uint16)
    lib().oracle_round_f32(_ptr(a), a.size, code, _ptr(out))
    return out


def widen(a: np.ndarray, code: int) -> np.ndarray:
    """fp32 values of f32/bf16/f16 storage."""
    a = np.ascontiguousarray(a)
    out = np.empty(a.shape, dtype=np.float32)
    lib().oracle_widen_f32(_ptr(a), a.size, code, _ptr(out))
    return out


def permute(ids: np.ndarray, E: int):
    """Dispatch permutation of ids[T, k] (tiny_model.py:108-138, stable):
    (counts int64[E], offsets int64[E + 1], rev int64[N], slot_pos int32[N], invalid_slots)."""
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    T, k = ids.shape
    N = T * k
    counts = np.zeros(E, dtype=np.int64)
    offsets = np.zeros(E + 1, dtype=np.int64)
    rev = np.zeros(N, dtype=np.int64)
    slot_pos = np.zeros(N, dtype=np.int32)
    bad = lib().oracle_permute(_ptr(ids), T, k, E, _ptr(counts), _ptr(offsets), _ptr(rev),
                               _ptr(slot_pos))
    return counts, offsets, rev, slot_pos, int(bad)
