"""numpy/ctypes front end of the CPU oracle (oracle/ccv1d_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker. The product package never imports it.

All inputs are numpy arrays (converted to contiguous float32 / int32 here); `None` means absent.
Outputs are the fp32 values before the cast to the output dtype (dweight/dbias in float64).
"""

import ctypes
import os
import subprocess

import numpy as np

_DIR = os.path.dirname(os.path.abspath(__file__))
_LIB = os.path.join(_DIR, "libccv1d_oracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64 = ctypes.c_int64


def build() -> str:
    """Compiles the oracle with its Makefile (gcc) and returns the library path."""
    subprocess.run(["make", "-s", "-C", _DIR], check=True)
    return _LIB


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB):
            build()
        lib = ctypes.CDLL(_LIB)
        lib.ccv1d_oracle_fwd.restype = None
        lib.ccv1d_oracle_fwd.argtypes = [_f32p, _f32p, _f32p, _i32p, _f32p, _f32p, _f32p,
                                         _i64, _i64, _i64, _i64, ctypes.c_int]
        lib.ccv1d_oracle_bwd.restype = ctypes.c_int
        lib.ccv1d_oracle_bwd.argtypes = [_f32p, _f32p, _f32p, _i32p, _f32p, _f32p, _f32p,
                                         _f32p, _f32p, _f64p, _f64p,
                                         _i64, _i64, _i64, _i64, ctypes.c_int]
        lib.ccv1d_oracle_set_mutation.restype = None
        lib.ccv1d_oracle_set_mutation.argtypes = [ctypes.c_int]
        _lib = lib
    return _lib


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _p(a, ptype):
    return None if a is None else a.ctypes.data_as(ptype)


def set_mutation(m: int) -> None:
    """Plants mistake number m in the oracle (0 restores it); used to show the pinning tests bite."""
    _load().ccv1d_oracle_set_mutation(int(m))


def fwd(x, weight, bias=None, seq_idx=None, initial_states=None, silu=False, final=False):
    """Returns (out, final_states or None) as float32 arrays."""
    lib = _load()
    x = _f32(x)
    w = _f32(weight)
    b = _f32(bias)
    init = _f32(initial_states)
    seq = None if seq_idx is None else np.ascontiguousarray(seq_idx, dtype=np.int32)
    B, T, D = x.shape
    W = w.shape[1]
    out = np.empty((B, T, D), np.float32)
    fin = np.empty((B, W - 1, D), np.float32) if final else None
    lib.ccv1d_oracle_fwd(_p(x, _f32p), _p(w, _f32p), _p(b, _f32p), _p(seq, _i32p), _p(init, _f32p),
                         _p(out, _f32p), _p(fin, _f32p), B, T, D, W, int(bool(silu)))
    return out, fin


def bwd(x, weight, dout, bias=None, seq_idx=None, initial_states=None, dfinal=None,
        need_dinit=False, silu=False):
    """Returns (dx float32, dinit float32 or None, dweight float64, dbias float64 or None)."""
    lib = _load()
    x = _f32(x)
    w = _f32(weight)
    b = _f32(bias)
    init = _f32(initial_states)
    dy = _f32(dout)
    dfin = _f32(dfinal)
    seq = None if seq_idx is None else np.ascontiguousarray(seq_idx, dtype=np.int32)
    B, T, D = x.shape
    W = w.shape[1]
    dx = np.empty((B, T, D), np.float32)
    dinit = np.empty((B, W - 1, D), np.float32) if need_dinit else None
    dw = np.empty((D, W), np.float64)
    db = np.empty((D,), np.float64) if b is not None else None
    rc = lib.ccv1d_oracle_bwd(_p(x, _f32p), _p(w, _f32p), _p(b, _f32p), _p(seq, _i32p),
                              _p(init, _f32p), _p(dy, _f32p), _p(dfin, _f32p), _p(dx, _f32p),
                              _p(dinit, _f32p), _p(dw, _f64p), _p(db, _f64p), B, T, D, W,
                              int(bool(silu)))
    if rc != 0:
        raise MemoryError("oracle scratch allocation failed")
    return dx, dinit, dw, db
