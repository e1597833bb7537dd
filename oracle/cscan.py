"""ctypes binding of ``scan_ref.c`` -- TEST INFRASTRUCTURE ONLY.

``selective_scan(...)`` mirrors the reference op signature
(mamba_metal/selective_scan.py:23-34) on numpy arrays.  Inputs of any float
dtype are upcast to float32 first, as experiments/10-fp16/test_fp16.py:147-156
does.  Returns (y, state) as float32.

Pinned by tests/test_oracle.py (closed forms, invariants, agreement of the
independent numpy restatement, fp32 vs fp64).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

_LIB_PATH = Path(__file__).resolve().parent / "liboracle_scan.so"
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i64 = ctypes.c_int64


def _load():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            from oracle.build import build

            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        argt = [_f32p] * 10 + [_i64] * 4 + [ctypes.c_int, _i64, _i64]
        for name in ("oracle_selective_scan_f64", "oracle_selective_scan_f32"):
            fn = getattr(lib, name)
            fn.argtypes = argt
            fn.restype = None
        lib.oracle_pair_scan_f64.argtypes = [_f32p] * 4 + [_i64]
        lib.oracle_pair_scan_f64.restype = None
        lib.oracle_num_threads.restype = ctypes.c_int
        lib.oracle_set_num_threads.argtypes = [ctypes.c_int]
        _lib = lib
    return _lib


def _ptr(a):
    if a is None:
        return ctypes.cast(None, _f32p)
    return a.ctypes.data_as(_f32p)


def _f32(a):
    if a is None:
        return None
    return np.ascontiguousarray(np.asarray(a), dtype=np.float32)


def num_threads() -> int:
    return _load().oracle_num_threads()


def set_num_threads(n: int) -> None:
    _load().oracle_set_num_threads(int(n))


def selective_scan(u, delta, A, B, C, *, D=None, z=None, delta_softplus=False,
                   h0=None, precision="f64", channels=None):
    """Sequential CPU scan.  ``channels=(c0, c1)`` restricts the work to flattened
    (batch*dim) channels [c0, c1) (outputs elsewhere stay zero); used to time a
    bounded sample of a large workload."""
    lib = _load()
    u, delta, A, B, C = map(_f32, (u, delta, A, B, C))
    D, z, h0 = _f32(D), _f32(z), _f32(h0)
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    assert delta.shape == u.shape
    assert B.shape == (batch, dstate, seqlen) == C.shape
    y = np.zeros_like(u)
    state = np.zeros((batch, dim, dstate), np.float32)
    c0, c1 = (0, batch * dim) if channels is None else channels
    fn = lib.oracle_selective_scan_f64 if precision == "f64" else lib.oracle_selective_scan_f32
    fn(_ptr(u), _ptr(delta), _ptr(A), _ptr(B), _ptr(C), _ptr(D), _ptr(z), _ptr(h0),
       _ptr(y), _ptr(state), batch, dim, dstate, seqlen, int(bool(delta_softplus)), c0, c1)
    return y, state


def pair_scan(a, b):
    lib = _load()
    a, b = _f32(a), _f32(b)
    a_out = np.zeros_like(a)
    h_out = np.zeros_like(a)
    lib.oracle_pair_scan_f64(_ptr(a), _ptr(b), _ptr(a_out), _ptr(h_out), a.size)
    return a_out, h_out
