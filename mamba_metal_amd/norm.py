"""Fused residual add + RMSNorm (replaces ``x + mixer(...)`` and the next nn.RMSNorm,
mamba_metal/mamba_model.py:40,48,53,57,69)."""

from __future__ import annotations

import torch

from mamba_metal_amd import _lib


def add_rmsnorm(resid, add, weight, eps, out=None):
    """resid (..., dim) is updated in place to resid + add (add may be None); returns
    RMSNorm(resid) * weight in resid's dtype.  Rows may be strided; columns contiguous."""
    lib = _lib.load()
    dev = _lib.require_cuda(resid, add, weight, out)
    dim = resid.shape[-1]
    r2 = resid.reshape(-1, dim)
    if r2.data_ptr() != resid.data_ptr() or r2.stride(1) != 1:
        raise ValueError("resid must be viewable as (rows, dim) with unit column stride")
    a2 = None if add is None else add.reshape(-1, dim)
    if a2 is not None and (a2.shape != r2.shape or a2.stride(1) != 1 or a2.dtype != resid.dtype):
        raise ValueError("add must match resid")
    if out is None:
        out = torch.empty_like(resid)
    o2 = out.reshape(-1, dim)
    with _lib.on_device(dev):
        st = lib.mm_add_rmsnorm(r2.data_ptr(), _lib.ptr(a2), weight.data_ptr(), o2.data_ptr(),
                                r2.shape[0], dim, r2.stride(0), 0 if a2 is None else a2.stride(0),
                                o2.stride(0), float(eps), _lib.dtype_code(resid.dtype),
                                _lib.dtype_code(weight.dtype), _lib.stream_of(dev))
    _lib.check(st, "mm_add_rmsnorm")
    return out
