"""Greedy token selection on the GPU (mm_argmax_rows).

Replaces ``mx.argmax(logits[:, -1, :], axis=-1)`` in generate_fast's greedy step
(mamba_metal/generate.py:91-93).  Ties go to the lowest index and NaN beats every
number, as torch.argmax does.
"""

from __future__ import annotations

import torch

from mamba_metal_amd import _lib


def argmax_rows(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """logits (rows, n) with unit inner stride -> int64 (rows,) indices."""
    lib = _lib.load()
    dev = _lib.require_cuda(logits, out)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("argmax_rows takes a (rows, n) tensor with unit inner stride")
    rows, n = logits.shape
    if out is None:
        out = torch.empty((rows,), dtype=torch.int64, device=dev)
    if out.shape != (rows,) or out.dtype != torch.int64 or not out.is_contiguous():
        raise ValueError("out must be a contiguous int64 (rows,) tensor")
    with _lib.on_device(dev):
        st = lib.mm_argmax_rows(logits.data_ptr(), rows, n, logits.stride(0),
                                _lib.dtype_code(logits.dtype), out.data_ptr(), _lib.stream_of(dev))
    _lib.check(st, "mm_argmax_rows")
    return out
