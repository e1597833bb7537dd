"""Causal depthwise conv1d (prefill) and the decode conv-window step.

``causal_conv1d`` replaces the MLX ``nn.Conv1d(groups=d_inner, padding=d_conv-1)``
+ slice + ``nn.silu`` of mamba_metal/mamba_block.py:45-52,77-78,129-130 and
captures the conv state of mamba_block.py:118-127 in the same pass.
``conv_step`` replaces the window shift / dot / bias / SiLU of
mamba_block.py:170-177, updating the resident conv state in place.
"""

from __future__ import annotations

import torch

from mamba_metal_amd import _lib


def _w2d(weight):
    """(dim, 1, K) torch/HF conv weight, or (dim, K) -> 2-D view and its strides."""
    w = weight[:, 0, :] if weight.dim() == 3 else weight
    return w, (_lib._i64a2)(*w.stride())


def causal_conv1d(x, weight, bias=None, *, apply_silu=True, out=None, conv_state_out=None):
    """x: (batch, seqlen, dim) channels-last (any strides).

    Returns out (batch, seqlen, dim) (allocated contiguous unless given);
    writes the last ``width`` inputs to conv_state_out (batch, dim, width) if given.
    """
    lib = _lib.load()
    dev = _lib.require_cuda(x, weight, bias, out, conv_state_out)
    batch, seqlen, dim = x.shape
    w, ws = _w2d(weight)
    width = w.shape[1]
    if w.shape[0] != dim:
        raise ValueError(f"weight has {w.shape[0]} channels, x has {dim}")
    if bias is not None and (bias.shape != (dim,) or bias.dtype != w.dtype or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous (dim,) tensor of the weight's dtype")
    if out is None:
        out = torch.empty((batch, seqlen, dim), dtype=x.dtype, device=dev)
    if conv_state_out is not None:
        if conv_state_out.shape != (batch, dim, width) or not conv_state_out.is_contiguous() \
                or conv_state_out.dtype != x.dtype:
            raise ValueError("conv_state_out must be contiguous (batch, dim, width) of x's dtype")
    if x.numel() == 0:
        if conv_state_out is not None:
            conv_state_out.zero_()
        return out
    with _lib.on_device(dev):
        st = lib.mm_causal_conv1d_fwd(
            x.data_ptr(), w.data_ptr(), _lib.ptr(bias), out.data_ptr(), _lib.ptr(conv_state_out),
            batch, seqlen, dim, width, (_lib._i64a3)(*x.stride()), (_lib._i64a3)(*out.stride()),
            ws, _lib.dtype_code(x.dtype), _lib.dtype_code(w.dtype), 1 if apply_silu else 0,
            _lib.stream_of(dev))
    _lib.check(st, "mm_causal_conv1d_fwd")
    return out


def conv_step(conv_state, x, weight, bias=None, *, apply_silu=True, out=None):
    """conv_state (batch, dim, width) contiguous, updated in place; x (batch, dim)
    with unit channel stride.  Returns out (batch, dim) in x's dtype."""
    lib = _lib.load()
    dev = _lib.require_cuda(conv_state, x, weight, bias, out)
    batch, dim = x.shape
    w, ws = _w2d(weight)
    width = w.shape[1]
    if conv_state.shape != (batch, dim, width) or not conv_state.is_contiguous():
        raise ValueError(f"conv_state must be contiguous {(batch, dim, width)}")
    if x.stride(1) != 1:
        raise ValueError("x must have unit channel stride")
    if bias is not None and (bias.shape != (dim,) or bias.dtype != w.dtype or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous (dim,) tensor of the weight's dtype")
    if out is None:
        out = torch.empty((batch, dim), dtype=x.dtype, device=dev)
    with _lib.on_device(dev):
        st = lib.mm_decode_conv_step(
            conv_state.data_ptr(), x.data_ptr(), w.data_ptr(), _lib.ptr(bias), out.data_ptr(),
            batch, dim, width, x.stride(0), out.stride(0), ws,
            _lib.dtype_code(conv_state.dtype), _lib.dtype_code(x.dtype), _lib.dtype_code(w.dtype),
            1 if apply_silu else 0, _lib.stream_of(dev))
    _lib.check(st, "mm_decode_conv_step")
    return out
