"""Fused O(1) decode SSM step (mamba_metal/mamba_block.py:183-195).

``ssm_step`` updates the resident fp32 SSM state in place and returns y:
  dt' = softplus(dt + dt_bias); h = exp(dt'*A)*h + dt'*x*B; y = (<h, C> + D*x) * silu(z)
"""

from __future__ import annotations

import torch

from mamba_metal_amd import _lib


def ssm_step(ssm_state, x, dt, A, B, C, *, D=None, z=None, dt_bias=None, dt_softplus=True,
             out=None):
    """ssm_state (batch, dim, dstate) contiguous float32 (updated in place);
    x, dt, z: (batch, dim); B, C: (batch, dstate) -- all with unit inner stride and
    one dtype; A (dim, dstate) contiguous float32; D, dt_bias (dim,) float32."""
    lib = _lib.load()
    dev = _lib.require_cuda(ssm_state, x, dt, A, B, C, D, z, dt_bias, out)
    batch, dim = x.shape
    dstate = A.shape[1]
    if ssm_state.shape != (batch, dim, dstate) or not ssm_state.is_contiguous() \
            or ssm_state.dtype != torch.float32:
        raise ValueError(f"ssm_state must be contiguous float32 {(batch, dim, dstate)}")
    if A.dtype != torch.float32 or not A.is_contiguous():
        A = A.float().contiguous()
    if D is not None and D.dtype != torch.float32:
        D = D.float()
    if dt_bias is not None and dt_bias.dtype != torch.float32:
        dt_bias = dt_bias.float()
    for name, t in (("x", x), ("dt", dt), ("B", B), ("C", C), ("z", z)):
        if t is not None and (t.dtype != x.dtype or t.stride(-1) != 1):
            raise ValueError(f"{name} must have x's dtype and unit inner stride")
    if out is None:
        out = torch.empty((batch, dim), dtype=x.dtype, device=dev)
    with _lib.on_device(dev):
        st = lib.mm_decode_ssm_step(
            ssm_state.data_ptr(), x.data_ptr(), dt.data_ptr(), _lib.ptr(dt_bias), A.data_ptr(),
            B.data_ptr(), C.data_ptr(), _lib.ptr(D), _lib.ptr(z), out.data_ptr(),
            batch, dim, dstate, x.stride(0), dt.stride(0), B.stride(0), C.stride(0),
            z.stride(0) if z is not None else 0, out.stride(0),
            _lib.dtype_code(x.dtype), 1 if dt_softplus else 0, _lib.stream_of(dev))
    _lib.check(st, "mm_decode_ssm_step")
    return out


FUSED_DSTATE = 16
FUSED_MAX_RANK = 256


def dtproj_fused_ok(dstate: int, rank: int, x_dtype, w_dtype) -> bool:
    """Shapes the fused kernel takes: dstate 16 (every Mamba-1 checkpoint), rank <= 256,
    dt_proj weight in the activation dtype."""
    return dstate == FUSED_DSTATE and 1 <= rank <= FUSED_MAX_RANK and x_dtype == w_dtype


def ssm_step_dtproj(ssm_state, x, dt_in, dt_weight, A, B, C, *, dt_bias=None, D=None, z=None,
                    out=None):
    """Decode step including the dt projection:
    dt = softplus(dt_in @ dt_weight.T + dt_bias), then the update of ``ssm_step``.

    dt_in (batch, rank) is typically the dt slice of x_proj's output; dt_weight
    (dim, rank) and dt_bias (dim,) are dt_proj's parameters.  Shapes outside
    ``dtproj_fused_ok`` run the projection as a GEMM followed by ``ssm_step``."""
    lib = _lib.load()
    dev = _lib.require_cuda(ssm_state, x, dt_in, dt_weight, A, B, C, D, z, dt_bias, out)
    batch, dim = x.shape
    dstate = A.shape[1]
    rank = dt_in.shape[1]
    if ssm_state.shape != (batch, dim, dstate) or not ssm_state.is_contiguous() \
            or ssm_state.dtype != torch.float32:
        raise ValueError(f"ssm_state must be contiguous float32 {(batch, dim, dstate)}")
    if dt_weight.shape != (dim, rank) or dt_weight.stride(1) != 1:
        raise ValueError(f"dt_weight must be ({dim}, {rank}) with unit inner stride")
    if dt_bias is not None and (dt_bias.dtype != dt_weight.dtype or not dt_bias.is_contiguous()):
        raise ValueError("dt_bias must be contiguous with dt_weight's dtype")
    if not dtproj_fused_ok(dstate, rank, x.dtype, dt_weight.dtype):
        dt = torch.nn.functional.linear(dt_in, dt_weight.to(x.dtype),
                                        None if dt_bias is None else dt_bias.to(x.dtype))
        return ssm_step(ssm_state, x, dt, A, B, C, D=D, z=z, dt_softplus=True, out=out)
    if A.dtype != torch.float32 or not A.is_contiguous():
        A = A.float().contiguous()
    if D is not None and D.dtype != torch.float32:
        D = D.float()
    for name, t in (("x", x), ("dt_in", dt_in), ("B", B), ("C", C), ("z", z)):
        if t is not None and (t.dtype != x.dtype or t.stride(-1) != 1):
            raise ValueError(f"{name} must have x's dtype and unit inner stride")
    if out is None:
        out = torch.empty((batch, dim), dtype=x.dtype, device=dev)
    with _lib.on_device(dev):
        st = lib.mm_decode_ssm_step_dtproj(
            ssm_state.data_ptr(), x.data_ptr(), dt_in.data_ptr(), dt_weight.data_ptr(),
            _lib.ptr(dt_bias), A.data_ptr(), B.data_ptr(), C.data_ptr(), _lib.ptr(D), _lib.ptr(z),
            out.data_ptr(), batch, dim, dstate, rank, x.stride(0), dt_in.stride(0),
            dt_weight.stride(0), B.stride(0), C.stride(0), z.stride(0) if z is not None else 0,
            out.stride(0), _lib.dtype_code(x.dtype), _lib.dtype_code(dt_weight.dtype),
            _lib.stream_of(dev))
    _lib.check(st, "mm_decode_ssm_step_dtproj")
    return out
