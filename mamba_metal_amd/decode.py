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
    with torch.cuda.device(dev):
        st = lib.mm_decode_ssm_step(
            ssm_state.data_ptr(), x.data_ptr(), dt.data_ptr(), _lib.ptr(dt_bias), A.data_ptr(),
            B.data_ptr(), C.data_ptr(), _lib.ptr(D), _lib.ptr(z), out.data_ptr(),
            batch, dim, dstate, x.stride(0), dt.stride(0), B.stride(0), C.stride(0),
            z.stride(0) if z is not None else 0, out.stride(0),
            _lib.dtype_code(x.dtype), 1 if dt_softplus else 0, _lib.stream_of(dev))
    _lib.check(st, "mm_decode_ssm_step")
    return out
