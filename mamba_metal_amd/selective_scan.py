"""selective_scan(): the op API of the selective-scan inference path.

Same signature, shapes, dtype rules and error behaviour as the reference's
mamba_metal/selective_scan.py:23-80:

  u, delta: (batch, dim, seqlen); A: (dim, dstate); B, C: (batch, dstate, seqlen);
  D: (dim,) optional; z: (batch, dim, seqlen) optional (gate SiLU(z));
  delta_softplus applies softplus (cutoff 20) to delta;
  returns y (u.shape, u.dtype) or (y, ssm_state_out (batch, dim, dstate) float32).

Shape violations raise AssertionError with the reference's conditions
(selective_scan.py:46-50).  Arithmetic is fp32 inside the HIP kernel for every
dtype (the reference's generated MSL promotes half loads to float).  Inputs may
be any strided view -- no contiguous copies are made; the kernel reads strides.
y has u's layout when u is a channel-contiguous view (e.g. a transposed (batch, seqlen,
dim) tensor), otherwise the (batch, dim, seqlen) row-major layout.
Mixed dtypes are promoted exactly (to float32) and y is rounded back to u.dtype,
which is what the reference's float arithmetic + half store does.
"""

from __future__ import annotations

import torch

from mamba_metal_amd import _lib

TG_SIZE = 1024          # reference constant (selective_scan.py:8); kept for API parity
MAX_DSTATE = _lib.MAX_DSTATE


def _strides3(t):
    s = t.stride()
    return (_lib._i64a3)(*s)


def _common_dtype(*ts):
    dts = {t.dtype for t in ts if t is not None}
    if len(dts) == 1:
        return dts.pop()
    return torch.float32


_STATUS: dict = {}   # device -> persistent int32 status word every scan ORs into
_WS_BYTES: dict = {}  # (batch, dim, dstate, seqlen) -> workspace bytes (a pure function)


def _dev_of(device) -> torch.device:
    if device is None:
        return torch.device("cuda", torch.cuda.current_device())
    dev = torch.device(device)
    return dev if dev.index is not None else torch.device("cuda", torch.cuda.current_device())


def _status_word(dev: torch.device) -> torch.Tensor:
    w = _STATUS.get(dev)
    if w is None:
        # a normal tensor even when the first scan runs under inference_mode, so that
        # reset_scan_status() may clear it anywhere
        with torch.inference_mode(False):
            w = torch.zeros(1, dtype=torch.int32, device=dev)
        _STATUS[dev] = w
    return w


def scan_status(device=None) -> int:
    """OR of the status bits of every scan on ``device`` since the last
    ``reset_scan_status`` (synchronises that device).  0 when every time segment of
    every call received its predecessor's carried state; nonzero
    (``_lib.SCAN_STATUS_HANDOFF_TIMEOUT``) when a bounded hand-off wait gave up -- not
    expected to happen -- and some call's y is not valid."""
    dev = _dev_of(device)
    w = _STATUS.get(dev)
    if w is None:
        return 0
    torch.cuda.synchronize(dev)
    return int(w.item())


def reset_scan_status(device=None) -> None:
    """Clear the status word of ``device`` (ordered on its current stream)."""
    dev = _dev_of(device)
    w = _STATUS.get(dev)
    if w is not None:
        w.zero_()


def selective_scan_into(u, delta, A, B, C, y, *, D=None, z=None, delta_softplus=False,
                        state_out=None, handoff_timeout_us: int = 0):
    """Run the scan writing into a caller-provided y (any strides, shape of u).

    ``state_out`` (batch, dim, dstate) contiguous float32 or None.  Used by the
    model to pass its (batch, seqlen, dim) buffers as transposed views.
    ``handoff_timeout_us`` bounds a time segment's wait for its predecessor's carried
    state (0 = the library default, 2 s); a wait that expires sets the bit
    ``_lib.SCAN_STATUS_HANDOFF_TIMEOUT`` of ``scan_status()`` and y is not valid."""
    lib = _lib.load()
    dev = _lib.require_cuda(u, delta, A, B, C, D, z, y, state_out)
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    xdt = _common_dtype(u, delta, z)
    if xdt != u.dtype or y.dtype != xdt:
        raise TypeError("selective_scan_into needs u, delta, z and y of one dtype")
    bcdt = _common_dtype(B, C)
    if B.dtype != bcdt:
        B = B.float()
    if C.dtype != bcdt:
        C = C.float()
    A = A if A.dtype == torch.float32 else A.float()
    if D is not None and D.dtype != torch.float32:
        D = D.float()
    if state_out is not None:
        assert state_out.shape == (batch, dim, dstate) and state_out.is_contiguous()
        assert state_out.dtype == torch.float32

    key = (batch, dim, dstate, seqlen)
    ws_bytes = _WS_BYTES.get(key)
    if ws_bytes is None:
        ws_bytes = _WS_BYTES.setdefault(key, lib.mm_selective_scan_workspace_size(*key))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if ws_bytes else None

    p = _lib.ScanParams()
    p.u, p.delta, p.A, p.B, p.C = u.data_ptr(), delta.data_ptr(), A.data_ptr(), B.data_ptr(), C.data_ptr()
    p.D = _lib.ptr(D)
    p.z = _lib.ptr(z)
    p.y = y.data_ptr()
    p.state_out = _lib.ptr(state_out)
    p.workspace = _lib.ptr(ws)
    p.workspace_bytes = ws_bytes
    p.batch, p.dim, p.dstate, p.seqlen = batch, dim, dstate, seqlen
    p.u_stride = _strides3(u)
    p.delta_stride = _strides3(delta)
    p.z_stride = _strides3(z) if z is not None else (_lib._i64a3)(0, 0, 0)
    p.y_stride = _strides3(y)
    p.B_stride = _strides3(B)
    p.C_stride = _strides3(C)
    p.A_stride = (_lib._i64a2)(*A.stride())
    p.D_stride = D.stride(0) if D is not None else 0
    p.x_dtype = _lib.dtype_code(xdt)
    p.bc_dtype = _lib.dtype_code(bcdt)
    p.delta_softplus = 1 if delta_softplus else 0
    p.handoff_timeout_us = int(handoff_timeout_us)
    p.status = _status_word(dev).data_ptr()
    with _lib.on_device(dev):
        st = lib.mm_selective_scan_fwd_strided(p, _lib.stream_of(dev))
    _lib.check(st, "mm_selective_scan_fwd_strided")
    return y


def selective_scan(
    u: torch.Tensor,
    delta: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    C: torch.Tensor,
    *,
    D: torch.Tensor | None = None,
    z: torch.Tensor | None = None,
    delta_softplus: bool = False,
    return_state: bool = False,
):
    """Mamba selective scan with optional D / z / softplus (see module docstring)."""
    batch, dim, seqlen = u.shape
    _, dstate = A.shape
    if not delta.shape == u.shape:
        raise AssertionError(f"delta.shape {tuple(delta.shape)} != u.shape {tuple(u.shape)}")
    if not (B.shape == (batch, dstate, seqlen) == C.shape):
        raise AssertionError(
            f"B {tuple(B.shape)} and C {tuple(C.shape)} must both be {(batch, dstate, seqlen)}")
    if not dstate <= MAX_DSTATE:
        raise AssertionError(f"dstate={dstate} > MAX_DSTATE={MAX_DSTATE}")
    if z is not None and z.shape != u.shape:
        raise AssertionError(f"z.shape {tuple(z.shape)} != u.shape {tuple(u.shape)}")
    if D is not None and D.shape != (dim,):
        raise AssertionError(f"D.shape {tuple(D.shape)} != ({dim},)")
    _lib.require_cuda(u, delta, A, B, C, D, z)

    if batch * dim * seqlen == 0:
        # Nothing to scan; h stays at its zero initial value (the reference's carry init).
        y = torch.empty((batch, dim, seqlen), dtype=u.dtype, device=u.device)
        if return_state:
            return y, torch.zeros((batch, dim, dstate), dtype=torch.float32, device=u.device)
        return y

    out_dtype = u.dtype
    xdt = _common_dtype(u, delta, z)
    _lib.dtype_code(xdt)
    uu = u if u.dtype == xdt else u.to(xdt)
    dd = delta if delta.dtype == xdt else delta.to(xdt)
    zz = z if (z is None or z.dtype == xdt) else z.to(xdt)

    # y takes u's layout when u is a channel-contiguous view (a transposed (batch, seqlen,
    # dim) tensor, as the model passes): with every operand along channels the kernel runs
    # its channel-contiguous fast path instead of the strided one a (batch, dim, seqlen)
    # y would force (B=64, D=5120, L=512 fp16: 1.26 -> ~1.0 ms).
    if uu.stride(1) == 1 and uu.stride(2) != 1:
        y = torch.empty_like(uu, dtype=xdt)
    else:
        y = torch.empty((batch, dim, seqlen), dtype=xdt, device=u.device)
    state = torch.empty((batch, dim, dstate), dtype=torch.float32, device=u.device) \
        if return_state else None
    selective_scan_into(uu, dd, A, B, C, y, D=D, z=zz, delta_softplus=delta_softplus,
                        state_out=state)
    if y.dtype != out_dtype:
        y = y.to(out_dtype)
    if return_state:
        return y, state
    return y
