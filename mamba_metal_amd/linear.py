"""Decode-step projections on the weight-streaming GEMM (mm_decode_linear).

At decode batch M <= 64 the nn.Linear layers of MambaBlock.step
(mamba_metal/mamba_block.py:166-196) and the tied LM head (mamba_model.py:78)
read each weight once and use it M times: HBM-bound on the weight bytes.  These
wrappers run them on libmamba_mi355x's MFMA kernel, with the decode step's
neighbouring element-wise ops folded into its epilogue:

* ``decode_linear(x, w)``                  y = x @ w.T
* ``decode_head_argmax(x, w, ids)``        y = x @ w.T and ids = argmax over each row of y
* ``decode_linear_resid_(resid, x, w)``    resid += round(x @ w.T)   (out_proj + residual add)
* ``decode_linear_resid_norm_(resid, x, w, norm_w, eps)``
      the same, then returns RMSNorm(resid) * norm_w (the next layer's input)
* ``decode_in_proj_conv(x, w, conv_state, conv_w, conv_b, n_conv)``
      xz = x @ w.T; the first n_conv columns go through the conv-window step
      (state shifted in place, SiLU) -> (x_conv, z)

``decode_linear_ok`` says whether a call fits the kernel (f16/bf16, M <= 64,
16-byte aligned rows, K % 64 == 0); callers use torch's GEMM otherwise.

``x_norm=(norm_w, eps)`` (``decode_linear`` and ``decode_in_proj_conv``, M <= 8,
K <= 4096, N <= 16384, see ``norm_in_ok``): x holds raw residual rows and the product uses
RMSNorm(x) * norm_w -- the residual block's pre-norm (mamba_model.py:57) -- computed
in the operand load, bit-identical to ``add_rmsnorm``'s output.

The kernel reads W in a packed operand order: ``packed_weight(w)`` makes that copy
once per weight (kept while the weight lives and is unchanged -- it doubles the
decode weights' HBM footprint, 5.6 GB for Mamba-2.8B of 288 GB).  Narrow-N calls
split K across workgroups through one fp32 partials workspace per device; calls are
expected on one stream per device.
"""

from __future__ import annotations

import ctypes
import weakref

import torch

from mamba_metal_amd import _lib

LIN_STORE, LIN_RESID, LIN_CONV, LIN_RESID_NORM = 0, 1, 2, 3
MAX_M = 64
K_MULTIPLE = 64
NORM_IN_MAX_M = 8
NORM_IN_MAX_K = 4096
NORM_IN_MAX_N = 512 * 32
_WS_MIN = 8 << 20

_PACKED: dict = {}    # id(w) -> (weakref to w, w._version, w.data_ptr(), packed copy)
_WORKSPACES: dict = {}
_RETIRED: list = []   # outgrown workspaces stay alive: captured graphs may hold them


def _make_packed(w: torch.Tensor) -> torch.Tensor:
    lib = _lib.load()
    dev = _lib.require_cuda(w)
    N, K = w.shape
    code = _lib.dtype_code(w.dtype)
    nbytes = lib.mm_packed_linear_weight_bytes(N, K, code)
    packed = torch.empty(nbytes // w.element_size(), dtype=w.dtype, device=dev)
    with _lib.on_device(dev):
        st = lib.mm_pack_linear_weight(w.data_ptr(), packed.data_ptr(), N, K, w.stride(0), code,
                                       _lib.stream_of(dev))
    _lib.check(st, "mm_pack_linear_weight")
    return packed


def packed_weight(w: torch.Tensor) -> torch.Tensor:
    """The packed copy of an (N, K) f16/bf16 weight, made on first use and remade
    when the weight changes in place; dropped when the weight is freed."""
    key = id(w)
    ent = _PACKED.get(key)
    if ent is not None and ent[0]() is w and ent[1] == w._version and ent[2] == w.data_ptr():
        return ent[3]
    packed = _make_packed(w)
    ref = weakref.ref(w, lambda _r, k=key: _PACKED.pop(k, None))
    _PACKED[key] = (ref, w._version, w.data_ptr(), packed)
    return packed


def _workspace(dev, nbytes: int):
    if nbytes == 0:
        return None
    ws = _WORKSPACES.get(dev)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _RETIRED.append(ws)
        ws = torch.empty(max(nbytes, _WS_MIN), dtype=torch.uint8, device=dev)
        _WORKSPACES[dev] = ws
    return ws


def _rows_ok(t: torch.Tensor) -> bool:
    es = t.element_size()
    return (t.dim() == 2 and t.stride(1) == 1 and t.stride(0) % 8 == 0
            and (t.data_ptr() % 16) == 0 and t.stride(0) >= t.shape[1] and es == 2)


def decode_linear_ok(x: torch.Tensor, w: torch.Tensor) -> bool:
    return (x.is_cuda and x.dtype in (torch.float16, torch.bfloat16) and w.dtype == x.dtype
            and x.dim() == 2 and w.dim() == 2 and 1 <= x.shape[0] <= MAX_M
            and x.shape[1] == w.shape[1] and x.shape[1] % K_MULTIPLE == 0
            and _rows_ok(x) and _rows_ok(w))


def _call(prm: _lib.LinearParams, dev) -> None:
    lib = _lib.load()
    ws = _workspace(dev, lib.mm_decode_linear_workspace_size(prm.M, prm.N, prm.K))
    if ws is not None:
        prm.workspace, prm.workspace_bytes = ws.data_ptr(), ws.numel()
    with _lib.on_device(dev):
        st = lib.mm_decode_linear(ctypes.byref(prm), _lib.stream_of(dev))
    _lib.check(st, "mm_decode_linear")


def split_k(M: int, w: torch.Tensor) -> bool:
    """Whether mm_decode_linear splits K over workgroups for (M, w) -- then a
    RESID_NORM epilogue runs the norm inside its ordered reduce."""
    return _lib.load().mm_decode_linear_workspace_size(M, w.shape[0], w.shape[1]) > 0


def norm_in_ok(x: torch.Tensor, w: torch.Tensor, norm_w: torch.Tensor) -> bool:
    """Whether the input RMSNorm can be folded into this call's operand load."""
    return (decode_linear_ok(x, w) and x.shape[0] <= NORM_IN_MAX_M and w.shape[0] <= NORM_IN_MAX_N
            and x.shape[1] <= NORM_IN_MAX_K
            and norm_w.dtype == x.dtype and norm_w.is_contiguous() and norm_w.dim() == 1
            and norm_w.shape[0] == x.shape[1] and norm_w.data_ptr() % 16 == 0)


def _base(x, w, epi, x_norm=None) -> _lib.LinearParams:
    if not decode_linear_ok(x, w):
        raise ValueError("decode_linear: x (M<=64, K) and w (N, K) must be f16/bf16 of one "
                         "dtype with unit inner stride, 16-byte aligned rows and K % 64 == 0")
    prm = _lib.LinearParams()
    prm.x, prm.w_packed = x.data_ptr(), packed_weight(w).data_ptr()
    prm.M, prm.N, prm.K = x.shape[0], w.shape[0], x.shape[1]
    prm.ldx = x.stride(0)
    prm.dtype = _lib.dtype_code(x.dtype)
    prm.epilogue = epi
    if x_norm is not None:
        norm_w, eps = x_norm
        _lib.require_cuda(x, norm_w)
        if not norm_in_ok(x, w, norm_w):
            raise ValueError("x_norm: needs M <= 8, K <= 4096, N <= 16384 and a contiguous, 16-byte "
                             "aligned (K,) weight in x's dtype")
        prm.x_norm_w, prm.x_eps = norm_w.data_ptr(), float(eps)
    return prm


def decode_linear(x: torch.Tensor, w: torch.Tensor, out: torch.Tensor | None = None,
                  x_norm=None):
    """y (M, N) = x (M, K) @ w (N, K).T  (x replaced by RMSNorm(x) * norm_w when
    x_norm = (norm_w, eps) is given)."""
    dev = _lib.require_cuda(x, w, out)
    prm = _base(x, w, LIN_STORE, x_norm)
    if out is None:
        out = torch.empty((x.shape[0], w.shape[0]), dtype=x.dtype, device=dev)
    if out.shape != (x.shape[0], w.shape[0]) or out.stride(1) != 1 or out.dtype != x.dtype:
        raise ValueError("out must be (M, N) with x's dtype and unit inner stride")
    prm.y, prm.ldy = out.data_ptr(), out.stride(0)
    _call(prm, dev)
    return out


def decode_head_argmax(x: torch.Tensor, w: torch.Tensor, ids: torch.Tensor,
                       out: torch.Tensor | None = None, embed_out: torch.Tensor | None = None):
    """logits (M, N) = x @ w.T as ``decode_linear``, and ids[m] = argmax(logits[m]) (int64,
    torch.argmax's tie and NaN conventions) -- the head and the greedy choice of a decode
    step (mm_decode_head_argmax).  With ``embed_out`` (M, K) the tied embedding rows of
    the chosen ids are written there too, embed_out[m] = w[ids[m]] -- the next step's
    input (mm_decode_head_argmax_embed).  Returns the logits."""
    dev = _lib.require_cuda(x, w, out, ids, embed_out)
    prm = _base(x, w, LIN_STORE)
    if out is None:
        out = torch.empty((x.shape[0], w.shape[0]), dtype=x.dtype, device=dev)
    if out.shape != (x.shape[0], w.shape[0]) or out.stride(1) != 1 or out.dtype != x.dtype:
        raise ValueError("out must be (M, N) with x's dtype and unit inner stride")
    if ids.shape != (x.shape[0],) or ids.dtype != torch.int64 or not ids.is_contiguous():
        raise ValueError("ids must be a contiguous int64 (M,) tensor")
    prm.y, prm.ldy = out.data_ptr(), out.stride(0)
    lib = _lib.load()
    ws = _workspace(dev, lib.mm_decode_head_argmax_workspace_size(prm.M, prm.N, prm.K))
    if ws is not None:
        prm.workspace, prm.workspace_bytes = ws.data_ptr(), ws.numel()
    if embed_out is not None:
        if embed_out.shape != x.shape or embed_out.dtype != w.dtype or not _rows_ok(embed_out):
            raise ValueError("embed_out must be (M, K) in w's dtype with 16-byte aligned rows")
        with _lib.on_device(dev):
            st = lib.mm_decode_head_argmax_embed(ctypes.byref(prm), ids.data_ptr(), w.data_ptr(),
                                                 w.stride(0), embed_out.data_ptr(),
                                                 embed_out.stride(0), _lib.stream_of(dev))
        _lib.check(st, "mm_decode_head_argmax_embed")
        return out
    with _lib.on_device(dev):
        st = lib.mm_decode_head_argmax(ctypes.byref(prm), ids.data_ptr(), _lib.stream_of(dev))
    _lib.check(st, "mm_decode_head_argmax")
    return out


def decode_linear_resid_(resid: torch.Tensor, x: torch.Tensor, w: torch.Tensor):
    """resid (M, N) += round(x @ w.T), in place in resid's (= x's) dtype."""
    dev = _lib.require_cuda(resid, x, w)
    prm = _base(x, w, LIN_RESID)
    if resid.shape != (x.shape[0], w.shape[0]) or resid.stride(1) != 1 or resid.dtype != x.dtype:
        raise ValueError("resid must be (M, N) with x's dtype and unit inner stride")
    prm.resid, prm.ldr = resid.data_ptr(), resid.stride(0)
    _call(prm, dev)
    return resid


def decode_linear_resid_norm_(resid: torch.Tensor, x: torch.Tensor, w: torch.Tensor,
                              norm_w: torch.Tensor, eps: float, out: torch.Tensor | None = None):
    """resid += round(x @ w.T) in place; returns RMSNorm(resid) * norm_w (M, N)."""
    dev = _lib.require_cuda(resid, x, w, norm_w, out)
    prm = _base(x, w, LIN_RESID_NORM)
    if resid.shape != (x.shape[0], w.shape[0]) or resid.stride(1) != 1 or resid.dtype != x.dtype:
        raise ValueError("resid must be (M, N) with x's dtype and unit inner stride")
    if norm_w.shape != (w.shape[0],) or norm_w.dtype != x.dtype or not norm_w.is_contiguous():
        raise ValueError("norm_w must be a contiguous (N,) vector in x's dtype")
    if out is None:
        out = torch.empty_like(resid)
    prm.resid, prm.ldr = resid.data_ptr(), resid.stride(0)
    prm.norm_w, prm.norm_out, prm.ldn, prm.eps = norm_w.data_ptr(), out.data_ptr(), out.stride(0), eps
    _call(prm, dev)
    return out


def xproj_weight_ok(x: torch.Tensor, w_x: torch.Tensor, n_conv: int) -> bool:
    """Whether w_x can be decode_in_proj_conv_xproj's x_proj weight for conv width n_conv."""
    return (w_x.dim() == 2 and w_x.shape[1] == n_conv and w_x.dtype == x.dtype and w_x.is_cuda
            and _rows_ok(w_x) and n_conv % K_MULTIPLE == 0)


def decode_in_proj_conv_xproj(x, w, conv_state, conv_w, conv_b, w_x, x_norm=None):
    """decode_in_proj_conv followed by x_proj: returns (x_conv (M, n_conv), z (M, n_z),
    x_dbl (M, N_x) = x_conv @ w_x.T) through mm_decode_in_proj_xproj, which takes the
    x_proj products inside in_proj's conv epilogue where the shape allows."""
    dev = _lib.require_cuda(x, w, conv_state, conv_w, conv_b, w_x)
    if not in_proj_conv_ok(x, w, conv_state, conv_w, conv_b):
        raise ValueError("decode_in_proj_conv_xproj: unsupported layout (see in_proj_conv_ok)")
    M, N = x.shape[0], w.shape[0]
    n_conv = conv_state.shape[1]
    if not xproj_weight_ok(x, w_x, n_conv):
        raise ValueError("w_x must be (N_x, n_conv) in x's dtype with 16-byte aligned rows and "
                         f"n_conv % {K_MULTIPLE} == 0")
    prm = _base(x, w, LIN_CONV, x_norm)
    x_conv = torch.empty((M, n_conv), dtype=x.dtype, device=dev)
    z = torch.empty((M, N - n_conv), dtype=x.dtype, device=dev)
    x_dbl = torch.empty((M, w_x.shape[0]), dtype=x.dtype, device=dev)
    prm.y, prm.ldy = z.data_ptr(), z.stride(0)
    prm.conv_state, prm.conv_w = conv_state.data_ptr(), conv_w.data_ptr()
    prm.conv_b = _lib.ptr(conv_b)
    prm.conv_out, prm.ldc = x_conv.data_ptr(), x_conv.stride(0)
    prm.n_conv = n_conv
    lib = _lib.load()
    ws = _workspace(dev, lib.mm_decode_in_proj_xproj_workspace_size(M, N, prm.K, n_conv,
                                                                     w_x.shape[0]))
    if ws is not None:
        prm.workspace, prm.workspace_bytes = ws.data_ptr(), ws.numel()
    with _lib.on_device(dev):
        st = lib.mm_decode_in_proj_xproj(ctypes.byref(prm), packed_weight(w_x).data_ptr(),
                                         w_x.shape[0], x_dbl.data_ptr(), x_dbl.stride(0),
                                         _lib.stream_of(dev))
    _lib.check(st, "mm_decode_in_proj_xproj")
    return x_conv, z, x_dbl


def in_proj_conv_ok(x, w, conv_state, conv_w, conv_b) -> bool:
    n_conv = conv_state.shape[1] if conv_state.dim() == 3 else -1
    return (decode_linear_ok(x, w) and conv_state.dim() == 3 and conv_state.shape[2] == 4
            and conv_state.dtype == x.dtype and conv_state.is_contiguous()
            and conv_state.shape[0] == x.shape[0] and 0 < n_conv <= w.shape[0]
            and conv_w.dtype == x.dtype and conv_w.is_contiguous() and conv_w.numel() == n_conv * 4
            and (conv_b is None or (conv_b.dtype == x.dtype and conv_b.is_contiguous()))
            and conv_state.data_ptr() % 8 == 0 and conv_w.data_ptr() % 8 == 0)


def decode_in_proj_conv(x, w, conv_state, conv_w, conv_b=None, x_norm=None):
    """in_proj + decode conv-window step.  x (M, K); w (N, K) with N = n_conv + n_z;
    conv_state (M, n_conv, 4) updated in place; conv_w (n_conv, 1, 4) or (n_conv, 4).
    With x_norm = (norm_w, eps), x is replaced by RMSNorm(x) * norm_w.
    Returns (x_conv (M, n_conv) = silu(conv), z (M, n_z))."""
    dev = _lib.require_cuda(x, w, conv_state, conv_w, conv_b)
    if not in_proj_conv_ok(x, w, conv_state, conv_w, conv_b):
        raise ValueError("decode_in_proj_conv: unsupported layout (see in_proj_conv_ok)")
    prm = _base(x, w, LIN_CONV, x_norm)
    M, N = x.shape[0], w.shape[0]
    n_conv = conv_state.shape[1]
    x_conv = torch.empty((M, n_conv), dtype=x.dtype, device=dev)
    z = torch.empty((M, N - n_conv), dtype=x.dtype, device=dev)
    prm.y, prm.ldy = z.data_ptr(), z.stride(0)
    prm.conv_state, prm.conv_w = conv_state.data_ptr(), conv_w.data_ptr()
    prm.conv_b = _lib.ptr(conv_b)
    prm.conv_out, prm.ldc = x_conv.data_ptr(), x_conv.stride(0)
    prm.n_conv = n_conv
    _call(prm, dev)
    return x_conv, z


# ---------------------------------------------------------------- prefill projections
# mm_prefill_linear, the matrix-core GEMM for short K (the dt projection, K = dt_rank),
# takes prefill calls up to these sizes; deeper or larger products stay on torch's GEMM.
PREFILL_MAX_K = 256
PREFILL_MAX_M = 4096


def _prefill_operands_ok(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None) -> bool:
    return (x.is_cuda and x.dim() == 2 and w.dim() == 2 and x.dtype in (torch.float16, torch.bfloat16)
            and w.dtype == x.dtype and w.device == x.device and x.shape[1] == w.shape[1]
            and x.shape[1] % 16 == 0 and x.stride(1) == 1 and w.stride(1) == 1
            and x.stride(0) % 8 == 0 and w.stride(0) % 8 == 0
            and x.data_ptr() % 16 == 0 and w.data_ptr() % 16 == 0
            and (bias is None or (bias.dtype == x.dtype and bias.device == x.device
                                  and tuple(bias.shape) == (w.shape[0],) and bias.stride(0) == 1)))


def prefill_linear_ok(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None) -> bool:
    """Whether a prefill projection should run on ``prefill_linear``: operands it takes
    (2-D x with unit column stride, f16/bf16, K a multiple of 16, 16-byte aligned rows)
    and short K (<= PREFILL_MAX_K, M <= PREFILL_MAX_M), where it beats torch's GEMM."""
    return (x.dim() == 2 and x.shape[0] <= PREFILL_MAX_M and x.shape[1] <= PREFILL_MAX_K
            and _prefill_operands_ok(x, w, bias))


def prefill_linear(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """y = x @ w.T (+ bias) for x (M, K) and nn.Linear's (N, K) weight with short K, on
    the library's matrix-core kernel (mm_prefill_linear); returns (M, N) in x's dtype."""
    lib = _lib.load()
    dev = _lib.require_cuda(x, w, bias, out)
    if not _prefill_operands_ok(x, w, bias):
        raise ValueError("prefill_linear: x (M, K) and w (N, K) must be f16/bf16 on one GPU with unit "
                         "column stride, K a multiple of 16, 16-byte aligned rows; bias (N,)")
    M, K = x.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=x.dtype, device=dev)
    if out.shape != (M, N) or out.dtype != x.dtype or out.stride(1) != 1:
        raise ValueError("out must be an (M, N) tensor of x's dtype with unit column stride")
    if M == 0 or N == 0:
        return out
    with _lib.on_device(dev):
        st = lib.mm_prefill_linear(x.data_ptr(), w.data_ptr(),
                                   bias.data_ptr() if bias is not None else None, out.data_ptr(),
                                   M, N, K, x.stride(0), w.stride(0), out.stride(0),
                                   _lib.dtype_code(x.dtype), _lib.stream_of(dev))
    _lib.check(st, "mm_prefill_linear")
    return out
