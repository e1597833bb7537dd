"""ctypes binding of libmamba_mi355x.so (the C ABI declared in include/mamba_mi355x.h).

The library is the only compute path of this package: if it is missing, every op
raises (there is no CPU or PyTorch fallback).  torch is imported before the
library is opened so that its DT_NEEDED ``libamdhip64.so.7`` resolves to the HIP
runtime torch already loaded -- streams and device pointers from torch are then
valid inside the library.  ``load()`` verifies that exactly one HIP runtime is
mapped.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (must be loaded before the HIP library; see module docstring)

LIB_NAME = "libmamba_mi355x.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME
ABI_VERSION = 6
MAX_DSTATE = 64

# mm_dtype
F32, F16, BF16 = 0, 1, 2
_DTYPES = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

# mm_status
OK = 0
ERR_NULL_POINTER = -1
ERR_SHAPE = -2
ERR_DSTATE = -3
ERR_DTYPE = -4
ERR_LAYOUT = -5
ERR_WORKSPACE = -6
ERR_HIP = -7

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_sz = ctypes.c_size_t
_i64a2 = ctypes.c_int64 * 2
_i64a3 = ctypes.c_int64 * 3


class ScanParams(ctypes.Structure):
    """Mirror of ``mm_scan_params`` (include/mamba_mi355x.h)."""

    _fields_ = [
        ("u", _vp), ("delta", _vp), ("A", _vp), ("B", _vp), ("C", _vp), ("D", _vp),
        ("z", _vp), ("y", _vp), ("state_out", _vp), ("workspace", _vp),
        ("workspace_bytes", _sz),
        ("batch", _i64), ("dim", _i64), ("dstate", _i64), ("seqlen", _i64),
        ("u_stride", _i64a3), ("delta_stride", _i64a3), ("z_stride", _i64a3),
        ("y_stride", _i64a3), ("B_stride", _i64a3), ("C_stride", _i64a3),
        ("A_stride", _i64a2), ("D_stride", _i64),
        ("x_dtype", _i32), ("bc_dtype", _i32), ("delta_softplus", _i32),
        ("handoff_timeout_us", _i32), ("status", _vp),
    ]


SCAN_STATUS_HANDOFF_TIMEOUT = 1
SCAN_SCRATCH_BYTES = 32 << 20   # MM_SCAN_SCRATCH_BYTES


class LinearParams(ctypes.Structure):
    """Mirror of ``mm_linear_params`` (include/mamba_mi355x.h)."""

    _fields_ = [
        ("x", _vp), ("w_packed", _vp), ("y", _vp), ("resid", _vp), ("conv_state", _vp),
        ("conv_w", _vp), ("conv_b", _vp), ("conv_out", _vp), ("norm_w", _vp), ("norm_out", _vp),
        ("workspace", _vp), ("workspace_bytes", _sz),
        ("M", _i64), ("N", _i64), ("K", _i64),
        ("ldx", _i64), ("ldy", _i64), ("ldr", _i64), ("ldc", _i64), ("ldn", _i64),
        ("n_conv", _i64), ("eps", ctypes.c_float), ("dtype", _i32), ("epilogue", _i32),
        ("x_norm_w", _vp), ("x_eps", ctypes.c_float), ("reserved", _i32),
    ]


_SIGNATURES = {
    "mm_abi_version": ([], ctypes.c_int),
    "mm_last_error": ([], ctypes.c_char_p),
    "mm_status_name": ([ctypes.c_int], ctypes.c_char_p),
    "mm_selective_scan_workspace_size": ([_i64, _i64, _i64, _i64], _sz),
    "mm_selective_scan_fwd": (
        [_vp] * 9 + [_i64] * 4 + [_i32, _i32, _i32, _vp, _sz, _vp], ctypes.c_int),
    "mm_selective_scan_fwd_strided": ([ctypes.POINTER(ScanParams), _vp], ctypes.c_int),
    "mm_selective_scan_fwd_noalloc": ([_vp] * 9 + [_i64] * 4 + [_i32, _i32, _i32, _vp, _vp],
                                      ctypes.c_int),
    "mm_causal_conv1d_fwd": (
        [_vp] * 5 + [_i64] * 4 + [_i64a3, _i64a3, _i64a2, _i32, _i32, _i32, _vp], ctypes.c_int),
    "mm_decode_conv_step": (
        [_vp] * 5 + [_i64] * 5 + [_i64a2, _i32, _i32, _i32, _i32, _vp], ctypes.c_int),
    "mm_decode_ssm_step": (
        [_vp] * 10 + [_i64] * 9 + [_i32, _i32, _vp], ctypes.c_int),
    "mm_decode_ssm_step_dtproj": (
        [_vp] * 11 + [_i64] * 11 + [_i32, _i32, _vp], ctypes.c_int),
    "mm_add_rmsnorm": ([_vp] * 4 + [_i64] * 5 + [ctypes.c_float, _i32, _i32, _vp], ctypes.c_int),
    "mm_packed_linear_weight_bytes": ([_i64, _i64, _i32], _sz),
    "mm_pack_linear_weight": ([_vp, _vp, _i64, _i64, _i64, _i32, _vp], ctypes.c_int),
    "mm_decode_linear_workspace_size": ([_i64, _i64, _i64], _sz),
    "mm_decode_linear": ([ctypes.POINTER(LinearParams), _vp], ctypes.c_int),
    "mm_decode_head_argmax_workspace_size": ([_i64, _i64, _i64], _sz),
    "mm_decode_head_argmax": ([ctypes.POINTER(LinearParams), _vp, _vp], ctypes.c_int),
    "mm_decode_head_argmax_embed": ([ctypes.POINTER(LinearParams), _vp, _vp, _i64, _vp, _i64, _vp],
                                    ctypes.c_int),
    "mm_decode_in_proj_xproj_workspace_size": ([_i64] * 5, _sz),
    "mm_decode_in_proj_xproj": ([ctypes.POINTER(LinearParams), _vp, _i64, _vp, _i64, _vp],
                                ctypes.c_int),
    "mm_prefill_linear": ([_vp] * 4 + [_i64] * 6 + [_i32, _vp], ctypes.c_int),
    "mm_argmax_rows": ([_vp, _i64, _i64, _i64, _i32, _vp, _vp], ctypes.c_int),
    "mm_pair_scan": ([_vp] * 4 + [_i64, _vp], ctypes.c_int),
}

# Every symbol include/mamba_mi355x.h declares (checked by the CPU ABI tests).
EXPORTED = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib = None


class KernelError(RuntimeError):
    """A C-ABI call returned a non-zero mm_status."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def _hip_runtimes_mapped() -> set[str]:
    try:
        with open("/proc/self/maps") as f:
            return {l.split()[-1] for l in f if "libamdhip64" in l}
    except OSError:
        return set()


def load():
    """Open libmamba_mi355x.so (once) and bind its C ABI.  Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_NAME} is not built at {LIB_PATH}; build it with "
                "`python -m mamba_metal_amd._build` (or __graft_entry__.build()). "
                "mamba_metal_amd has no CPU fallback.")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (argtypes, restype) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
        if lib.mm_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_NAME} ABI {lib.mm_abi_version()} != expected {ABI_VERSION}")
        runtimes = _hip_runtimes_mapped()
        if len(runtimes) > 1 and not os.environ.get("MM_ALLOW_MULTIPLE_HIP_RUNTIMES"):
            raise RuntimeError(f"more than one HIP runtime mapped: {sorted(runtimes)}")
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != OK:
        lib = load()
        msg = lib.mm_last_error().decode(errors="replace")
        raise KernelError(status, f"{what} failed: {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """The raw HIP stream handle of ``device``'s current stream."""
    if _raw_stream is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def on_device(device: torch.device):
    """Context for a library call on ``device``: switches the current device only when it
    differs (entering ``torch.cuda.device`` costs microseconds per call, which adds up over
    the dozens of calls of a model prefill)."""
    if device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


_DEVICES: dict = {}  # device index -> torch.device (one object per index)


def require_cuda(*tensors) -> torch.device:
    """The one GPU all given tensors (None entries skipped) live on; raises otherwise.
    Device indices are compared as ints: called a few times per layer of a model prefill,
    where building a torch.device per tensor showed up in the host time."""
    idx = None
    for t in tensors:
        if t is None:
            continue
        i = t.get_device()
        if i < 0 or not t.is_cuda:
            raise ValueError("mamba_metal_amd ops need GPU (HIP) tensors; got a tensor on "
                             f"{t.device} (there is no CPU fallback)")
        if idx is None:
            idx = i
        elif i != idx:
            raise ValueError(f"tensors on different devices: cuda:{idx} and cuda:{i}")
    if idx is None:
        return None
    dev = _DEVICES.get(idx)
    if dev is None:
        dev = _DEVICES.setdefault(idx, torch.device("cuda", idx))
    return dev
