"""load_kernel(): the reference's kernel-loading entry point, over prebuilt HIP kernels.

The reference (mamba_metal/_loader.py:29-42) reads an MSL body from
``kernels/<name>.metal`` and wraps it with ``mx.fast.metal_kernel``; callers then
invoke it as ``kernel(inputs=[...], output_shapes=..., output_dtypes=...,
grid=..., threadgroup=...)``.  Here the kernels are compiled ahead of time into
libmamba_mi355x.so, so ``load_kernel`` looks a kernel up by the same name and
returns a callable with the same calling convention: inputs in the reference's
order (arrays, then 0-d / int scalars), outputs returned as a list in the
reference's order.  ``grid``/``threadgroup`` are accepted and ignored -- launch
geometry is chosen by the library for gfx950.

Kernels available (reference name -> reference binding):
  selective_scan_chunked  inputs u, delta, A, B, C, D, z, batch, dim, dstate, seqlen,
                          apply_softplus, use_D, use_z -> [y, ssm_state_out]
                          (mamba_metal/selective_scan.py:12-20,62-77)
  pair_scan               inputs a_in, b_in, n -> [a_out, h_out]
                          (experiments/05-pair-scan/pair_scan.py:16-33)
"""

from __future__ import annotations

import torch

from mamba_metal_amd import _lib

KERNELS = ("selective_scan_chunked", "pair_scan")


def _scalar(x) -> int:
    return int(x.item()) if isinstance(x, torch.Tensor) else int(x)


class _Kernel:
    def __init__(self, name, input_names, output_names):
        self.name = name
        self.input_names = list(input_names) if input_names else None
        self.output_names = list(output_names) if output_names else None

    def __call__(self, inputs, output_shapes=None, output_dtypes=None, grid=None,
                 threadgroup=None, **_):
        if self.name == "selective_scan_chunked":
            return self._scan(inputs)
        return self._pair_scan(inputs)

    def _scan(self, inputs):
        from mamba_metal_amd.selective_scan import selective_scan

        u, delta, A, B, C, D, z = inputs[:7]
        apply_softplus, use_D, use_z = (_scalar(v) for v in inputs[11:14])
        y, state = selective_scan(u, delta, A, B, C, D=D if use_D else None,
                                  z=z if use_z else None, delta_softplus=bool(apply_softplus),
                                  return_state=True)
        return [y, state]

    def _pair_scan(self, inputs):
        a, b = inputs[0], inputs[1]
        n = _scalar(inputs[2]) if len(inputs) > 2 else a.numel()
        return list(pair_scan(a, b, n))


def pair_scan(a, b, n=None):
    """Inclusive (a, b) pair scan; returns (a_out, h_out) (mamba_metal/kernels/pair_scan.metal)."""
    lib = _lib.load()
    dev = _lib.require_cuda(a, b)
    a = a.contiguous().float()
    b = b.contiguous().float()
    n = a.numel() if n is None else int(n)
    a_out = torch.empty_like(a)
    h_out = torch.empty_like(b)
    if n:
        with _lib.on_device(dev):
            st = lib.mm_pair_scan(a.data_ptr(), b.data_ptr(), a_out.data_ptr(), h_out.data_ptr(),
                                  n, _lib.stream_of(dev))
        _lib.check(st, "mm_pair_scan")
    return a_out, h_out


def read_kernel_source(name: str, params: dict | None = None) -> str:
    """The reference returns MSL text (mamba_metal/_loader.py:16-26); here kernels are
    compiled HIP, so this returns the name of the HIP entry point serving ``name``."""
    if name not in KERNELS:
        raise FileNotFoundError(f"no kernel named {name!r}; available: {KERNELS}")
    return {"selective_scan_chunked": "mm_selective_scan_fwd", "pair_scan": "mm_pair_scan"}[name]


def load_kernel(name: str, input_names: list[str] | None = None,
                output_names: list[str] | None = None, params: dict | None = None):
    """Look up a prebuilt HIP kernel by its reference name (see module docstring)."""
    if name not in KERNELS:
        raise FileNotFoundError(f"no kernel named {name!r}; available: {KERNELS}")
    _lib.load()
    return _Kernel(name, input_names, output_names)
