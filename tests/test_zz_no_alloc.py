"""mm_selective_scan_fwd_noalloc: the allocation-free scan entry point, through the C ABI.

Its output must equal mm_selective_scan_fwd's (same kernels; the workspace is the
library's static per-device array instead of a caller-allocated buffer), on two calls
in a row -- the second smaller than the first, so the array holds the first call's
contents when the second starts; a shape whose split-scan summaries do not fit the array
runs chained; a shape beyond the array is rejected.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(dev, batch, dim, seqlen, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    f16 = torch.float16
    u = torch.randn((batch, dim, seqlen), generator=g, device=dev).to(f16)
    d = (torch.randn((batch, dim, seqlen), generator=g, device=dev) * 0.5 - 1.0).to(f16)
    z = torch.randn((batch, dim, seqlen), generator=g, device=dev).to(f16)
    B = torch.randn((batch, 16, seqlen), generator=g, device=dev).to(f16)
    C = torch.randn((batch, 16, seqlen), generator=g, device=dev).to(f16)
    A = -torch.rand((dim, 16), generator=g, device=dev) * 2 - 0.01
    D = torch.randn(dim, generator=g, device=dev)
    return u, d, z, B, C, A, D


def _call(lib, fn, ins, ws=None):
    from mamba_metal_amd import _lib

    u, d, z, B, C, A, D = ins
    batch, dim, seqlen = u.shape
    y = torch.full_like(u, float("nan"))
    h = torch.full((batch, dim, 16), float("nan"), device=u.device)
    common = [u.data_ptr(), d.data_ptr(), A.data_ptr(), B.data_ptr(), C.data_ptr(), D.data_ptr(),
              z.data_ptr(), y.data_ptr(), h.data_ptr(), batch, dim, 16, seqlen, _lib.F16, _lib.F16, 1]
    stream = torch.cuda.current_stream(u.device).cuda_stream
    if fn == "noalloc":
        st = lib.mm_selective_scan_fwd_noalloc(*common, stream)
    else:
        st = lib.mm_selective_scan_fwd(*common, ws.data_ptr(), ws.numel(), stream)
    _lib.check(st, fn)
    return y, h


def test_noalloc_matches_workspace_entry_point(dev):
    from mamba_metal_amd import _lib

    lib = _lib.load()
    # (4, 5120, 2048): 320 channel chains, chained segment hand-offs through the static
    # array; (3, 1000, 5000): 48 chains, the split mode's segment summaries; then a
    # smaller call on the same array
    for shape, seed in (((4, 5120, 2048), 1), ((3, 1000, 5000), 2), ((1, 200, 700), 3)):
        ins = _inputs(dev, *shape, seed)
        need = lib.mm_selective_scan_workspace_size(shape[0], shape[1], 16, shape[2])
        assert 0 < need <= _lib.SCAN_SCRATCH_BYTES
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        y0, h0 = _call(lib, "fwd", ins, ws)
        y1, h1 = _call(lib, "noalloc", ins)
        torch.cuda.synchronize()
        assert int(ws[4:8].view(torch.int32).item()) == 0
        assert torch.isfinite(y0).all() and torch.isfinite(h0).all()
        assert torch.equal(y1, y0), f"{shape}: y differs"
        assert torch.equal(h1, h0), f"{shape}: state differs"


def test_noalloc_chained_when_summaries_do_not_fit(dev):
    """B=4, D=4096 (256 64-channel blocks), L=32768: the full workspace (with the split
    scan's segment summaries) exceeds the static array, the chained share fits, so the
    allocation-free call runs the chained scan while the caller-allocated one splits.
    The two paths round differently (a segment's carried decay is a product of exp2s in
    one, exp2 of a sum in the other): equal at the fp16 bar, on every output."""
    from mamba_metal_amd import _lib

    from helpers import assert_close

    lib = _lib.load()
    shape = (4, 4096, 32768)
    need = lib.mm_selective_scan_workspace_size(shape[0], shape[1], 16, shape[2])
    assert need > _lib.SCAN_SCRATCH_BYTES
    ins = _inputs(dev, *shape, 4)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    y0, h0 = _call(lib, "fwd", ins, ws)
    y1, h1 = _call(lib, "noalloc", ins)
    torch.cuda.synchronize()
    assert int(ws[4:8].view(torch.int32).item()) == 0
    assert torch.isfinite(y1).all() and torch.isfinite(h1).all()
    assert_close(y1.float().cpu().numpy(), y0.float().cpu().numpy(), 1e-3, 1e-3, "y")
    assert_close(h1.cpu().numpy(), h0.cpu().numpy(), 1e-3, 1e-3, "state")


def test_noalloc_rejects_oversize(dev):
    from mamba_metal_amd import _lib

    lib = _lib.load()
    F = 0x1000   # never dereferenced: the call fails host-side validation
    batch, dim, seqlen = 8, 5120, 65536
    assert lib.mm_selective_scan_workspace_size(batch, dim, 16, seqlen) > _lib.SCAN_SCRATCH_BYTES
    st = lib.mm_selective_scan_fwd_noalloc(F, F, F, F, F, None, None, F, None, batch, dim, 16, seqlen,
                                           _lib.F16, _lib.F16, 1, None)
    assert st == _lib.ERR_WORKSPACE
    assert b"allocation-free" in lib.mm_last_error()
