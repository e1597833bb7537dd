"""mm_selective_scan_fwd_noalloc: the allocation-free scan entry point, through the C ABI.

Its output must equal mm_selective_scan_fwd's (same kernels; the workspace is the
library's static per-device array instead of a caller-allocated buffer), on two calls
in a row -- the second smaller than the first, so the array holds the first call's
contents when the second starts; a shape whose split-scan summaries do not fit the array
runs chained; a shape beyond the array is rejected.  Every call passes a status word,
which must stay zero (no segment gave up waiting for its carried state).  The call is
also recorded into a HIP graph (the first call of this module on the device, so the
array's address lookup happens under capture) and replayed several times with eager work
in between, each replay against the eager result.
"""

from __future__ import annotations

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


def _call(lib, fn, ins, ws=None, status=None, out=None):
    """One scan call through the C ABI; returns (y, state).  ``out``: preallocated (y, h)."""
    from mamba_metal_amd import _lib

    u, d, z, B, C, A, D = ins
    batch, dim, seqlen = u.shape
    if out is None:
        y = torch.full_like(u, float("nan"))
        h = torch.full((batch, dim, 16), float("nan"), device=u.device)
    else:
        y, h = out
    common = [u.data_ptr(), d.data_ptr(), A.data_ptr(), B.data_ptr(), C.data_ptr(), D.data_ptr(),
              z.data_ptr(), y.data_ptr(), h.data_ptr(), batch, dim, 16, seqlen, _lib.F16, _lib.F16, 1]
    stream = torch.cuda.current_stream(u.device).cuda_stream
    if fn == "noalloc":
        st = lib.mm_selective_scan_fwd_noalloc(*common, _lib.ptr(status), stream)
    else:
        st = lib.mm_selective_scan_fwd(*common, ws.data_ptr(), ws.numel(), stream)
    _lib.check(st, fn)
    return y, h


def test_noalloc_graph_capture_replays(dev):
    """The allocation-free call recorded into a HIP graph -- the first noalloc call of this
    module, so its per-device address lookup runs under capture -- then replayed four
    times with eager scans of other inputs through the same static array in between;
    every replay must equal the eager call on the same inputs bit for bit, with a zero
    status word."""
    from mamba_metal_amd import _lib

    lib = _lib.load()
    ins = _inputs(dev, 2, 1536, 4096, 11)
    other = _inputs(dev, 1, 640, 3000, 12)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    y = torch.full_like(ins[0], float("nan"))
    h = torch.full((2, 1536, 16), float("nan"), device=dev)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _call(lib, "noalloc", ins, status=status, out=(y, h))
    need = lib.mm_selective_scan_workspace_size(2, 1536, 16, 4096)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    y_ref, h_ref = _call(lib, "fwd", ins, ws)
    for rep in range(4):
        y.fill_(float("nan"))
        h.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref), f"replay {rep}: y differs from the eager call"
        assert torch.equal(h, h_ref), f"replay {rep}: state differs from the eager call"
        _call(lib, "noalloc", other, status=status)   # eager use of the same array between replays
        torch.cuda.synchronize()
    assert int(status.item()) == 0


def test_noalloc_matches_workspace_entry_point(dev):
    from mamba_metal_amd import _lib

    lib = _lib.load()
    # (4, 5120, 2048): 320 channel chains, chained segment hand-offs through the static
    # array; (3, 1000, 5000): 48 chains, the split mode's segment summaries; then a
    # smaller call on the same array
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    for shape, seed in (((4, 5120, 2048), 1), ((3, 1000, 5000), 2), ((1, 200, 700), 3)):
        ins = _inputs(dev, *shape, seed)
        need = lib.mm_selective_scan_workspace_size(shape[0], shape[1], 16, shape[2])
        assert 0 < need <= _lib.SCAN_SCRATCH_BYTES
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        y0, h0 = _call(lib, "fwd", ins, ws)
        y1, h1 = _call(lib, "noalloc", ins, status=status)
        torch.cuda.synchronize()
        assert int(ws[4:8].view(torch.int32).item()) == 0
        assert int(status.item()) == 0, f"{shape}: hand-off timeout reported"
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
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    y0, h0 = _call(lib, "fwd", ins, ws)
    y1, h1 = _call(lib, "noalloc", ins, status=status)
    torch.cuda.synchronize()
    assert int(ws[4:8].view(torch.int32).item()) == 0
    assert int(status.item()) == 0
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
                                           _lib.F16, _lib.F16, 1, None, None)
    assert st == _lib.ERR_WORKSPACE
    assert b"allocation-free" in lib.mm_last_error()
