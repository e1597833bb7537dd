"""CPU tests of the C ABI boundary (no GPU needed).

  - libmamba_mi355x.so loads next to torch's HIP runtime and exports every
    function include/mamba_mi355x.h declares;
  - the ctypes mirror of mm_scan_params matches the C layout (offsets compiled
    from the header with gcc);
  - host-only validation rejects invalid arguments with the documented status
    BEFORE any HIP call (these calls never reach the device).
"""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from mamba_metal_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mamba_mi355x.h"
FAKE = 0x1000  # never dereferenced: every call below fails validation first


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mm_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 10, names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in {HEADER.name} but not exported"
    assert set(names) == set(_lib.EXPORTED), "python binding and header disagree"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (mm_[a-z0-9_]+)$", out, flags=re.M))
    assert set(names) <= exported


def test_version_and_status_names(lib):
    assert lib.mm_abi_version() == _lib.ABI_VERSION == 6
    assert lib.mm_status_name(0) == b"MM_OK"
    assert lib.mm_status_name(-3) == b"MM_ERR_DSTATE"
    assert lib.mm_status_name(-99) == b"MM_ERR_UNKNOWN"


def test_single_hip_runtime_mapped(lib):
    assert len(_lib._hip_runtimes_mapped()) == 1


@pytest.mark.parametrize("cname,cls", [("mm_scan_params", _lib.ScanParams),
                                        ("mm_linear_params", _lib.LinearParams)])
def test_params_layout_matches_header(tmp_path, cname, cls):
    fields = [f for f, _ in cls._fields_]
    src = tmp_path / "off.c"
    body = "\n".join(f'printf("{f} %zu\\n", offsetof({cname}, {f}));' for f in fields)
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "mamba_mi355x.h"\n'
                   'int main(void){\n' + body + f'\nprintf("sizeof %zu\\n", sizeof({cname}));'
                   "return 0;}\n")
    exe = tmp_path / "off"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = dict(l.split() for l in subprocess.run([str(exe)], capture_output=True, text=True,
                                                 check=True).stdout.splitlines())
    for f in fields:
        assert int(got[f]) == getattr(cls, f).offset, f
    assert int(got["sizeof"]) == ctypes.sizeof(cls)


def _scan(lib, **over):
    args = dict(u=FAKE, delta=FAKE, A=FAKE, B=FAKE, C=FAKE, D=None, z=None, y=FAKE, state=None,
                batch=1, dim=16, dstate=16, seqlen=64, x_dtype=0, bc_dtype=0, softplus=0,
                ws=FAKE, ws_bytes=1 << 30)
    args.update(over)
    return lib.mm_selective_scan_fwd(
        args["u"], args["delta"], args["A"], args["B"], args["C"], args["D"], args["z"],
        args["y"], args["state"], args["batch"], args["dim"], args["dstate"], args["seqlen"],
        args["x_dtype"], args["bc_dtype"], args["softplus"], args["ws"], args["ws_bytes"], None)


@pytest.mark.parametrize("over,status", [
    (dict(u=None), _lib.ERR_NULL_POINTER),
    (dict(B=None), _lib.ERR_NULL_POINTER),
    (dict(y=None), _lib.ERR_NULL_POINTER),
    (dict(dstate=65), _lib.ERR_DSTATE),
    (dict(dstate=0), _lib.ERR_DSTATE),
    (dict(batch=-1), _lib.ERR_SHAPE),
    (dict(seqlen=-5), _lib.ERR_SHAPE),
    (dict(x_dtype=7), _lib.ERR_DTYPE),
    (dict(bc_dtype=-1), _lib.ERR_DTYPE),
    (dict(ws=None), _lib.ERR_WORKSPACE),
    (dict(ws_bytes=16), _lib.ERR_WORKSPACE),
    (dict(ws=FAKE + 16), _lib.ERR_WORKSPACE),
])
def test_scan_validation_errors(lib, over, status):
    st = _scan(lib, **over)
    assert st == status
    msg = lib.mm_last_error().decode()
    assert msg.startswith(lib.mm_status_name(status).decode())


def test_workspace_size(lib):
    # control block (256 B) + one flag per 16-channel block (the smallest channel block)
    # + carried state (per 64-channel block) + packed fp32 B/C (16 states -> 8 groups x 2
    # per lane, padded to 32-step tiles)
    ncb = 4 * 5120 // 64
    flags_end = 256 + 4 * (4 * 5120 // 16)
    carry = -(-flags_end // 256) * 256
    bc = -(-(carry + 4 * ncb * 16 * 64) // 256) * 256
    assert lib.mm_selective_scan_workspace_size(4, 5120, 16, 32768) == bc + 4 * 4 * 16 * 32768 * 2
    assert lib.mm_selective_scan_workspace_size(1, 64, 65, 100) == 0
    assert lib.mm_selective_scan_workspace_size(0, 64, 16, 100) == 0
    # more than 128 channel blocks: no summary region; 64 states pack more B/C per step
    assert lib.mm_selective_scan_workspace_size(3, 5120, 64, 100) > \
        lib.mm_selective_scan_workspace_size(3, 5120, 16, 100)
    # <= 128 64-channel blocks and dstate <= 16: + segment summaries for the split scan,
    # min(256, 4096 / blocks) segments x (8 groups x 2 states x 64 lanes + 64 delta sums)
    # fp32 per block
    small = 20992  # ctl/flags 512 + carry 4096 + B/C 16384 (one 128-step padded row)
    assert lib.mm_selective_scan_workspace_size(1, 64, 16, 100) == small + 4 * 256 * (16 * 64 + 64)
    # 128 blocks: 32 segments each (ctl + 512 flags 2304 B, carry 524288, B/C 2097152)
    assert lib.mm_selective_scan_workspace_size(128, 64, 16, 100) == \
        2304 + 524288 + 2097152 + 4 * 128 * 32 * (16 * 64 + 64)
    # 129..256 blocks: summaries only for sequences of >= 512 tiles (16384 steps):
    # 2 x 5120 = 160 blocks, 4096 // 160 = 25 segments each
    def base(batch, dim, L):
        up = lambda v, a: -(-v // a) * a
        carry = up(256 + 4 * batch * (-(-dim // 16)), 256)
        bc = up(carry + 4 * batch * (-(-dim // 64)) * 16 * 64, 256)
        return up(bc + 4 * batch * 8 * up(L, 128) * 4, 256)
    assert lib.mm_selective_scan_workspace_size(2, 5120, 16, 16384) == \
        base(2, 5120, 16384) + 4 * 160 * 25 * (16 * 64 + 64)
    assert lib.mm_selective_scan_workspace_size(2, 5120, 16, 16256) == base(2, 5120, 16256)
    assert lib.mm_selective_scan_workspace_size(3, 5120, 16, 32768) == base(3, 5120, 32768) + \
        4 * 240 * (4096 // 240) * (16 * 64 + 64)
    assert lib.mm_selective_scan_workspace_size(5, 5120, 16, 32768) == base(5, 5120, 32768)


def test_strided_null_params(lib):
    assert lib.mm_selective_scan_fwd_strided(None, None) == _lib.ERR_NULL_POINTER
    p = _lib.ScanParams()
    p.u = p.delta = p.A = p.B = p.C = p.y = FAKE
    p.batch, p.dim, p.dstate, p.seqlen = 1, 4, 4, 8
    p.workspace, p.workspace_bytes = FAKE, 1 << 20
    p.handoff_timeout_us = -1
    assert lib.mm_selective_scan_fwd_strided(ctypes.byref(p), None) == _lib.ERR_SHAPE
    assert b"handoff_timeout_us" in lib.mm_last_error()


def test_conv_and_decode_validation(lib):
    s3 = (_lib._i64a3)(1, 1, 1)
    s2 = (_lib._i64a2)(4, 1)
    assert lib.mm_causal_conv1d_fwd(None, FAKE, None, FAKE, None, 1, 8, 8, 4, s3, s3, s2, 1, 1, 1,
                                    None) == _lib.ERR_NULL_POINTER
    assert lib.mm_causal_conv1d_fwd(FAKE, FAKE, None, FAKE, None, 1, 8, 8, 9, s3, s3, s2, 1, 1, 1,
                                    None) == _lib.ERR_SHAPE
    assert lib.mm_causal_conv1d_fwd(FAKE, FAKE, None, FAKE, None, 1, 8, 8, 4, s3, s3, s2, 5, 1, 1,
                                    None) == _lib.ERR_DTYPE
    assert lib.mm_decode_conv_step(FAKE, FAKE, FAKE, None, FAKE, 1, 8, 0, 8, 8, s2, 1, 1, 1, 1,
                                   None) == _lib.ERR_SHAPE
    assert lib.mm_decode_ssm_step(FAKE, FAKE, FAKE, None, FAKE, FAKE, FAKE, None, None, FAKE,
                                  1, 8, 65, 8, 8, 16, 16, 8, 8, 1, 1, None) == _lib.ERR_DSTATE
    assert lib.mm_decode_ssm_step(FAKE + 4, FAKE, FAKE, None, FAKE, FAKE, FAKE, None, None, FAKE,
                                  1, 8, 16, 8, 8, 16, 16, 8, 8, 1, 1, None) == _lib.ERR_LAYOUT
    assert lib.mm_pair_scan(FAKE, FAKE, None, FAKE, -1, None) == _lib.ERR_SHAPE
    assert lib.mm_pair_scan(None, FAKE, None, FAKE, 4, None) == _lib.ERR_NULL_POINTER


def test_fused_decode_and_norm_validation(lib):
    """The fused decode step takes dstate 16, rank 1..256 and one dtype for x and W;
    add_rmsnorm rejects negative sizes and eps < 0 -- all before any device access."""
    def dtproj(dstate=16, rank=160, x_dtype=1, w_dtype=1, state=FAKE):
        return lib.mm_decode_ssm_step_dtproj(state, FAKE, FAKE, FAKE, None, FAKE, FAKE, FAKE,
                                             None, None, FAKE, 2, 64, dstate, rank, 64, 192, rank,
                                             192, 192, 0, 64, x_dtype, w_dtype, None)
    assert dtproj(dstate=8) == _lib.ERR_DSTATE
    assert b"dstate" in lib.mm_last_error()
    assert dtproj(rank=0) == _lib.ERR_SHAPE
    assert dtproj(rank=257) == _lib.ERR_SHAPE
    assert dtproj(w_dtype=0) == _lib.ERR_DTYPE
    assert dtproj(state=FAKE + 4) == _lib.ERR_LAYOUT
    assert lib.mm_add_rmsnorm(FAKE, None, FAKE, FAKE, -1, 8, 8, 8, 8, 1e-5, 1, 1, None) == _lib.ERR_SHAPE
    assert lib.mm_add_rmsnorm(FAKE, None, FAKE, FAKE, 1, 8, 8, 8, 8, -1.0, 1, 1, None) == _lib.ERR_SHAPE
    assert lib.mm_add_rmsnorm(None, None, FAKE, FAKE, 1, 8, 8, 8, 8, 1e-5, 1, 1, None) == \
        _lib.ERR_NULL_POINTER


def test_decode_linear_validation(lib):
    """mm_decode_linear / mm_pack_linear_weight check shape, dtype, layout and the
    workspace before touching memory."""
    def call(**kw):
        prm = _lib.LinearParams()
        prm.x = prm.w_packed = prm.y = FAKE
        prm.M, prm.N, prm.K = 4, 32, 64
        prm.ldx, prm.ldy = 64, 32
        prm.dtype, prm.epilogue = _lib.F16, 0
        for k, v in kw.items():
            setattr(prm, k, v)
        return lib.mm_decode_linear(ctypes.byref(prm), None)
    assert lib.mm_decode_linear(None, None) == _lib.ERR_NULL_POINTER
    assert call(M=65) == _lib.ERR_SHAPE
    assert call(dtype=_lib.F32) == _lib.ERR_DTYPE
    assert call(K=48, ldx=48) == _lib.ERR_LAYOUT
    assert call(ldx=32) == _lib.ERR_LAYOUT
    assert call(x=FAKE + 8) == _lib.ERR_LAYOUT
    assert call(epilogue=7) == _lib.ERR_SHAPE
    assert call(epilogue=1) == _lib.ERR_NULL_POINTER          # RESID without resid
    assert call(epilogue=2, n_conv=16) == _lib.ERR_NULL_POINTER
    assert call(M=0) == _lib.OK and call(N=0) == _lib.OK
    # input RMSNorm: M <= 8, N <= 16384, aligned weight, eps >= 0; reserved must be 0
    assert call(x_norm_w=FAKE, M=9) == _lib.ERR_SHAPE
    assert call(x_norm_w=FAKE, N=16385) == _lib.ERR_SHAPE
    assert call(x_norm_w=FAKE, K=4160, ldx=4160) == _lib.ERR_SHAPE
    assert call(x_norm_w=FAKE + 8) == _lib.ERR_LAYOUT
    assert call(x_norm_w=FAKE, x_eps=-1.0) == _lib.ERR_SHAPE
    assert call(x_norm_w=FAKE, M=0) == _lib.OK
    assert call(reserved=1) == _lib.ERR_LAYOUT
    # narrow N splits K across workgroups: needs a workspace
    need = lib.mm_decode_linear_workspace_size(64, 192, 5120)
    assert need > 0
    assert call(M=64, N=192, K=5120, ldx=5120) == _lib.ERR_WORKSPACE
    assert call(M=64, N=192, K=5120, ldx=5120, workspace=FAKE, workspace_bytes=need - 1) == \
        _lib.ERR_WORKSPACE
    assert lib.mm_decode_linear_workspace_size(64, 50280, 2560) == 0   # wide N: no split
    assert lib.mm_packed_linear_weight_bytes(50, 64, _lib.F16) == 64 * 64 * 2
    assert lib.mm_pack_linear_weight(FAKE, FAKE, 50, 48, 48, _lib.F16, None) == _lib.ERR_LAYOUT
    assert lib.mm_pack_linear_weight(FAKE, FAKE, 50, 64, 64, _lib.F32, None) == _lib.ERR_DTYPE


def test_decode_in_proj_xproj_validation(lib):
    """mm_decode_in_proj_xproj: the in_proj params as for mm_decode_linear (conv
    epilogue required) plus the x_proj weight / output, all checked before any launch."""
    def call(xp_w=FAKE, xp_n=192, xp_y=FAKE, ld_xp=192, **kw):
        prm = _lib.LinearParams()
        prm.x = prm.w_packed = prm.y = prm.conv_state = prm.conv_w = prm.conv_out = FAKE
        prm.M, prm.N, prm.K = 64, 10240, 2560
        prm.ldx, prm.ldy, prm.ldc = 2560, 5120, 5120
        prm.n_conv = 5120
        prm.dtype, prm.epilogue = _lib.F16, 2   # MM_LIN_CONV
        for k, v in kw.items():
            setattr(prm, k, v)
        return lib.mm_decode_in_proj_xproj(ctypes.byref(prm), xp_w, xp_n, xp_y, ld_xp, None)
    assert lib.mm_decode_in_proj_xproj(None, FAKE, 192, FAKE, 192, None) == _lib.ERR_NULL_POINTER
    assert call(epilogue=0) == _lib.ERR_SHAPE                 # in_proj must carry the conv step
    assert call(xp_w=None) == _lib.ERR_NULL_POINTER
    assert call(xp_y=None) == _lib.ERR_NULL_POINTER
    assert call(xp_n=0) == _lib.ERR_SHAPE
    assert call(ld_xp=100) == _lib.ERR_LAYOUT
    assert call(xp_w=FAKE + 8) == _lib.ERR_LAYOUT
    assert call(n_conv=5100, ldc=5100) == _lib.ERR_LAYOUT    # x_proj's K must be a multiple of 64
    assert call(conv_out=FAKE + 8) == _lib.ERR_LAYOUT
    # the fused path needs its partial planes (one 64 x 192 fp32 plane per 32 conv columns)
    need = lib.mm_decode_in_proj_xproj_workspace_size(64, 10240, 2560, 5120, 192)
    assert need >= 160 * 64 * 192 * 4
    assert call() == _lib.ERR_WORKSPACE
    assert call(workspace=FAKE, workspace_bytes=need - 1) == _lib.ERR_WORKSPACE
    assert call(M=0) == _lib.OK
    # batch <= 4 runs in_proj as a GEMV and x_proj as its own (split-K) GEMM
    assert lib.mm_decode_in_proj_xproj_workspace_size(2, 10240, 2560, 5120, 192) == \
        lib.mm_decode_linear_workspace_size(2, 192, 5120)
    assert lib.mm_decode_in_proj_xproj_workspace_size(0, 10240, 2560, 5120, 192) == 0


def test_decode_head_argmax_validation(lib):
    """mm_decode_head_argmax: the head params as for mm_decode_linear (plain store) plus the
    int64 ids; the fused path keeps one (value, column) candidate per workgroup and row in
    the workspace.  All checked before any launch."""
    def call(ids=FAKE, **kw):
        prm = _lib.LinearParams()
        prm.x = prm.w_packed = prm.y = FAKE
        prm.M, prm.N, prm.K = 64, 50280, 2560
        prm.ldx, prm.ldy = 2560, 50280
        prm.dtype, prm.epilogue = _lib.F16, 0
        for k, v in kw.items():
            setattr(prm, k, v)
        return lib.mm_decode_head_argmax(ctypes.byref(prm), ids, None)
    assert lib.mm_decode_head_argmax(None, FAKE, None) == _lib.ERR_NULL_POINTER
    assert call(ids=None) == _lib.ERR_NULL_POINTER
    assert call(ids=FAKE + 4) == _lib.ERR_LAYOUT
    assert call(epilogue=1) == _lib.ERR_SHAPE
    assert call(ldy=50000) == _lib.ERR_LAYOUT
    assert call(M=65) == _lib.ERR_SHAPE
    need = lib.mm_decode_head_argmax_workspace_size(64, 50280, 2560)
    assert need == 197 * 64 * 8       # 197 workgroups of 8 x 32 columns
    assert call() == _lib.ERR_WORKSPACE
    assert call(workspace=FAKE, workspace_bytes=need - 1) == _lib.ERR_WORKSPACE
    assert call(M=0) == _lib.OK
    # narrow N (no shared-X head): mm_decode_linear's workspace, then mm_argmax_rows
    assert lib.mm_decode_head_argmax_workspace_size(4, 3072, 768) == \
        lib.mm_decode_linear_workspace_size(4, 3072, 768)


def test_decode_head_argmax_embed_validation(lib):
    """mm_decode_head_argmax_embed: mm_decode_head_argmax's checks plus the tied (N, K)
    table and the (M, K) rows, both with row strides >= K, multiples of 8, 16-byte
    aligned; all checked before any launch."""
    def call(table=FAKE, ld_t=2560, rows=FAKE, ld_r=2560, ids=FAKE, **kw):
        prm = _lib.LinearParams()
        prm.x = prm.w_packed = prm.y = FAKE
        prm.M, prm.N, prm.K = 64, 50280, 2560
        prm.ldx, prm.ldy = 2560, 50280
        prm.dtype, prm.epilogue = _lib.F16, 0
        for k, v in kw.items():
            setattr(prm, k, v)
        return lib.mm_decode_head_argmax_embed(ctypes.byref(prm), ids, table, ld_t, rows, ld_r, None)
    assert lib.mm_decode_head_argmax_embed(None, FAKE, FAKE, 2560, FAKE, 2560, None) == \
        _lib.ERR_NULL_POINTER
    assert call(table=None) == _lib.ERR_NULL_POINTER
    assert call(rows=None) == _lib.ERR_NULL_POINTER
    assert call(ld_t=2552) == _lib.ERR_LAYOUT
    assert call(ld_r=2564) == _lib.ERR_LAYOUT
    assert call(table=FAKE + 8) == _lib.ERR_LAYOUT
    assert call(rows=FAKE + 8) == _lib.ERR_LAYOUT
    assert call(ids=None) == _lib.ERR_NULL_POINTER     # then mm_decode_head_argmax's checks
    assert call(epilogue=1) == _lib.ERR_SHAPE
    assert call() == _lib.ERR_WORKSPACE
    assert call(M=0, workspace=FAKE, workspace_bytes=1 << 30) == _lib.OK


def test_argmax_validation(lib):
    out = FAKE
    assert lib.mm_argmax_rows(None, 2, 8, 8, _lib.F16, out, None) == _lib.ERR_NULL_POINTER
    assert lib.mm_argmax_rows(FAKE, 2, 0, 8, _lib.F16, out, None) == _lib.ERR_SHAPE
    assert lib.mm_argmax_rows(FAKE, 2, 16, 8, _lib.F16, out, None) == _lib.ERR_LAYOUT
    assert lib.mm_argmax_rows(FAKE, 2, 8, 8, 9, out, None) == _lib.ERR_DTYPE
    assert lib.mm_argmax_rows(FAKE, 0, 8, 8, _lib.F16, out, None) == _lib.OK


def test_prefill_linear_validation(lib):
    f = lib.mm_prefill_linear  # x, w, bias, y, M, N, K, ldx, ldw, ldy, dtype, stream
    ok = dict(M=4, N=4, K=16, ldx=16, ldw=16, ldy=4, dt=_lib.F16)

    def call(x=FAKE, w=FAKE, y=FAKE, **kw):
        a = {**ok, **kw}
        return f(x, w, None, y, a["M"], a["N"], a["K"], a["ldx"], a["ldw"], a["ldy"], a["dt"], None)

    assert call(x=None) == _lib.ERR_NULL_POINTER
    assert call(y=None) == _lib.ERR_NULL_POINTER
    assert call(dt=_lib.F32) == _lib.ERR_DTYPE              # f16 / bf16 only
    assert call(M=-1) == _lib.ERR_SHAPE
    assert call(K=24, ldx=24, ldw=24) == _lib.ERR_SHAPE     # K not a multiple of 16
    assert call(ldx=8) == _lib.ERR_LAYOUT                   # row stride below K
    assert call(ldy=2) == _lib.ERR_LAYOUT                   # output row stride below N
    assert call(ldx=20) == _lib.ERR_LAYOUT                  # rows not 16-byte aligned
    assert call(w=FAKE + 2) == _lib.ERR_LAYOUT              # misaligned base
    assert call(M=0) == _lib.OK                             # nothing to do
    assert call(N=0, ldy=0) == _lib.OK


def test_zero_sizes_are_noops(lib):
    # Nothing to do -> MM_OK without touching the (fake) pointers or the device.
    assert _scan(lib, batch=0) == _lib.OK
    assert _scan(lib, dim=0) == _lib.OK
    s3 = (_lib._i64a3)(1, 1, 1)
    s2 = (_lib._i64a2)(4, 1)
    assert lib.mm_causal_conv1d_fwd(FAKE, FAKE, None, FAKE, None, 1, 0, 8, 4, s3, s3, s2, 1, 1, 1,
                                    None) == _lib.OK
    assert lib.mm_pair_scan(FAKE, FAKE, None, FAKE, 0, None) == _lib.OK


def test_noalloc_scan_rejects_oversize_host_side(lib):
    # a shape whose workspace exceeds the static per-device array is refused before any
    # HIP call; invalid arguments are refused as by mm_selective_scan_fwd
    batch, dim, seqlen = 8, 5120, 65536
    assert lib.mm_selective_scan_workspace_size(batch, dim, 16, seqlen) > _lib.SCAN_SCRATCH_BYTES
    st = lib.mm_selective_scan_fwd_noalloc(FAKE, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, None,
                                           batch, dim, 16, seqlen, _lib.F16, _lib.F16, 1, None, None)
    assert st == _lib.ERR_WORKSPACE
    assert b"allocation-free" in lib.mm_last_error()
    assert lib.mm_selective_scan_fwd_noalloc(None, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, None,
                                             1, 64, 16, 64, 1, 1, 1, None, None) == _lib.ERR_NULL_POINTER
    assert lib.mm_selective_scan_fwd_noalloc(FAKE, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, None,
                                             1, 64, 65, 64, 1, 1, 1, None, None) == _lib.ERR_DSTATE
    assert lib.mm_selective_scan_fwd_noalloc(FAKE, FAKE, FAKE, FAKE, FAKE, None, None, FAKE, None,
                                             0, 64, 16, 64, 1, 1, 1, None, None) == _lib.OK
