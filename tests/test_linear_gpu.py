"""Decode-step GEMM (mm_decode_linear) against a float32 torch reference.

The reference is x.float() @ w.float().T on the GPU (a plain fp32 GEMM of the same
op); outputs are rounded once to f16/bf16, so the tolerance is the output dtype's
half-ulp plus fp32 accumulation-order noise, relative to the output's scale."""

import numpy as np
import pytest
import torch

from helpers import assert_close
from oracle import numpy_ref

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def _ref(x, w):
    return x.float() @ w.float().T


def _check(got, ref, dtype, what):
    scale = float(ref.abs().max()) + 1e-6
    tol = TOL[dtype]
    assert_close(got.float().cpu().numpy(), ref.cpu().numpy(), tol, tol * scale * 0.05, what)


# decode shapes of Mamba-2.8B (in/out/x projections, head) and 130M, ragged M/N,
# split-K (narrow N) and single-chunk K
# (37, 4096, 100) and (64, 5120, 192) split K over the grid with ragged / narrow N; the
# 130M batch-1 shapes and the small ones keep K in the workgroup; (64, 2560, 10240) and
# (20, 128, 8200) give each wave two column tiles.  > 512 column tiles run the shared-X
# kernel: (37, 256, 20000) with 4 waves and a ragged last tile, (64, 2560, 50280) and
# (1, 768, 50280) (130M head at batch 1: one 32-row MFMA tile, X staged by half the
# waves) with 8.  M <= 4 runs the GEMV, whose workgroup size and load group follow K:
# (1, 768, 3072) 256 threads, groups of 3; (1, 1536, 80) 512, 3; (1, 1024, 136) 256, 4;
# (2, 2560, 200) 1024, 3; (3, 5120, 72) 1024 threads, two rounds of 3 with one clamped
# step; (4, 320, 40) 256 threads, one group of 3 with one clamped step; (1, 4096, 64) 1024, 4.
@pytest.mark.parametrize("M,K,N", [(64, 2560, 10240), (64, 5120, 2560), (64, 5120, 192),
                                   (1, 768, 3072), (1, 1536, 80), (37, 1536, 100), (33, 256, 50),
                                   (37, 4096, 100), (32, 64, 33), (64, 2560, 50280), (5, 64, 7),
                                   (64, 64, 4096), (1, 768, 50280), (37, 256, 20000),
                                   (20, 128, 8200), (1, 1024, 136), (2, 2560, 200), (3, 5120, 72),
                                   (4, 320, 40), (1, 4096, 64)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_linear(dev, M, K, N, dtype):
    from mamba_metal_amd.linear import decode_linear

    g = torch.Generator(device=dev).manual_seed(M * 7 + K * 3 + N)
    x = torch.randn((M, K), generator=g, device=dev).to(dtype)
    w = (torch.randn((N, K), generator=g, device=dev) * 0.05).to(dtype)
    y = decode_linear(x, w)
    torch.cuda.synchronize()
    _check(y, _ref(x, w), dtype, f"linear M={M} K={K} N={N}")
    # deterministic: fixed-order split-K reduction
    y2 = decode_linear(x, w)
    assert torch.equal(y, y2)
    # the split-K workspace is left zeroed: a third call on other data is right too
    x3 = torch.randn((M, K), generator=g, device=dev).to(dtype)
    _check(decode_linear(x3, w), _ref(x3, w), dtype, f"linear again M={M} K={K} N={N}")


def test_decode_linear_split_sequence(dev):
    """Split-K calls of different shapes in a row share one partials workspace; each
    must be right whatever the previous call left there (narrow and wide calls mixed)."""
    from mamba_metal_amd.linear import decode_linear

    g = torch.Generator(device=dev).manual_seed(11)
    for (M, K, N) in [(64, 5120, 192), (37, 4096, 100), (64, 5120, 192), (64, 5120, 2560),
                      (33, 5120, 2000), (64, 5120, 2560)]:
        x = torch.randn((M, K), generator=g, device=dev).half()
        w = (torch.randn((N, K), generator=g, device=dev) * 0.05).half()
        _check(decode_linear(x, w), _ref(x, w), torch.float16, f"sequence M={M} K={K} N={N}")


def test_packed_weight_refreshes_on_update(dev):
    """The packed copy follows in-place weight updates (version counter)."""
    from mamba_metal_amd.linear import decode_linear

    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn((8, 128), generator=g, device=dev).half()
    w = (torch.randn((64, 128), generator=g, device=dev) * 0.05).half()
    decode_linear(x, w)
    with torch.no_grad():
        w.mul_(-2.0)
    _check(decode_linear(x, w), _ref(x, w), torch.float16, "after update")


def test_decode_linear_strided_rows(dev):
    """x as a column slice of a wider buffer (row stride > K), y into a wider buffer."""
    from mamba_metal_amd.linear import decode_linear

    g = torch.Generator(device=dev).manual_seed(1)
    big = torch.randn((40, 1024 + 64), generator=g, device=dev).half()
    x = big[:, 64:]                                       # 16-byte aligned, stride 1088
    w = (torch.randn((300, 1024), generator=g, device=dev) * 0.05).half()
    outbuf = torch.zeros((40, 320), device=dev, dtype=torch.float16)
    y = decode_linear(x, w, out=outbuf[:, :300])
    _check(y, _ref(x, w), torch.float16, "strided")
    assert torch.count_nonzero(outbuf[:, 300:]) == 0      # nothing written past N


# (64, 5120, 2560): 2.8B out_proj (split K); (40, 128, 16600): shared-X kernel, ragged
# (2, 1536, 768) and (4, 5120, 2560): the M <= 4 GEMV path with the RESID epilogue.
@pytest.mark.parametrize("M,K,N", [(64, 5120, 2560), (40, 128, 16600), (2, 1536, 768),
                                   (4, 5120, 2560)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_linear_resid(dev, M, K, N, dtype):
    from mamba_metal_amd.linear import decode_linear_resid_

    g = torch.Generator(device=dev).manual_seed(2 + N)
    y = torch.randn((M, K), generator=g, device=dev).to(dtype)
    w = (torch.randn((N, K), generator=g, device=dev) * 0.02).to(dtype)
    resid = torch.randn((M, N), generator=g, device=dev).to(dtype)
    r0 = resid.float().cpu().numpy()
    yr = _ref(y, w).to(dtype).float().cpu().numpy()
    expect = (r0 + yr).astype(np.float64)
    decode_linear_resid_(resid, y, w)
    # resid + y cancels: the bound scales with the operands, not with the sum (one
    # rounding of y and one of the sum, each a fraction of |operand|).
    err = np.abs(resid.float().cpu().numpy() - expect)
    bound = TOL[dtype] * (np.abs(r0) + np.abs(yr)) + 1e-6
    assert (err <= bound).all(), f"resid: worst excess {float((err - bound).max()):.3e}"


# (64, 5120, 2560): split K, fused reduce + residual + norm pass; (64, 1024, 8192):
# unsplit, RESID epilogue then the norm kernel; (40, 4096, 1001): split with N % 4 != 0
# (ordered reduce, then the norm kernel); (1, 1536, 768): 130M out_proj at batch 1 (unsplit).
@pytest.mark.parametrize("M,K,N", [(64, 5120, 2560), (64, 1024, 8192), (40, 4096, 1001),
                                   (1, 1536, 768)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_linear_resid_norm(dev, M, K, N, dtype):
    """resid += round(y @ w.T); out = RMSNorm(resid) * norm_w, against fp32 torch."""
    from mamba_metal_amd.linear import decode_linear_resid_norm_

    g = torch.Generator(device=dev).manual_seed(M + K + N)
    y = torch.randn((M, K), generator=g, device=dev).to(dtype)
    w = (torch.randn((N, K), generator=g, device=dev) * 0.02).to(dtype)
    resid = torch.randn((M, N), generator=g, device=dev).to(dtype)
    nw = (1.0 + 0.1 * torch.randn((N,), generator=g, device=dev)).to(dtype)
    r0 = resid.float().cpu().numpy()
    yr = _ref(y, w).to(dtype).float().cpu().numpy()
    out = decode_linear_resid_norm_(resid, y, w, nw, 1e-5)
    got_r = resid.float().cpu().numpy()
    err = np.abs(got_r - (r0 + yr))
    assert (err <= TOL[dtype] * (np.abs(r0) + np.abs(yr)) + 1e-6).all(), "residual"
    # the norm of the residual the kernel produced (rounded to dtype, as stored)
    ref = numpy_ref.rms_norm(got_r.astype(np.float64), nw.float().cpu().numpy().astype(np.float64),
                             eps=1e-5)
    assert_close(out.float().cpu().numpy(), ref, TOL[dtype], TOL[dtype], f"norm M={M} N={N}")


# di = 1536: 130M shape; di = 5120: 2.8B width (two column tiles per wave); di = 8300
# (the conv / z boundary inside a 32-column tile): > 512 column tiles, shared-X kernel
@pytest.mark.parametrize("K,di", [(768, 1536), (256, 5120), (128, 8300)])
@pytest.mark.parametrize("M", [64, 3, 1])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_in_proj_conv(dev, K, di, M, dtype):
    """in_proj + conv-window step == GEMM, then the oracle's decode conv step."""
    from mamba_metal_amd.linear import decode_in_proj_conv

    g = torch.Generator(device=dev).manual_seed(3 + M + di)
    x = torch.randn((M, K), generator=g, device=dev).to(dtype)
    w = (torch.randn((2 * di, K), generator=g, device=dev) * 0.05).to(dtype)
    cw = torch.randn((di, 1, 4), generator=g, device=dev).to(dtype)
    cb = torch.randn((di,), generator=g, device=dev).to(dtype)
    st = torch.randn((M, di, 4), generator=g, device=dev).to(dtype)
    st0 = st.clone()
    x_conv, z = decode_in_proj_conv(x, w, st, cw, cb)
    xz = _ref(x, w).to(dtype)                              # the rounded projection
    _check(z, xz[:, di:].float(), dtype, "z")
    ref, ref_st = numpy_ref.decode_conv_step(st0.float().cpu().numpy().astype(np.float64),
                                             xz[:, :di].float().cpu().numpy().astype(np.float64),
                                             cw.float().cpu().numpy()[:, 0].astype(np.float64),
                                             cb.float().cpu().numpy().astype(np.float64))
    tol = TOL[dtype]
    # an input that lands on a rounding boundary may differ by one ulp of dtype
    assert_close(x_conv.float().cpu().numpy(), ref, tol * 4, tol * 4, "x_conv")
    assert_close(st.float().cpu().numpy(), ref_st, tol, tol * 4, "conv state")


# in_proj + conv window + x_proj (mm_decode_in_proj_xproj).  Fused -- x_proj products
# taken in in_proj's conv epilogue, fp32 partial planes summed by one kernel: 2.8B shape
# at batch 64 and 16 and the 1.4B shape (the split kernel: 32-column conv blocks, one
# plane each, and 64-column z blocks), 130M at batch 16 (one m-tile) and 33 (two), an
# x_proj of 256 columns (every wave two tiles).  Falling back to
# two GEMMs: batch 3 (GEMV in_proj), an x_proj width that is not a multiple of 4, the
# input RMSNorm.  The in_proj outputs must equal decode_in_proj_conv's bit for bit; x_dbl
# is checked against the fp32 product of the returned conv outputs.
@pytest.mark.parametrize("M,K,di,nx,norm,fused", [
    (64, 2560, 5120, 192, False, True), (16, 2560, 5120, 192, False, True),
    (64, 2048, 4096, 160, False, True), (16, 768, 1536, 80, False, True),
    (33, 768, 1536, 80, False, True), (64, 512, 640, 256, False, True),
    (3, 768, 1536, 80, False, False), (8, 768, 1536, 50, False, False),
    (8, 768, 1536, 80, True, False)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_in_proj_conv_xproj(dev, M, K, di, nx, norm, fused, dtype):
    from mamba_metal_amd import _lib
    from mamba_metal_amd.linear import decode_in_proj_conv, decode_in_proj_conv_xproj

    g = torch.Generator(device=dev).manual_seed(7 + M + di + nx)
    x = torch.randn((M, K), generator=g, device=dev).to(dtype)
    w = (torch.randn((2 * di, K), generator=g, device=dev) * 0.05).to(dtype)
    cw = torch.randn((di, 1, 4), generator=g, device=dev).to(dtype)
    cb = torch.randn((di,), generator=g, device=dev).to(dtype)
    wx = (torch.randn((nx, di), generator=g, device=dev) * 0.05).to(dtype)
    st_a = torch.randn((M, di, 4), generator=g, device=dev).to(dtype)
    st_b = st_a.clone()
    st_c = st_a.clone()
    fold = (torch.rand((K,), generator=g, device=dev).to(dtype) + 0.5, 1e-5) if norm else None
    x_conv, z = decode_in_proj_conv(x, w, st_a, cw, cb, x_norm=fold)
    x_conv2, z2, x_dbl = decode_in_proj_conv_xproj(x, w, st_b, cw, cb, wx, x_norm=fold)
    torch.cuda.synchronize()
    assert torch.equal(x_conv2, x_conv) and torch.equal(z2, z) and torch.equal(st_b, st_a)
    _check(x_dbl, _ref(x_conv, wx), dtype, "x_proj")
    _, _, x_dbl2 = decode_in_proj_conv_xproj(x, w, st_c, cw, cb, wx, x_norm=fold)
    assert torch.equal(x_dbl2, x_dbl)                      # fixed summation order
    # the fused shapes size the workspace for one fp32 plane of M x nx per 32 conv columns
    if fused:
        ws = _lib.load().mm_decode_in_proj_xproj_workspace_size(M, 2 * di, K, di, nx)
        assert ws >= (di // 32) * M * nx * 4


# Input RMSNorm folded into the operand load: the product must be bit-identical to the
# separate add_rmsnorm + GEMM (the kernel recomputes the norm in add_rmsnorm's order).
# Shapes: 130M in_proj (conv) at M = 1, 3, 8; 2.8B in_proj (two tiles per wave); a
# split-K store (narrow N, K = 4096: the longest row add_rmsnorm's vector kernel takes,
# 8 chunks per lane); a K whose chunk count is not a multiple of 64 lanes' worth
# (K = 576: 72 chunks of 8).
@pytest.mark.parametrize("M,K,N,conv", [(1, 768, 3072, True), (3, 768, 3072, True),
                                        (8, 768, 3072, True), (1, 2560, 10240, True),
                                        (2, 4096, 192, False), (8, 576, 300, False)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_input_rmsnorm_matches_separate_norm(dev, M, K, N, conv, dtype):
    from mamba_metal_amd.linear import decode_in_proj_conv, decode_linear, norm_in_ok
    from mamba_metal_amd.norm import add_rmsnorm

    g = torch.Generator(device=dev).manual_seed(M * 11 + K + N)
    resid = (torch.randn((M, K), generator=g, device=dev) * 3.0).to(dtype)
    nw = (1.0 + 0.1 * torch.randn((K,), generator=g, device=dev)).to(dtype)
    w = (torch.randn((N, K), generator=g, device=dev) * 0.05).to(dtype)
    eps = 1e-5
    assert norm_in_ok(resid, w, nw)
    h = add_rmsnorm(resid, None, nw, eps)
    if conv:
        n_conv = N // 2
        st0 = torch.randn((M, n_conv, 4), generator=g, device=dev).to(dtype)
        cw = torch.randn((n_conv, 1, 4), generator=g, device=dev).to(dtype)
        cb = torch.randn((n_conv,), generator=g, device=dev).to(dtype)
        st_a, st_b = st0.clone(), st0.clone()
        xa, za = decode_in_proj_conv(h, w, st_a, cw, cb)
        xb, zb = decode_in_proj_conv(resid, w, st_b, cw, cb, x_norm=(nw, eps))
        torch.cuda.synchronize()
        assert torch.equal(xa, xb) and torch.equal(za, zb) and torch.equal(st_a, st_b)
    else:
        ya = decode_linear(h, w)
        yb = decode_linear(resid, w, x_norm=(nw, eps))
        torch.cuda.synchronize()
        assert torch.equal(ya, yb)
        _check(yb, _ref(h, w), dtype, f"norm-in M={M} K={K} N={N}")
    # the residual rows are read, not written
    assert torch.equal(resid, (torch.randn((M, K), generator=torch.Generator(device=dev)
                                           .manual_seed(M * 11 + K + N), device=dev) * 3.0).to(dtype))


def test_input_rmsnorm_rejects_large_m(dev):
    from mamba_metal_amd.linear import decode_linear, norm_in_ok

    x = torch.randn((9, 256), device=dev).half()
    w = torch.randn((64, 256), device=dev).half()
    nw = torch.ones(256, device=dev).half()
    assert not norm_in_ok(x, w, nw)
    with pytest.raises(ValueError):
        decode_linear(x, w, x_norm=(nw, 1e-5))
    x8 = torch.randn((8, 4160), device=dev).half()      # K beyond the vector norm's rows
    w8 = torch.randn((64, 4160), device=dev).half()
    assert not norm_in_ok(x8, w8, torch.ones(4160, device=dev).half())


# The M <= 4 GEMV path (8 output columns per workgroup, all of K): every M it
# instantiates (1, 2 and 4 rows; 3 runs the 4-row kernel with a clamped row), N not a
# multiple of 8 (the last workgroup's columns past N are computed on column 0 and not
# stored), K of one 16-wide step group (64) up to 5120 (several load groups per thread).
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("K,N", [(64, 50), (768, 3072), (5120, 203), (2560, 16384)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_linear_small_m(dev, M, K, N, dtype):
    from mamba_metal_amd.linear import decode_linear

    g = torch.Generator(device=dev).manual_seed(M * 100 + K + N)
    x = torch.randn((M, K), generator=g, device=dev).to(dtype)
    w = (torch.randn((N, K), generator=g, device=dev) * 0.05).to(dtype)
    y = decode_linear(x, w)
    torch.cuda.synchronize()
    _check(y, _ref(x, w), dtype, f"gemv M={M} K={K} N={N}")
    assert torch.equal(y, decode_linear(x, w))      # deterministic


# LM head + greedy argmax in one call (mm_decode_head_argmax): the logits equal
# decode_linear's bit for bit and the ids equal argmax_rows on them.  Shapes: the 130M head
# at batch 1 and 4 and the 2.8B head at batch 64 (shared-X kernel, candidates in its
# epilogue), a narrow N (GEMV / linear_kernel, then mm_argmax_rows); planted ties (two
# equal weight rows: the lower column wins) and a NaN column (it wins, the first of two).
@pytest.mark.parametrize("M,K,N", [(1, 768, 50280), (4, 768, 50280), (64, 2560, 50280),
                                   (8, 512, 3000)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_head_argmax(dev, M, K, N, dtype):
    from mamba_metal_amd.linear import decode_head_argmax, decode_linear
    from mamba_metal_amd.sample import argmax_rows

    g = torch.Generator(device=dev).manual_seed(M + K + N)
    x = torch.randn((M, K), generator=g, device=dev).to(dtype)
    w = (torch.randn((N, K), generator=g, device=dev) * 0.05).to(dtype)
    ids = torch.empty((M,), dtype=torch.int64, device=dev)
    logits = decode_head_argmax(x, w, ids)
    ref = decode_linear(x, w)
    torch.cuda.synchronize()
    assert torch.equal(logits, ref)
    assert torch.equal(ids, argmax_rows(ref))
    assert torch.equal(ids, ref.float().argmax(dim=1))
    # with the next step's embedding rows (the head's tied table) written beside the ids
    emb = torch.full((M, K), float("nan"), dtype=dtype, device=dev)
    ids_e = torch.empty_like(ids)
    lg_e = decode_head_argmax(x, w, ids_e, embed_out=emb)
    torch.cuda.synchronize()
    assert torch.equal(lg_e, ref) and torch.equal(ids_e, ids)
    assert torch.equal(emb, w[ids])
    # ties: every row's winner duplicated at a lower and a higher column
    top = ids.clone()
    w2 = w.clone()
    lo = int(top.min())
    w2[max(lo - 7, 0)] = w2[lo]          # a lower column with the same weights as row lo
    w2[N - 1] = w2[lo]
    ids2 = torch.empty_like(ids)
    lg2 = decode_head_argmax(x, w2, ids2)
    torch.cuda.synchronize()
    assert torch.equal(ids2, argmax_rows(lg2))
    assert torch.equal(ids2, lg2.float().argmax(dim=1))
    # NaN columns: the first one wins on every row
    w3 = w.clone()
    w3[N // 3, 0] = float("nan")
    w3[N // 2, 0] = float("nan")
    ids3 = torch.empty_like(ids)
    decode_head_argmax(x, w3, ids3)
    torch.cuda.synchronize()
    assert torch.equal(ids3, torch.full_like(ids3, N // 3))
