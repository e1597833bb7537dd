"""Parity of the conv1d, decode-step and pair-scan HIP kernels against the oracle.

  causal_conv1d    vs numpy_ref.causal_conv1d (itself pinned to torch conv1d):
                   widths 2/3/4 (templated) and 5/8 (generic path), fp32/fp16/bf16,
                   the model's strided (B, L, 2*d_inner) view, D % 8 != 0 (gather path),
                   L < width and conv-state capture (mamba_block.py:118-127)
  conv_step        vs numpy_ref.decode_conv_step, in-place state, fp32/fp16 states
  ssm_step         vs numpy_ref.decode_ssm_step, dstate 4/12/16/64, in-place state
  pair_scan        reference KATs (experiments/05-pair-scan/pair_scan.py:57-81),
                   n = 33/100/513 and beyond one 1024 chunk
Tolerances: fp32 rtol/atol 1e-5; fp16 1e-3; bf16 8e-3 (output rounding).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close
from oracle import numpy_ref

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-5, 1e-5), torch.float16: (1e-3, 1e-3), torch.bfloat16: (8e-3, 8e-3)}


def _r(x, dtype):
    return torch.as_tensor(x).to(dtype).float().numpy().astype(np.float64)


@pytest.mark.parametrize("width", [2, 3, 4, 5, 8])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_causal_conv1d(dev, width, dtype):
    from mamba_metal_amd.conv1d import causal_conv1d

    rng = np.random.default_rng(width)
    b, L, D = 2, 77, 96
    x = rng.standard_normal((b, L, D)).astype(np.float32)
    w = (rng.standard_normal((D, 1, width)) * 0.5).astype(np.float32)
    bias = rng.standard_normal(D).astype(np.float32)
    xt = torch.as_tensor(x).to(dev, dtype)
    wt = torch.as_tensor(w).to(dev, dtype)
    bt = torch.as_tensor(bias).to(dev, dtype)
    st = torch.empty((b, D, width), dtype=dtype, device=dev)
    out = causal_conv1d(xt, wt, bt, conv_state_out=st)
    ref, ref_st = numpy_ref.causal_conv1d(_r(x, dtype), _r(w, dtype)[:, 0], _r(bias, dtype))
    rt, at = TOL[dtype]
    assert_close(out.float().cpu().numpy(), ref, rt, at, f"conv w={width} {dtype}")
    assert_close(st.float().cpu().numpy(), ref_st, 0, 0, "conv state")


@pytest.mark.parametrize("case", ["model_view", "odd_dim", "short", "single"])
def test_causal_conv1d_layouts(dev, case):
    from mamba_metal_amd.conv1d import causal_conv1d

    rng = np.random.default_rng(7)
    b, L, D, K = {"model_view": (3, 50, 64, 4), "odd_dim": (2, 40, 13, 4),
                  "short": (2, 3, 16, 4), "single": (1, 1, 8, 4)}[case]
    xz = rng.standard_normal((b, L, 2 * D)).astype(np.float32)
    w = rng.standard_normal((D, 1, K)).astype(np.float32)
    bias = rng.standard_normal(D).astype(np.float32)
    xzt = torch.as_tensor(xz, device=dev).half()
    x = xzt[..., :D]  # the model's in_proj split: stride (L*2D, 2D, 1)
    st = torch.empty((b, D, K), dtype=torch.float16, device=dev)
    out = causal_conv1d(x, torch.as_tensor(w, device=dev).half(), torch.as_tensor(bias, device=dev).half(),
                        conv_state_out=st)
    ref, ref_st = numpy_ref.causal_conv1d(_r(xz[..., :D], torch.float16), _r(w, torch.float16)[:, 0],
                                          _r(bias, torch.float16))
    assert_close(out.float().cpu().numpy(), ref, 1e-3, 1e-3, case)
    assert_close(st.float().cpu().numpy(), ref_st, 0, 0, case + " state")


def test_causal_conv1d_no_silu_fp32_weights(dev):
    from mamba_metal_amd.conv1d import causal_conv1d

    rng = np.random.default_rng(8)
    x = rng.standard_normal((1, 30, 32)).astype(np.float32)
    w = rng.standard_normal((32, 1, 4)).astype(np.float32)
    out = causal_conv1d(torch.as_tensor(x, device=dev).half(), torch.as_tensor(w, device=dev), None,
                        apply_silu=False)
    ref, _ = numpy_ref.causal_conv1d(_r(x, torch.float16), w[:, 0].astype(np.float64), None,
                                     apply_silu=False)
    assert_close(out.float().cpu().numpy(), ref, 1e-3, 1e-3, "no silu")


@pytest.mark.parametrize("state_dtype,dtype", [(torch.float32, torch.float32),
                                               (torch.float32, torch.float16),
                                               (torch.float16, torch.float16),
                                               (torch.bfloat16, torch.bfloat16)])
def test_conv_step(dev, state_dtype, dtype):
    from mamba_metal_amd.conv1d import conv_step

    rng = np.random.default_rng(9)
    b, D, K = 5, 200, 4
    st0 = rng.standard_normal((b, D, K)).astype(np.float32)
    x = rng.standard_normal((b, 2 * D)).astype(np.float32)       # xz row; x = first half
    w = rng.standard_normal((D, 1, K)).astype(np.float32)
    bias = rng.standard_normal(D).astype(np.float32)
    st = torch.as_tensor(st0).to(dev, state_dtype)
    xt = torch.as_tensor(x).to(dev, dtype)[:, :D]
    out = conv_step(st, xt, torch.as_tensor(w).to(dev, dtype), torch.as_tensor(bias).to(dev, dtype))
    ref, ref_st = numpy_ref.decode_conv_step(_r(st0, state_dtype), _r(x[:, :D], dtype),
                                             _r(w, dtype)[:, 0], _r(bias, dtype))
    rt, at = TOL[dtype]
    assert_close(out.float().cpu().numpy(), ref, rt, at, "conv step")
    assert_close(st.float().cpu().numpy(), _r(ref_st, state_dtype), 0, 0, "conv step state")


@pytest.mark.parametrize("N", [4, 12, 16, 64])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_ssm_step(dev, N, dtype):
    from mamba_metal_amd.decode import ssm_step

    rng = np.random.default_rng(N)
    b, D, R = 3, 300, 6
    h0 = rng.standard_normal((b, D, N)).astype(np.float32)
    x = rng.standard_normal((b, D)).astype(np.float32)
    dt = rng.uniform(-4, 3, (b, D)).astype(np.float32)
    xdbl = rng.standard_normal((b, R + 2 * N)).astype(np.float32)   # B, C as slices, like the model
    z = rng.standard_normal((b, D)).astype(np.float32)
    A = -rng.uniform(0.1, 2.0, (D, N)).astype(np.float32)
    Dp = rng.standard_normal(D).astype(np.float32)
    hb = rng.uniform(-1, 1, D).astype(np.float32)
    h = torch.as_tensor(h0, device=dev)
    xd = torch.as_tensor(xdbl).to(dev, dtype)
    y = ssm_step(h, torch.as_tensor(x).to(dev, dtype), torch.as_tensor(dt).to(dev, dtype),
                 torch.as_tensor(A, device=dev), xd[:, R:R + N], xd[:, R + N:],
                 D=torch.as_tensor(Dp, device=dev), z=torch.as_tensor(z).to(dev, dtype),
                 dt_bias=torch.as_tensor(hb, device=dev))
    ref_y, ref_h = numpy_ref.decode_ssm_step(h0, _r(x, dtype), _r(dt, dtype), A,
                                             _r(xdbl, dtype)[:, R:R + N], _r(xdbl, dtype)[:, R + N:],
                                             D=Dp, z=_r(z, dtype), dt_bias=hb)
    rt, at = TOL[dtype]
    assert_close(y.float().cpu().numpy(), ref_y, rt, at, f"ssm step y N={N}")
    assert_close(h.cpu().numpy(), ref_h, 1e-5, 1e-5, f"ssm step h N={N}")


def _pair(dev, a, b):
    from mamba_metal_amd._loader import pair_scan

    pa, h = pair_scan(torch.as_tensor(a, device=dev), torch.as_tensor(b, device=dev))
    torch.cuda.synchronize()
    return pa.cpu().numpy(), h.cpu().numpy()


def test_pair_scan_known_answers(dev):
    n = 1024
    i = np.arange(n)
    pa, h = _pair(dev, np.full(n, 0.5, np.float32), np.ones(n, np.float32))
    assert_close(h, 2.0 * (1.0 - 0.5 ** (i + 1)), 1e-6, 1e-7, "a=0.5 b=1")
    assert abs(h[-1] - 2.0) < 1e-6
    rng = np.random.default_rng(0)
    a = rng.uniform(0.0, 1.0, n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    ref_pa, ref_h = numpy_ref.pair_scan(a, b)
    pa, h = _pair(dev, a, b)
    assert_close(h, ref_h, 1e-5, 1e-6, "random")
    assert_close(pa, ref_pa, 1e-5, 1e-30, "random prod")
    delta = rng.uniform(0.01, 0.1, n).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    a = np.exp(-delta).astype(np.float32)
    b = (delta * u).astype(np.float32)
    _, h = _pair(dev, a, b)
    assert_close(h, numpy_ref.pair_scan(a, b)[1], 1e-5, 1e-6, "mamba-like")


@pytest.mark.parametrize("n", [1, 33, 100, 513, 1025, 5000])
def test_pair_scan_sizes(dev, n):
    rng = np.random.default_rng(n)
    a = rng.uniform(0.5, 1.0, n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    pa, h = _pair(dev, a, b)
    ref_pa, ref_h = numpy_ref.pair_scan(a, b)
    assert_close(h, ref_h, 1e-5, 1e-5, f"n={n}")
    assert_close(pa, ref_pa, 1e-5, 1e-30, f"n={n} prod")


def test_load_kernel_calling_convention(dev):
    """load_kernel keeps the reference's mx.fast.metal_kernel calling convention."""
    from mamba_metal_amd import load_kernel

    k = load_kernel("pair_scan", input_names=["a_in", "b_in", "n"], output_names=["a_out", "h_out"])
    a = torch.full((100,), 0.5, device=dev)
    b = torch.ones(100, device=dev)
    a_out, h_out = k(inputs=[a, b, 100], output_shapes=[(100,), (100,)],
                     output_dtypes=[torch.float32] * 2, grid=(1024, 1, 1), threadgroup=(1024, 1, 1))
    assert abs(float(h_out[-1]) - 2.0) < 1e-6
    with pytest.raises(FileNotFoundError):
        load_kernel("vector_add", ["a", "b"], ["c"])


# (16, R): the fused kernel -- R 48/100/160/200/256 hit each register-slice width,
# 30 and 100 take the element-wise W loads (R % 8 != 0 / misaligned rows); other N
# take the GEMM + ssm_step composition.
@pytest.mark.parametrize("N,R", [(16, 160), (16, 48), (16, 30), (16, 100), (16, 200), (16, 256),
                                 (4, 7), (64, 256), (12, 30)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_ssm_step_dtproj(dev, N, R, dtype):
    """Fused dt_proj + softplus + SSM step == oracle step on dt = dt_in @ W.T + b."""
    from mamba_metal_amd.decode import ssm_step_dtproj

    rng = np.random.default_rng(N * 1000 + R)
    b, D = 37, 200
    h0 = rng.standard_normal((b, D, N)).astype(np.float32)
    x = rng.standard_normal((b, D)).astype(np.float32)
    xdbl = (rng.standard_normal((b, R + 2 * N)) * 0.5).astype(np.float32)
    W = (rng.standard_normal((D, R)) * 0.2).astype(np.float32)
    bias = rng.uniform(-3, 0, D).astype(np.float32)
    z = rng.standard_normal((b, D)).astype(np.float32)
    A = -rng.uniform(0.1, 2.0, (D, N)).astype(np.float32)
    Dp = rng.standard_normal(D).astype(np.float32)
    h = torch.as_tensor(h0, device=dev)
    xd = torch.as_tensor(xdbl).to(dev, dtype)
    y = ssm_step_dtproj(h, torch.as_tensor(x).to(dev, dtype), xd[:, :R], torch.as_tensor(W).to(dev, dtype),
                        torch.as_tensor(A, device=dev), xd[:, R:R + N], xd[:, R + N:],
                        dt_bias=torch.as_tensor(bias).to(dev, dtype), D=torch.as_tensor(Dp, device=dev),
                        z=torch.as_tensor(z).to(dev, dtype))
    from mamba_metal_amd.decode import dtproj_fused_ok

    fused = dtproj_fused_ok(N, R, dtype, dtype)
    xr = _r(xdbl, dtype)
    dt = xr[:, :R] @ _r(W, dtype).T + _r(bias, dtype)[None]
    if not fused:
        dt = _r(dt, dtype)   # the GEMM composition rounds dt to the activation dtype
    ref_y, ref_h = numpy_ref.decode_ssm_step(h0, _r(x, dtype), dt, A, xr[:, R:R + N], xr[:, R + N:],
                                             D=Dp, z=_r(z, dtype))
    rt, at = TOL[dtype]
    assert_close(y.float().cpu().numpy(), ref_y, rt, at, f"dtproj y N={N} R={R}")
    # fp32 state: the fused kernel keeps dt in fp32, so h meets fp32 tolerance; the
    # composition's rounded dt may sit one ulp of the activation dtype away.
    ht = (1e-5, 1e-5) if fused or dtype == torch.float32 else (rt, at)
    assert_close(h.cpu().numpy(), ref_h, *ht, f"dtproj h N={N} R={R}")



@pytest.mark.parametrize("dim", [64, 768, 2560, 1000])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_add_rmsnorm(dev, dim, dtype):
    from mamba_metal_amd.norm import add_rmsnorm

    rng = np.random.default_rng(dim)
    rows = 33
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    a = rng.standard_normal((rows, dim)).astype(np.float32)
    w = rng.standard_normal(dim).astype(np.float32)
    xt = torch.as_tensor(x).to(dev, dtype)
    wt = torch.as_tensor(w).to(dev, dtype)
    out = add_rmsnorm(xt, torch.as_tensor(a).to(dev, dtype), wt, 1e-5)
    s = torch.as_tensor(_r(x, dtype) + _r(a, dtype)).to(dtype).float().numpy()  # residual rounds
    assert_close(xt.float().cpu().numpy(), s, 0, 0, "residual")
    ref = numpy_ref.rms_norm(s, _r(w, dtype))
    rt, at = TOL[dtype]
    assert_close(out.float().cpu().numpy(), ref, rt, at, f"rmsnorm dim={dim}")
    out2 = add_rmsnorm(xt, None, wt, 1e-5)           # no add: plain RMSNorm
    assert_close(out2.float().cpu().numpy(), ref, rt, at, "rmsnorm no-add")


@pytest.mark.parametrize("n", [50280, 50277, 768, 1])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_argmax_rows(dev, n, dtype):
    """Greedy ids == torch.argmax, incl. planted ties (lowest index wins) and NaN."""
    from mamba_metal_amd.sample import argmax_rows

    g = torch.Generator(device=dev).manual_seed(n)
    x = torch.randn((37, n), generator=g, device=dev).to(dtype)
    if n > 10:
        x[3, 5] = x[3, n - 2] = 100.0            # tie: index 5 wins
        x[4, 7] = float("nan")                   # NaN beats numbers
        x[5, :] = 1.0                            # all equal: index 0
        x[6, :] = float("-inf")                  # all -inf: index 0
        x[7, 9:] = float("nan")                  # many NaNs: the first one
    got = argmax_rows(x)
    assert torch.equal(got, torch.argmax(x, dim=-1))
    # strided rows (a column slice of a wider buffer)
    wide = torch.randn((9, n + 24), generator=g, device=dev).to(dtype)
    assert torch.equal(argmax_rows(wide[:, :n]), torch.argmax(wide[:, :n], dim=-1))
