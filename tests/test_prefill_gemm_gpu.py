"""Prefill projection GEMM (mm_prefill_linear) against a float32 torch reference.

The reference is x.float() @ w.float().T (+ bias) on the GPU, a plain fp32 GEMM of the
same op.  The kernel accumulates in fp32 and rounds once to f16/bf16, so the tolerance is
the output dtype's half-ulp plus fp32 accumulation-order noise, relative to the output's
scale (as for the decode GEMM)."""

import pytest
import torch

from helpers import assert_close

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def _inputs(M, K, N, dtype, seed, ldx=None, bias=False):
    g = torch.Generator(device="cuda").manual_seed(seed)
    ldx = ldx or K
    xb = torch.randn((M, ldx), generator=g, device="cuda").to(dtype)
    x = xb[:, :K]
    w = (torch.randn((N, K), generator=g, device="cuda") / K ** 0.5).to(dtype)
    b = torch.randn((N,), generator=g, device="cuda").to(dtype) if bias else None
    return x, w, b


def _check(got, x, w, b, dtype, what):
    ref = x.float() @ w.float().T
    if b is not None:
        ref = ref + b.float()
    scale = float(ref.abs().max()) + 1e-6
    tol = TOL[dtype]
    assert_close(got.float().cpu().numpy(), ref.cpu().numpy(), tol, tol * scale * 0.05, what)


# The dt projection of the Mamba-130M and 2.8B prefills (K = dt_rank, bias, on the strided
# dt slice of x_proj's output), then the other projection shapes (deep K: computed
# correctly, though the model leaves them on torch's GEMM), ragged M and N (partial
# 32-row / 32-column tiles), N <= 96 (the K-split workgroups) with K not a multiple of the
# split, single-step K, and strided x rows.
@pytest.mark.parametrize("M,K,N,ldx,bias", [
    (2048, 768, 3072, None, False), (2048, 1536, 80, None, False), (2048, 48, 1536, 80, True),
    (2048, 1536, 768, None, False), (512, 2560, 10240, None, False), (512, 160, 5120, 192, True),
    (1000, 256, 200, None, False), (37, 64, 33, None, True), (4099, 32, 130, 40, False),
    (100, 1552, 96, None, False), (65, 16, 7, None, True), (1, 768, 3072, None, False),
    (1000, 320, 200, None, True), (77, 1024, 130, 1032, False), (8192, 160, 5120, 192, True),
])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_linear(M, K, N, ldx, bias, dtype):
    from mamba_metal_amd.linear import PREFILL_MAX_K, PREFILL_MAX_M, prefill_linear, prefill_linear_ok
    x, w, b = _inputs(M, K, N, dtype, seed=M + N, ldx=ldx, bias=bias)
    # the model routes short K (and M up to the cap) here; every case is computed either way
    assert prefill_linear_ok(x, w, b) == (K <= PREFILL_MAX_K and M <= PREFILL_MAX_M)
    y = prefill_linear(x, w, b)
    torch.cuda.synchronize()
    _check(y, x, w, b, dtype, f"prefill_linear M={M} K={K} N={N}")


def test_prefill_linear_out_rows_and_empty():
    """A strided output (rows of a wider buffer) keeps the columns past N; M = 0 is a no-op."""
    from mamba_metal_amd.linear import prefill_linear
    x, w, _ = _inputs(300, 128, 100, torch.float16, seed=5)
    buf = torch.full((300, 112), 7.0, dtype=torch.float16, device="cuda")
    y = prefill_linear(x, w, out=buf[:, :100])
    torch.cuda.synchronize()
    _check(y, x, w, None, torch.float16, "strided out")
    assert bool((buf[:, 100:] == 7.0).all())
    e = prefill_linear(x[:0], w)
    assert e.shape == (0, 100)


def test_prefill_linear_deterministic():
    """The K-split workgroups sum their partial tiles in a fixed order: two calls agree
    bit for bit."""
    from mamba_metal_amd.linear import prefill_linear
    x, w, _ = _inputs(2048, 1536, 80, torch.float16, seed=9)
    a = prefill_linear(x, w)
    b = prefill_linear(x, w)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
