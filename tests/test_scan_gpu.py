"""Parity of the HIP selective scan against the CPU oracle (runs on the MI355X).

Cases restate the reference's own scan checks, now with assertions:
  06-selective-scan (minimal shapes), 07-chunked (chunk boundaries 1024/1025),
  09-features (D / z / softplus matrix), 10-fp16 (fp16 in, fp32 math),
  18-prefill/verify_state_out (final state)
plus edge shapes, strided layouts, dtypes, determinism and the BASELINE
configs (config 0 against the committed golden fixture; configs 2 and 4 at full
size with one channel of every 16-channel block against the oracle -- channels are
independent, so any subset must match the oracle run on that subset alone).

Tolerances (from the task's parity bar): fp32 rtol 1e-5 (atol 1e-5 for |y| ~ 0);
fp16 / bf16 inputs with fp32 math: rtol 1e-3, atol 1e-3 against the oracle run on
the same rounded inputs (bf16 output rounding needs rtol 8e-3).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import (assert_close, config0_inputs, features_inputs, fp16_inputs, plain_inputs)

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL = {torch.float32: (1e-5, 1e-5), torch.float16: (1e-3, 1e-3), torch.bfloat16: (8e-3, 2e-3)}


def to_dev(a, dtype, dev):
    return None if a is None else torch.as_tensor(a).to(dev, dtype)


def rounded(a, dtype):
    if a is None:
        return None
    return torch.as_tensor(a).to(dtype).float().numpy()


def gpu_scan(inp, dev, dtype=torch.float32, bc_dtype=None, softplus=False, use_D=True,
             use_z=True, return_state=True, layout="bdl"):
    from mamba_metal_amd import selective_scan

    bc_dtype = bc_dtype or dtype
    u, d, z = (to_dev(inp[k], dtype, dev) for k in ("u", "delta", "z"))
    B, C = (to_dev(inp[k], bc_dtype, dev) for k in ("B", "C"))
    A = to_dev(inp["A"], torch.float32, dev)
    D = to_dev(inp["D"], torch.float32, dev) if use_D else None
    z = z if use_z else None
    if layout == "bld":  # (batch, seqlen, dim) storage viewed as (batch, dim, seqlen)
        u, d = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (u, d))
        z = None if z is None else z.transpose(1, 2).contiguous().transpose(1, 2)
        B, C = (t.transpose(1, 2).contiguous().transpose(1, 2) for t in (B, C))
    elif layout == "gather":  # non-unit strides on every axis
        def spread(t):
            big = torch.zeros((t.shape[0], t.shape[1] * 2, t.shape[2] * 3), dtype=t.dtype, device=dev)
            big[:, ::2, ::3] = t
            return big[:, ::2, ::3]
        u, d, B, C = map(spread, (u, d, B, C))
        z = None if z is None else spread(z)
    out = selective_scan(u, d, A, B, C, D=D, z=z, delta_softplus=softplus,
                         return_state=return_state)
    torch.cuda.synchronize()
    if return_state:
        y, h = out
        assert y.dtype == dtype and h.dtype == torch.float32
        return y.float().cpu().numpy(), h.cpu().numpy()
    return out.float().cpu().numpy(), None


def oracle_scan(oracle_lib, inp, dtype=torch.float32, bc_dtype=None, softplus=False, use_D=True,
                use_z=True, precision="f64"):
    bc_dtype = bc_dtype or dtype
    r = {k: rounded(inp[k], dtype) for k in ("u", "delta", "z")}
    r.update({k: rounded(inp[k], bc_dtype) for k in ("B", "C")})
    return oracle_lib.selective_scan(r["u"], r["delta"], inp["A"], r["B"], r["C"],
                                     D=inp["D"] if use_D else None,
                                     z=r["z"] if use_z else None, delta_softplus=softplus,
                                     precision=precision)


def check(oracle_lib, dev, inp, what, dtype=torch.float32, bc_dtype=None, softplus=False,
          use_D=True, use_z=True, layout="bdl"):
    yg, hg = gpu_scan(inp, dev, dtype, bc_dtype, softplus, use_D, use_z, layout=layout)
    yo, ho = oracle_scan(oracle_lib, inp, dtype, bc_dtype, softplus, use_D, use_z)
    rt, at = TOL[dtype]
    assert_close(yg, yo, rt, at, f"{what} y")
    assert_close(hg, ho, max(rt, 1e-5), max(at, 1e-5), f"{what} state")


# --- experiments/06-selective-scan/selective_scan.py:79-82 ------------------
@pytest.mark.parametrize("shape", [(1, 1, 4, 32), (1, 1, 16, 128), (2, 4, 16, 256), (2, 8, 16, 1024)])
def test_minimal_shapes(oracle_lib, dev, shape):
    check(oracle_lib, dev, plain_inputs(*shape, seed=0), f"minimal {shape}", use_D=False, use_z=False)


# --- experiments/07-chunked/selective_scan_chunked.py:139-145 ---------------
@pytest.mark.parametrize("shape", [(1, 2, 8, 512), (1, 2, 8, 1024), (1, 2, 8, 1025), (1, 4, 16, 2048),
                                   (2, 4, 16, 4096), (1, 2, 16, 8192), (1, 2, 16, 16384)])
def test_chunked_shapes(oracle_lib, dev, shape):
    check(oracle_lib, dev, plain_inputs(*shape, seed=1), f"chunked {shape}", use_D=False, use_z=False)


# --- experiments/09-features/test_features.py:100-115 -----------------------
FLAGS = [(False, False, False), (True, False, False), (False, False, True), (False, True, False),
         (True, True, False), (True, False, True), (True, True, True)]


@pytest.mark.parametrize("use_D,use_z,softplus", FLAGS)
@pytest.mark.parametrize("T", [1024, 4096])
def test_feature_matrix(oracle_lib, dev, use_D, use_z, softplus, T):
    if T == 4096 and not (use_D and use_z and softplus):
        pytest.skip("the reference runs only the all-flags case at T=4096")
    inp = features_inputs(2, 4, 16, T, seed=2)
    if not softplus:  # the reference feeds softplus(delta) when the kernel flag is off
        inp["delta"] = np.log1p(np.exp(inp["delta"].astype(np.float64))).astype(np.float32)
    check(oracle_lib, dev, inp, f"features D={use_D} z={use_z} sp={softplus}", softplus=softplus,
          use_D=use_D, use_z=use_z)


# --- experiments/10-fp16/test_fp16.py:229-243 --------------------------------
@pytest.mark.parametrize("use_D,use_z,softplus,shape", [
    (False, False, False, (2, 4, 16, 1024)), (True, False, False, (2, 4, 16, 1024)),
    (False, True, False, (2, 4, 16, 1024)), (False, False, True, (2, 4, 16, 1024)),
    (True, True, True, (2, 4, 16, 1024)), (True, True, True, (2, 4, 16, 4096)),
    (True, True, True, (1, 2, 16, 16384))])
def test_fp16(oracle_lib, dev, use_D, use_z, softplus, shape):
    check(oracle_lib, dev, fp16_inputs(*shape, seed=3), f"fp16 {shape}", dtype=torch.float16,
          softplus=softplus, use_D=use_D, use_z=use_z)


# --- experiments/18-prefill/verify_state_out.py:31-49 -----------------------
@pytest.mark.parametrize("shape", [(1, 2, 8, 256), (2, 4, 16, 1024), (1, 4, 16, 4096)])
def test_state_out(oracle_lib, dev, shape):
    check(oracle_lib, dev, plain_inputs(*shape, seed=4), f"state {shape}", use_D=False, use_z=False)


# --- edges -------------------------------------------------------------------
@pytest.mark.parametrize("L", [1, 2, 7, 8, 31, 32, 33, 63, 1023, 1025])
def test_edge_seqlen(oracle_lib, dev, L):
    check(oracle_lib, dev, config0_inputs(1, 3, 16, L, seed=L), f"L={L}", softplus=True)


@pytest.mark.parametrize("N", [1, 2, 3, 4, 5, 8, 9, 12, 15, 16, 17, 24, 32, 33, 48, 64])
def test_edge_dstate(oracle_lib, dev, N):
    check(oracle_lib, dev, features_inputs(2, 5, N, 200, seed=N), f"N={N}", softplus=True)


@pytest.mark.parametrize("N", [4, 8, 16, 24, 64])
def test_dstate_many_chains(oracle_lib, dev, N):
    """dstate shapes on the chained path with many channel blocks (2 x 4160 channels: 130
    64-channel blocks, past the split mode's 128): 32-channel blocks with 1 or 2 states per
    lane for N <= 16, 64-channel blocks with 8 or 16 for larger N; 4160 = 130 x 32, and a
    300-step sequence ends inside a tile.  y is a sum of N terms C[n]*h[n] of magnitude ~2-4
    that largely cancel, so its fp32 rounding grows with N (over these 2.5 M outputs the
    worst N = 64 element was 6.1e-5 off at |y| = 0.86).  The bar is therefore set by a
    plain fp32 evaluation of the same recurrence (the C oracle in fp32, libm expf): y's
    absolute bar is the larger of 1e-5 and twice the fp32 oracle's own worst error against
    the fp64 one on these inputs, so the kernel must be no worse than that; the states keep
    the plain 1e-5 bar."""
    inp = features_inputs(2, 4160, N, 300, seed=100 + N)
    yg, hg = gpu_scan(inp, dev, torch.float32, None, True, True, True)
    yo, ho = oracle_scan(oracle_lib, inp, torch.float32, None, True, True, True)
    y32, _ = oracle_scan(oracle_lib, inp, torch.float32, None, True, True, True, precision="f32")
    e32 = float(np.abs(y32.astype(np.float64) - yo).max())
    eg = float(np.abs(np.asarray(yg, np.float64) - yo).max())
    print(f"[dstate {N}] max |y - fp64 oracle|: kernel {eg:.2e}, fp32 oracle {e32:.2e}")
    assert_close(yg, yo, 1e-5, max(1e-5, 2 * e32), f"N={N} many chains y")
    assert_close(hg, ho, 1e-5, 1e-5, f"N={N} many chains state")


@pytest.mark.parametrize("dim", [1, 63, 64, 65, 130])
def test_edge_dim(oracle_lib, dev, dim):
    check(oracle_lib, dev, features_inputs(3, dim, 16, 96, seed=dim), f"D={dim}", softplus=True)


def test_empty_and_state_only(dev):
    from mamba_metal_amd import selective_scan

    u = torch.zeros((2, 3, 0), device=dev)
    A = -torch.ones((3, 16), device=dev)
    B = torch.zeros((2, 16, 0), device=dev)
    y, h = selective_scan(u, u, A, B, B, return_state=True)
    assert y.shape == (2, 3, 0) and h.shape == (2, 3, 16) and torch.all(h == 0)


# --- layouts and dtypes ------------------------------------------------------
@pytest.mark.parametrize("layout", ["bld", "gather"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_layouts(oracle_lib, dev, layout, dtype):
    inp = config0_inputs(2, 64, 16, 256, seed=5) if dtype == torch.float32 else \
        fp16_inputs(2, 64, 16, 256, seed=5)
    check(oracle_lib, dev, inp, f"layout {layout}", dtype=dtype, softplus=True, layout=layout)


@pytest.mark.parametrize("layout", ["bdl", "bld"])
def test_48_and_16_channel_blocks(oracle_lib, dev, layout):
    """B=8 D=1536 (384 32-channel chains, 256 48-channel ones, 768 16-channel ones on 256
    CUs): channel-contiguous inputs run the 48-channel blocks of 6 waves (thread t: channel
    t % 48, state group t / 48), time-contiguous ones the 16-channel blocks of one state per
    lane; a 300-step sequence ends inside a tile."""
    inp = fp16_inputs(8, 1536, 16, 300, seed=48)
    check(oracle_lib, dev, inp, f"48/16-channel blocks {layout}", dtype=torch.float16,
          softplus=True, layout=layout)


def _single_state_dim(cus, batch):
    """A ragged dim (16 k - 8) whose time-contiguous scan runs the 16-channel blocks of one
    state per lane on a part with `cus` CUs: 2 cus < batch * k <= 3 cus 16-channel chains
    and more than 128 64-channel ones (no split scan at short lengths)."""
    for k in range(2 * cus // batch + 1, 3 * cus // batch + 1):
        dim = 16 * k - 8
        if batch * -(-dim // 64) > 128:
            return dim
    pytest.skip(f"no ragged 16-channel-block shape at batch {batch} on {cus} CUs")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("seqlen", [300, 301])
def test_16_channel_blocks_ragged(oracle_lib, dev, dtype, seqlen):
    """16-channel blocks (one state per lane) with a partial last block (dim = 16 k - 8,
    2728 at batch 3 on 256 CUs) and a sequence ending inside a tile; an odd length takes the
    element-wise (non-vector) loads.  dstate 16 and 12 (padded states)."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    dim = _single_state_dim(cus, 3)
    for n, seed in ((16, 16), (12, 12)):
        inp = fp16_inputs(3, dim, n, seqlen, seed=seed) if dtype != torch.float32 else \
            features_inputs(3, dim, n, seqlen, seed=seed)
        check(oracle_lib, dev, inp, f"16-channel blocks N={n} L={seqlen} {dtype}", dtype=dtype,
              softplus=True)


def test_channel_contiguous_views_keep_their_layout(oracle_lib, dev):
    """Transposed (batch, seqlen, dim) views in: y comes back in the same layout (so the
    kernel's channel-contiguous path runs end to end) with the oracle's values."""
    from mamba_metal_amd import selective_scan

    inp = fp16_inputs(2, 128, 16, 512, seed=8)
    t = lambda a: torch.as_tensor(a).to(dev, torch.float16).transpose(1, 2).contiguous().transpose(1, 2)
    u, d, z, B, C = (t(inp[k]) for k in ("u", "delta", "z", "B", "C"))
    A = torch.as_tensor(inp["A"]).to(dev)
    D = torch.as_tensor(inp["D"]).to(dev)
    y, h = selective_scan(u, d, A, B, C, D=D, z=z, delta_softplus=True, return_state=True)
    torch.cuda.synchronize()
    assert y.shape == u.shape and y.stride() == u.stride()
    yo, ho = oracle_scan(oracle_lib, inp, torch.float16, softplus=True)
    assert_close(y.float().cpu().numpy(), yo, 1e-3, 1e-3, "channel-contiguous y")
    assert_close(h.cpu().numpy(), ho, 1e-3, 1e-3, "channel-contiguous state")


def test_unaligned_seqlen_uses_gather_path(oracle_lib, dev):
    # L % 8 != 0 disables the 16-byte vector path for the (batch, dim, seqlen) layout.
    check(oracle_lib, dev, fp16_inputs(2, 40, 16, 101, seed=6), "L=101 fp16", dtype=torch.float16,
          softplus=True)


@pytest.mark.parametrize("dtype,bc_dtype", [(torch.bfloat16, torch.bfloat16),
                                            (torch.float16, torch.float32),
                                            (torch.bfloat16, torch.float32),
                                            (torch.float32, torch.float16)])
def test_dtype_mixes(oracle_lib, dev, dtype, bc_dtype):
    check(oracle_lib, dev, fp16_inputs(2, 8, 16, 512, seed=7), f"{dtype}/{bc_dtype}", dtype=dtype,
          bc_dtype=bc_dtype, softplus=True)


def test_mixed_input_dtypes_promote(oracle_lib, dev):
    """u fp16 with delta fp32: computed from the exact values, y stored as fp16."""
    from mamba_metal_amd import selective_scan

    inp = fp16_inputs(1, 4, 16, 256, seed=8)
    u = torch.as_tensor(inp["u"]).to(dev, torch.float16)
    d = torch.as_tensor(inp["delta"]).to(dev, torch.float32)
    A, B, C = (torch.as_tensor(inp[k]).to(dev) for k in ("A", "B", "C"))
    y = selective_scan(u, d, A, B, C, delta_softplus=True)
    assert y.dtype == torch.float16
    yo, _ = oracle_lib.selective_scan(u.float().cpu().numpy(), inp["delta"], inp["A"], inp["B"],
                                      inp["C"], delta_softplus=True)
    assert_close(y.float().cpu().numpy(), yo, 1e-3, 1e-3, "promoted")


def test_deterministic(dev):
    inp = fp16_inputs(2, 128, 16, 2048, seed=9)
    y1, h1 = gpu_scan(inp, dev, torch.float16, softplus=True)
    y2, h2 = gpu_scan(inp, dev, torch.float16, softplus=True)
    assert np.array_equal(y1, y2) and np.array_equal(h1, h2)


def test_shape_asserts(dev):
    from mamba_metal_amd import selective_scan

    u = torch.zeros((1, 4, 8), device=dev)
    A = torch.zeros((4, 16), device=dev)
    B = torch.zeros((1, 16, 8), device=dev)
    with pytest.raises(AssertionError):
        selective_scan(u, u[:, :, :4], A, B, B)
    with pytest.raises(AssertionError):
        selective_scan(u, u, A, B, B[:, :8])
    with pytest.raises(AssertionError):
        selective_scan(u, u, torch.zeros((4, 65), device=dev), torch.zeros((1, 65, 8), device=dev),
                       torch.zeros((1, 65, 8), device=dev))


# --- BASELINE configs ----------------------------------------------------------
def test_config0_against_golden(dev):
    """Config 0 (fp32 B=1 D=16 N=16 L=4096, all flags) against the committed fixture."""
    g = np.load(GOLDEN / "scan_config0.npz")
    inp = config0_inputs(1, 16, 16, 4096, seed=0)
    assert np.array_equal(inp["u"][0, 0, :8], g["u_head"]), "input generator drifted"
    y, h = gpu_scan(inp, dev, torch.float32, softplus=True)
    assert_close(y, g["y"], 1e-5, 1e-5, "config0 y")
    assert_close(h, g["state"], 1e-5, 1e-5, "config0 state")


def _blockwise_parity(oracle_lib, dev, batch, dim, seqlen, seed, dtype=torch.float16):
    """Full-size fp16 (or bf16) scan on the GPU; the fp64 oracle on one channel of EVERY 16-channel
    block (a random lane per block, plus the first and last channel): the kernel's
    chains are blocks of 64, 48, 32 or 16 channels, each with its own segment hand-offs, so
    every chain's hand-offs are checked.  Channels are independent, so a subset must match the
    oracle run on that subset."""
    from mamba_metal_amd import selective_scan
    from mamba_metal_amd.selective_scan import reset_scan_status, scan_status

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    f16 = dtype
    u = torch.randn((batch, dim, seqlen), generator=g, device=dev, dtype=torch.float32).to(f16)
    d = (torch.randn((batch, dim, seqlen), generator=g, device=dev) * 0.5 - 1.0).to(f16)
    z = torch.randn((batch, dim, seqlen), generator=g, device=dev).to(f16)
    B = torch.randn((batch, 16, seqlen), generator=g, device=dev).to(f16)
    C = torch.randn((batch, 16, seqlen), generator=g, device=dev).to(f16)
    A = -torch.arange(1, 17, device=dev, dtype=torch.float32).expand(dim, 16).contiguous()
    D = torch.ones(dim, device=dev)
    reset_scan_status(dev)
    y, h = selective_scan(u, d, A, B, C, D=D, z=z, delta_softplus=True, return_state=True)
    torch.cuda.synchronize()
    assert scan_status(dev) == 0    # every segment hand-off completed
    assert torch.isfinite(y).all()
    rng = np.random.default_rng(seed)
    nblk = -(-dim // 16)
    checked = 0
    for b in range(batch):
        chans = np.minimum(np.arange(nblk) * 16 + rng.integers(0, 16, nblk), dim - 1)
        chans = np.unique(np.concatenate([chans, [0, dim - 1]]))
        idx = torch.as_tensor(chans, device=dev)
        pick = lambda t: t[b:b + 1].index_select(1, idx).float().cpu().numpy()
        yo, ho = oracle_lib.selective_scan(pick(u), pick(d), A.index_select(0, idx).cpu().numpy(),
                                           B[b:b + 1].float().cpu().numpy(),
                                           C[b:b + 1].float().cpu().numpy(),
                                           D=D.index_select(0, idx).cpu().numpy(), z=pick(z),
                                           delta_softplus=True)
        ytol = 1e-3 if dtype == torch.float16 else 8e-3  # bf16 output rounding
        assert_close(pick(y), yo, ytol, ytol, f"batch {b} channels {chans.tolist()} y")
        assert_close(h[b:b + 1].index_select(1, idx).cpu().numpy(), ho, 1e-3, 1e-3,
                     f"batch {b} state")
        checked += len(chans)
    assert checked >= batch * nblk


def test_split_mode_matches_chained(oracle_lib, dev):
    """Few channel chains take the split path (segment summaries, then every segment from
    the folded carry); many take the chained path.  A slice of a chained-mode call, rerun
    alone, goes split: each must match the fp64 oracle at the fp32 bar, so the two lie
    within twice that of each other.  A spans [-2, -0.001] with delta <= 0.1 and no
    softplus, so the slowest states carry across many 128-step segments (checked below)."""
    from mamba_metal_amd import selective_scan

    g = torch.Generator(device=dev)
    g.manual_seed(11)
    batch, dim, n, L = 3, 5120, 16, 2048    # 240 channel blocks: chained
    u = torch.randn((batch, dim, L), generator=g, device=dev)
    d = torch.rand((batch, dim, L), generator=g, device=dev) * 0.09 + 0.01
    z = torch.randn((batch, dim, L), generator=g, device=dev)
    B = torch.randn((batch, n, L), generator=g, device=dev)
    C = torch.randn((batch, n, L), generator=g, device=dev)
    A = -(torch.rand((dim, n), generator=g, device=dev) * 1.999 + 0.001)
    D = torch.randn(dim, generator=g, device=dev)
    y, h = selective_scan(u, d, A, B, C, D=D, z=z, return_state=True)
    b, c0, c1 = 1, 64, 192                   # 2 channel blocks: split
    sl = lambda t: t[b:b + 1, c0:c1].contiguous()
    ys, hs = selective_scan(sl(u), sl(d), A[c0:c1].contiguous(), B[b:b + 1].contiguous(),
                            C[b:b + 1].contiguous(), D=D[c0:c1].contiguous(), z=sl(z),
                            return_state=True)
    torch.cuda.synchronize()
    cpu = lambda t: t.cpu().numpy()
    yo, ho = oracle_lib.selective_scan(cpu(sl(u)), cpu(sl(d)), cpu(A[c0:c1]), cpu(B[b:b + 1]),
                                       cpu(C[b:b + 1]), D=cpu(D[c0:c1]), z=cpu(sl(z)))
    assert_close(cpu(y[b:b + 1, c0:c1]), yo, 1e-5, 1e-5, "chained y")
    assert_close(cpu(h[b:b + 1, c0:c1]), ho, 1e-5, 1e-5, "chained state")
    assert_close(cpu(ys), yo, 1e-5, 1e-5, "split y")
    assert_close(cpu(hs), ho, 1e-5, 1e-5, "split state")
    assert_close(cpu(ys), cpu(y[b:b + 1, c0:c1]), 2e-5, 2e-5, "split vs chained y")
    # the carry matters here: dropping it (a zero-state scan of the last 128 steps) is far off
    y0 = selective_scan(sl(u)[..., -128:].contiguous(), sl(d)[..., -128:].contiguous(),
                        A[c0:c1].contiguous(), B[b:b + 1, :, -128:].contiguous(),
                        C[b:b + 1, :, -128:].contiguous(), D=D[c0:c1].contiguous(),
                        z=sl(z)[..., -128:].contiguous())
    assert (y0 - ys[..., -128:]).abs().max().item() > 0.1


def test_split_lone_chain_many_segments(oracle_lib, dev):
    """The reference's benchmark shape (B=1, D=16, N=16, L=32768; one chain) splits into
    up to 256 segments, so the last segment folds 255 summaries.  Slow decay (A in
    [-2, -0.001], delta <= 0.1) keeps states alive across many segments; fp32 bar against
    the fp64 oracle, y and final state."""
    from mamba_metal_amd import selective_scan

    g = torch.Generator(device=dev)
    g.manual_seed(12)
    batch, dim, n, L = 1, 16, 16, 32768
    u = torch.randn((batch, dim, L), generator=g, device=dev)
    d = torch.rand((batch, dim, L), generator=g, device=dev) * 0.09 + 0.01
    B = torch.randn((batch, n, L), generator=g, device=dev)
    C = torch.randn((batch, n, L), generator=g, device=dev)
    A = -(torch.rand((dim, n), generator=g, device=dev) * 1.999 + 0.001)
    y, h = selective_scan(u, d, A, B, C, return_state=True)
    torch.cuda.synchronize()
    cpu = lambda t: t.cpu().numpy()
    yo, ho = oracle_lib.selective_scan(cpu(u), cpu(d), cpu(A), cpu(B), cpu(C))
    assert_close(cpu(y), yo, 1e-5, 1e-5, "lone chain y")
    assert_close(cpu(h), ho, 1e-5, 1e-5, "lone chain state")


def test_split_few_chains_full_length(oracle_lib, dev):
    """B=1, D=5120, L=32768 fp16 (80 64-channel blocks: the split path with up to 51
    segments per chain), one channel of every 16-channel block against the oracle."""
    _blockwise_parity(oracle_lib, dev, 1, 5120, 32768, seed=5)


def test_split_long_sequence_160_blocks(oracle_lib, dev):
    """B=2, D=5120, L=32768 fp16: 160 64-channel blocks take the split path only because
    the sequence is long (25 segment summaries per block), one channel of every 16-channel
    block against the oracle."""
    _blockwise_parity(oracle_lib, dev, 2, 5120, 32768, seed=6)


@pytest.mark.parametrize("dim,seqlen", [(16352, 512), (16384, 512), (24544, 384), (24576, 384)])
def test_grid_regime_boundaries(oracle_lib, dev, dim, seqlen):
    """Chain counts (32-channel blocks, batch 1) on either side of the persistent grid's
    switches on a 256-CU part: 511 / 512 chains (all resident slots / two workgroups per
    CU) and 767 / 768 (two per CU / all slots).  One channel of every block against the
    oracle."""
    _blockwise_parity(oracle_lib, dev, 1, dim, seqlen, seed=dim % 97)


def test_bf16_large_every_block(oracle_lib, dev):
    """bf16 inputs and output at B=2 D=5120 L=8192 (640 16-channel chains of one state per
    lane on 256 CUs): one channel of every block against the oracle."""
    _blockwise_parity(oracle_lib, dev, 2, 5120, 8192, seed=7, dtype=torch.bfloat16)


def test_16_channel_blocks_four_per_cu_every_block(oracle_lib, dev):
    """B=7 D=2048 L=2048 fp16 (896 16-channel chains: between 3 and 4 per CU on 256 CUs, so
    four workgroups per CU, one segment each): one channel of every block against the
    oracle."""
    _blockwise_parity(oracle_lib, dev, 7, 2048, 2048, seed=27)


def test_16_channel_blocks_full_length_every_block(oracle_lib, dev):
    """B=1 D=8704 L=8192 fp16 (544 16-channel chains of one state per lane on 256 CUs, four
    segment hand-offs each): one channel of every block against the oracle."""
    _blockwise_parity(oracle_lib, dev, 1, 8704, 8192, seed=17)


def test_config2_full_size_every_block(oracle_lib, dev):
    _blockwise_parity(oracle_lib, dev, 8, 1536, 8192, seed=2)


def test_config4_full_size_every_block(oracle_lib, dev):
    _blockwise_parity(oracle_lib, dev, 4, 5120, 32768, seed=4)


def test_edges_against_golden(dev):
    g = np.load(GOLDEN / "scan_edges.npz")
    for i, (b, d, n, L, seed) in enumerate(g["shapes"]):
        inp = features_inputs(int(b), int(d), int(n), int(L), seed=int(seed))
        y, h = gpu_scan(inp, dev, torch.float32, softplus=True)
        assert_close(y, g[f"y{i}"], 1e-5, 1e-5, f"edge {i} y")
        assert_close(h, g[f"state{i}"], 1e-5, 1e-5, f"edge {i} state")


def test_handoff_timeout_is_reported_and_bounded(dev):
    """Failure handling of the chained scan's segment hand-off, forced from the host: with
    a 1-microsecond bound (every real predecessor segment takes far longer) the waits give
    up, the kernel still exits, and the status word carries the timeout bit; the same call
    with the default bound then completes with a clear status and the oracle's result
    (one channel of every block).  640 chains of 32 channels, several segments each."""
    from mamba_metal_amd import _lib
    from mamba_metal_amd.selective_scan import (reset_scan_status, scan_status,
                                                selective_scan_into)

    import time

    batch, dim, seqlen = 4, 5120, 8192
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    f16 = torch.float16
    u = torch.randn((batch, dim, seqlen), generator=g, device=dev).to(f16)
    d = (torch.randn((batch, dim, seqlen), generator=g, device=dev) * 0.5 - 1.0).to(f16)
    B = torch.randn((batch, 16, seqlen), generator=g, device=dev).to(f16)
    C = torch.randn((batch, 16, seqlen), generator=g, device=dev).to(f16)
    A = -torch.arange(1, 17, device=dev, dtype=torch.float32).expand(dim, 16).contiguous()
    y = torch.empty_like(u)
    reset_scan_status(dev)
    t0 = time.perf_counter()
    selective_scan_into(u, d, A, B, C, y, delta_softplus=True, handoff_timeout_us=1)
    torch.cuda.synchronize()
    waited = time.perf_counter() - t0
    assert scan_status(dev) & _lib.SCAN_STATUS_HANDOFF_TIMEOUT, "forced timeout not reported"
    assert waited < 5.0, f"a timed-out call took {waited:.1f} s"
    reset_scan_status(dev)
    selective_scan_into(u, d, A, B, C, y, delta_softplus=True)
    torch.cuda.synchronize()
    assert scan_status(dev) == 0
    from oracle import cscan

    rng = np.random.default_rng(5)
    chans = np.minimum(np.arange(dim // 32) * 32 + rng.integers(0, 32, dim // 32), dim - 1)
    b = 2
    uu, dd = u[b, chans].float().cpu().numpy()[None], d[b, chans].float().cpu().numpy()[None]
    yr, _ = cscan.selective_scan(uu, dd, A[chans].cpu().numpy(), B[b:b + 1].float().cpu().numpy(),
                                 C[b:b + 1].float().cpu().numpy(), delta_softplus=True)
    assert_close(y[b, chans].float().cpu().numpy()[None], yr, 1e-3, 1e-3, "after timeout")
