"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

The reference ships no golden vectors for this path (its scan scripts print
errors against re-implemented numpy loops), so each oracle function is pinned by
checks whose answer is fixed independently of the oracle's own formula:
closed forms, library routines (torch), invariants of the recurrence, and the
agreement of two independently written restatements (C and numpy).  Each test
names the plausible mistake it would catch.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import assert_close, config0_inputs, features_inputs, plain_inputs
from oracle import numpy_ref

SCANS = ["c64", "c32", "np"]


def run_scan(kind, oracle_lib, inp, softplus, h0=None):
    args = (inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"])
    kw = dict(D=inp.get("D"), z=inp.get("z"), delta_softplus=softplus, h0=h0)
    if kind == "np":
        y, h = numpy_ref.selective_scan(*args, **kw)
        return y, h
    return oracle_lib.selective_scan(*args, precision="f64" if kind == "c64" else "f32", **kw)


def tol(kind):
    # c32: float32 arithmetic; c64: float64 arithmetic, float32 outputs (rounding
    # 6e-8 relative); np: float64 throughout.
    return {"c32": (2e-5, 2e-5), "c64": (3e-7, 1e-9), "np": (1e-9, 1e-9)}[kind]


# ---------------------------------------------------------------------------
# softplus / silu: library routines.  Catches a wrong cutoff direction or a
# log(exp) vs log1p slip.
def test_softplus_matches_torch_and_cutoff():
    x = np.array([-40.0, -20.0, -3.0, -1e-3, 0.0, 1.0, 19.9, 20.0, 20.5, 50.0])
    ref = F.softplus(torch.tensor(x, dtype=torch.float64), beta=1.0, threshold=20.0).numpy()
    assert_close(numpy_ref.softplus_safe(x), ref, 1e-14, 1e-300, "softplus_safe")
    assert numpy_ref.softplus_safe(np.array([0.0]))[0] == pytest.approx(math.log(2.0), rel=1e-15)
    assert numpy_ref.softplus_safe(np.array([25.0]))[0] == 25.0
    assert_close(numpy_ref.softplus(x), np.logaddexp(x, 0.0), 1e-15, 0, "softplus(logaddexp)")


def test_silu_matches_torch():
    x = np.linspace(-30, 30, 101)
    assert_close(numpy_ref.silu(x), F.silu(torch.tensor(x)).numpy(), 1e-14, 1e-300, "silu")
    assert numpy_ref.silu(np.array([0.0]))[0] == 0.0


# ---------------------------------------------------------------------------
# Scan closed forms.
@pytest.mark.parametrize("kind", SCANS)
def test_scan_constant_decay_closed_form(kind, oracle_lib):
    """a = exp(delta*A) constant, b = delta*u*B constant => h_t = b(1-a^(t+1))/(1-a).
    The reference's pair-scan KAT (a=0.5, b=1 -> 2) is the n=0 row.  Catches a
    wrong sign of A, exp(A) instead of exp(delta*A), or an off-by-one in t."""
    L, N = 300, 4
    avals = np.array([0.5, 0.9, 0.99, 0.999])
    bvals = np.array([1.0, 0.25, -2.0, 3.0])
    Cvals = np.array([1.0, -0.5, 0.75, 2.0])
    delta = 0.7
    A = (np.log(avals) / delta)[None, :].astype(np.float32)
    u = np.full((1, 1, L), 1.3, np.float32)
    # choose B so that delta*u*B == b exactly in float64 up to input rounding
    B = np.repeat((bvals / (delta * 1.3))[None, :, None], L, axis=2).astype(np.float32)
    C = np.repeat(Cvals[None, :, None], L, axis=2).astype(np.float32)
    dl = np.full((1, 1, L), delta, np.float32)
    y, h = run_scan(kind, oracle_lib, dict(u=u, delta=dl, A=A, B=B, C=C), False)
    a = np.exp(np.float64(np.float32(delta)) * A[0].astype(np.float64))
    b = np.float64(np.float32(delta)) * np.float64(np.float32(1.3)) * B[0, :, 0].astype(np.float64)
    t = np.arange(L)[:, None]
    h_cf = b * (1 - a ** (t + 1)) / (1 - a)
    y_cf = h_cf @ C[0, :, 0].astype(np.float64)
    rt, at = tol(kind)
    assert_close(y[0, 0], y_cf, rt * 10, at * 10, f"{kind} y closed form")
    assert_close(h[0, 0], h_cf[-1], rt * 10, at * 10, f"{kind} state closed form")
    # the reference's pair-scan KAT: a = 0.5, b = 1 converges to b / (1 - a) = 2
    assert abs(h[0, 0, 0] - 2.0) < 1e-5


@pytest.mark.parametrize("kind", SCANS)
def test_scan_zero_A_is_cumsum(kind, oracle_lib):
    """A = 0 => a = 1 => h_t = cumsum(delta*u*B) (block-scan KAT = cumsum).
    Catches dropping delta or u from the input term."""
    inp = plain_inputs(2, 3, 5, 200, seed=3)
    inp["A"] = np.zeros_like(inp["A"])
    y, h = run_scan(kind, oracle_lib, inp, False)
    d, u, B, C = (inp[k].astype(np.float64) for k in ("delta", "u", "B", "C"))
    hc = np.cumsum((d * u)[:, :, None, :] * B[:, None, :, :], axis=-1)   # (b, d, n, t)
    y_cf = np.einsum("bdnt,bnt->bdt", hc, C)
    rt, at = tol(kind)
    assert_close(y, y_cf, rt * 20, at * 20, f"{kind} cumsum")
    assert_close(h, hc[..., -1], rt * 20, at * 20, f"{kind} cumsum state")


@pytest.mark.parametrize("kind", SCANS)
def test_scan_single_step_and_features(kind, oracle_lib):
    """L = 1 => h = delta'*u*B; y = (<h, C> + D*u) * silu(z), delta' = softplus(delta).
    Catches D / z applied in the wrong order or softplus skipped."""
    inp = features_inputs(2, 5, 7, 1, seed=5)
    y, h = run_scan(kind, oracle_lib, inp, True)
    d = np.log1p(np.exp(inp["delta"].astype(np.float64)))
    hh = (d * inp["u"])[:, :, None, 0] * inp["B"][:, None, :, 0]
    core = np.einsum("bdn,bn->bd", hh, inp["C"][:, :, 0].astype(np.float64))
    zz = inp["z"][:, :, 0].astype(np.float64)
    Du = inp["D"][None, :].astype(np.float64) * inp["u"][:, :, 0].astype(np.float64)
    y_cf = (core + Du) * zz / (1 + np.exp(-zz))
    rt, at = tol(kind)
    assert_close(y[:, :, 0], y_cf, rt, at, f"{kind} L=1")
    assert_close(h, hh, rt, at, f"{kind} L=1 state")


@pytest.mark.parametrize("kind", SCANS)
def test_scan_zero_delta_is_skip_only(kind, oracle_lib):
    """delta = 0 (no softplus) => a = 1, b = 0 => y = D*u*silu(z), state 0."""
    inp = features_inputs(1, 4, 16, 64, seed=6)
    inp["delta"] = np.zeros_like(inp["delta"])
    y, h = run_scan(kind, oracle_lib, inp, False)
    zz = inp["z"].astype(np.float64)
    y_cf = inp["D"][None, :, None] * inp["u"] * zz / (1 + np.exp(-zz))
    assert_close(y, y_cf, 1e-6, 1e-7, f"{kind} delta=0")
    assert np.all(h == 0)


# ---------------------------------------------------------------------------
# Invariants.
@pytest.mark.parametrize("kind", SCANS)
def test_state_equals_h_read_through_onehot_C(kind, oracle_lib):
    """state_out == h[L-1]: reading h through C = e_n at the last step gives the
    state (verify_state_out.py semantics) via the y path, an independent route.
    Catches writing h before the last update or the wrong state index."""
    inp = plain_inputs(1, 3, 4, 97, seed=7)
    _, h = run_scan(kind, oracle_lib, inp, False)
    for n in range(4):
        C = inp["C"].copy()
        C[:, :, -1] = 0.0
        C[:, n, -1] = 1.0
        y, _ = run_scan(kind, oracle_lib, dict(inp, C=C), False)
        rt, at = tol(kind)
        assert_close(y[:, :, -1], h[:, :, n], rt, at, f"{kind} onehot n={n}")


@pytest.mark.parametrize("kind", SCANS)
def test_scan_concatenation(kind, oracle_lib):
    """scan(x1 ++ x2) == (scan(x1), scan(x2, h0=state(x1))): the recurrence is a
    pure state machine.  Catches any dependence on absolute position."""
    inp = features_inputs(2, 3, 8, 150, seed=8)
    y, h = run_scan(kind, oracle_lib, inp, True)
    k = 61
    cut = lambda s: {key: (v[..., s] if (v is not None and key in ("u", "delta", "B", "C", "z")) else v)
                     for key, v in inp.items()}
    y1, h1 = run_scan(kind, oracle_lib, cut(slice(0, k)), True)
    h0 = h1 if kind == "np" else np.asarray(h1, np.float32)  # C oracle takes float32 state
    y2, h2 = run_scan(kind, oracle_lib, cut(slice(k, None)), True, h0=h0)
    rt, at = tol(kind)
    assert_close(y1, y[..., :k], rt, at, f"{kind} first half")
    assert_close(y2, y[..., k:], rt * 5, at * 5, f"{kind} second half")
    assert_close(h2, h, rt * 5, at * 5, f"{kind} state")


@pytest.mark.parametrize("kind", ["c64", "np"])
def test_scan_linear_in_u(kind, oracle_lib):
    """With delta fixed (no softplus), z off: y(a*u1 + b*u2) = a*y(u1) + b*y(u2).
    Catches a u-dependence in the decay or a squared u."""
    inp = features_inputs(1, 4, 6, 80, seed=9)
    inp["delta"] = np.abs(inp["delta"])
    inp["z"] = None
    u1 = inp["u"]
    u2 = np.random.default_rng(10).standard_normal(u1.shape).astype(np.float32)
    ya, _ = run_scan(kind, oracle_lib, dict(inp, u=u1), False)
    yb, _ = run_scan(kind, oracle_lib, dict(inp, u=u2), False)
    yc, _ = run_scan(kind, oracle_lib, dict(inp, u=(2.0 * u1 - 0.5 * u2).astype(np.float32)), False)
    assert_close(yc, 2.0 * ya - 0.5 * yb, 1e-6, 1e-6, f"{kind} linearity")


def test_c_and_numpy_restatements_agree(oracle_lib):
    """Two independently written restatements agree (float64) on the BASELINE
    config-0 distribution and on the feature matrix inputs."""
    for inp, sp in ((config0_inputs(1, 4, 16, 1000, seed=1), True),
                    (features_inputs(2, 3, 16, 700, seed=2), True),
                    (plain_inputs(1, 2, 8, 1025, seed=3), False)):
        yc, hc = run_scan("c64", oracle_lib, inp, sp)
        yn, hn = run_scan("np", oracle_lib, inp, sp)
        assert_close(yc, yn, 1e-6, 1e-6, "c64 vs numpy y")   # c64 stores float32 outputs
        assert_close(hc, hn, 1e-6, 1e-6, "c64 vs numpy h")
        y32, h32 = run_scan("c32", oracle_lib, inp, sp)
        assert_close(y32, yn, 1e-4, 1e-4, "c32 vs numpy y")


def test_channel_range_sampling(oracle_lib):
    """channels=(c0, c1) computes exactly those flattened channels (used to time a
    bounded sample of a large workload) and leaves the rest zero."""
    inp = config0_inputs(2, 5, 16, 64, seed=4)
    y, h = oracle_lib.selective_scan(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"],
                                     D=inp["D"], z=inp["z"], delta_softplus=True)
    ys, hs = oracle_lib.selective_scan(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"],
                                       D=inp["D"], z=inp["z"], delta_softplus=True, channels=(3, 7))
    yf, yfs = y.reshape(10, 64), ys.reshape(10, 64)
    assert np.array_equal(yfs[3:7], yf[3:7])
    assert np.all(yfs[:3] == 0) and np.all(yfs[7:] == 0)


# ---------------------------------------------------------------------------
# Pair scan.
def test_pair_scan_known_answers(oracle_lib):
    n = 1024
    a = np.full(n, 0.5, np.float32)
    b = np.ones(n, np.float32)
    i = np.arange(n)
    for fn in (numpy_ref.pair_scan, oracle_lib.pair_scan):
        pa, h = fn(a, b)
        assert_close(h, 2.0 * (1.0 - 0.5 ** (i + 1)), 1e-6, 1e-30, "a=0.5,b=1")
        assert abs(h[-1] - 2.0) < 1e-6
        assert_close(pa, 0.5 ** (i + 1), 1e-6, 1e-45, "prod a")
    rng = np.random.default_rng(0)
    bb = rng.standard_normal(333).astype(np.float32)
    for fn in (numpy_ref.pair_scan, oracle_lib.pair_scan):
        _, h = fn(np.ones(333, np.float32), bb)
        assert_close(h, np.cumsum(bb.astype(np.float64)), 1e-6, 1e-5, "a=1 cumsum")


# ---------------------------------------------------------------------------
# Conv1d and the decode steps.
def test_causal_conv1d_matches_torch_and_impulse():
    rng = np.random.default_rng(11)
    for (b, L, D, K) in ((2, 37, 5, 4), (1, 3, 4, 4), (1, 9, 3, 2)):
        x = rng.standard_normal((b, L, D))
        w = rng.standard_normal((D, K))
        bias = rng.standard_normal(D)
        out, st = numpy_ref.causal_conv1d(x, w, bias, apply_silu=False)
        ref = F.conv1d(torch.tensor(x).transpose(1, 2), torch.tensor(w)[:, None, :],
                       torch.tensor(bias), padding=K - 1, groups=D)[..., :L].transpose(1, 2)
        assert_close(out, ref.numpy(), 1e-12, 1e-12, "conv vs torch")
        outs, _ = numpy_ref.causal_conv1d(x, w, bias, apply_silu=True)
        assert_close(outs, F.silu(ref).numpy(), 1e-12, 1e-12, "conv+silu vs torch")
        xp = np.concatenate([np.zeros((b, K, D)), x], 1)
        assert_close(st, np.transpose(xp[:, -K:, :], (0, 2, 1)), 0, 0, "conv state")
    # impulse: x = e_{t0} => out[t0 + j] = w[K-1-j]  (cross-correlation, no flip)
    x = np.zeros((1, 10, 1)); x[0, 3, 0] = 1.0
    w = np.array([[1.0, 2.0, 3.0, 4.0]])
    out, _ = numpy_ref.causal_conv1d(x, w, None, apply_silu=False)
    assert list(out[0, 3:7, 0]) == [4.0, 3.0, 2.0, 1.0]
    # state for L < K is left zero-padded: [0, x0, x1, x2] for K=4, L=3
    x = np.arange(1, 4, dtype=np.float64).reshape(1, 3, 1)
    _, st = numpy_ref.causal_conv1d(x, np.ones((1, 4)), None)
    assert list(st[0, 0]) == [0.0, 1.0, 2.0, 3.0]


def test_decode_conv_step_equals_prefill_last_position():
    rng = np.random.default_rng(12)
    b, L, D, K = 2, 11, 6, 4
    x = rng.standard_normal((b, L + 1, D))
    w = rng.standard_normal((D, K))
    bias = rng.standard_normal(D)
    _, st = numpy_ref.causal_conv1d(x[:, :L], w, bias)
    full, st_full = numpy_ref.causal_conv1d(x, w, bias)
    out, st2 = numpy_ref.decode_conv_step(st, x[:, L], w, bias)
    assert_close(out, full[:, L], 1e-12, 1e-12, "conv step")
    assert_close(st2, st_full, 0, 0, "conv step state")


def test_decode_ssm_step_equals_scan_one_step(oracle_lib):
    inp = features_inputs(3, 5, 16, 1, seed=13)
    h0 = np.random.default_rng(14).standard_normal((3, 5, 16)).astype(np.float32)
    y, h = numpy_ref.decode_ssm_step(h0, inp["u"][..., 0], inp["delta"][..., 0], inp["A"],
                                     inp["B"][..., 0], inp["C"][..., 0], D=inp["D"],
                                     z=inp["z"][..., 0])
    ys, hs = oracle_lib.selective_scan(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"],
                                       D=inp["D"], z=inp["z"], delta_softplus=True, h0=h0)
    assert_close(y, ys[..., 0], 1e-6, 1e-6, "ssm step y")
    assert_close(h, hs, 1e-6, 1e-6, "ssm step h")


def test_rms_norm_matches_torch():
    rng = np.random.default_rng(15)
    x = rng.standard_normal((3, 7, 32))
    w = rng.standard_normal(32)
    ref = F.rms_norm(torch.tensor(x), (32,), torch.tensor(w), eps=1e-5).numpy()
    assert_close(numpy_ref.rms_norm(x, w), ref, 1e-12, 1e-12, "rms_norm")
