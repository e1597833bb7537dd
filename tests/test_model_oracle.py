"""Pins the CPU model oracle (oracle/model_ref.RefModel) before it is trusted.

RefModel carries every model-level parity test (prefill logits, decode steps, greedy
ids), so it is checked here on its own, on the CPU, against answers that do not come
from its own composition:

  * closed forms of the whole model and of one block in special cases whose result
    another formulation gives (a zero mixer; B = C = 0; A = 0, where the recurrence is
    a cumulative sum), each built from numpy / torch library routines;
  * the reference's own invariants evaluated on RefModel itself:
      prefill(L) then step(x_L) == prefill(L + 1) at position L
          (experiments/17-incremental/test_step.py:31-41),
      causality (experiments/11-mamba-block/test_block.py:42-61),
      conv-state left padding for L < d_conv (mamba_metal/mamba_block.py:118-127).

Each test names the composition mistake it would catch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import assert_close
from oracle.model_ref import RefConfig, RefModel


def random_weights(cfg: RefConfig, seed: int, A_log=None) -> dict:
    """HF-named weights (``backbone.`` stripped) with non-trivial norm weights, D and
    biases, so that a norm applied without its weight or a dropped bias shows."""
    rng = np.random.default_rng(seed)
    di, n, r, K, dm = cfg.d_inner, cfg.d_state, cfg.dt_rank, cfg.d_conv, cfg.d_model
    g = lambda *s, sd=0.2: rng.standard_normal(s) * sd
    w = {"embeddings.weight": g(cfg.vocab_size, dm, sd=1.0),
         "norm_f.weight": 1.0 + g(dm, sd=0.3)}
    for i in range(cfg.n_layer):
        p = f"layers.{i}."
        dt = rng.uniform(1e-3, 1e-1, di)
        w.update({
            p + "norm.weight": 1.0 + g(dm, sd=0.3),
            p + "mixer.in_proj.weight": g(2 * di, dm),
            p + "mixer.conv1d.weight": g(di, 1, K, sd=0.5),
            p + "mixer.conv1d.bias": g(di, sd=0.1),
            p + "mixer.x_proj.weight": g(r + 2 * n, di),
            p + "mixer.dt_proj.weight": g(di, r),
            p + "mixer.dt_proj.bias": np.log(np.expm1(dt)),
            p + "mixer.A_log": (np.log(np.broadcast_to(np.arange(1, n + 1, dtype=np.float64), (di, n)))
                                if A_log is None else np.full((di, n), A_log)),
            p + "mixer.D": 1.0 + g(di, sd=0.5),
            p + "mixer.out_proj.weight": g(dm, di),
        })
    return {k: np.array(v, dtype=np.float64) for k, v in w.items()}


CFG = dict(d_model=16, n_layer=2, vocab_size=40, d_state=4, d_conv=4, expand=2)


def make(seed=0, **over):
    cfg = RefConfig(**{**CFG, **over})
    return cfg, random_weights(cfg, seed)


def rms_np(x, w, eps):
    """RMSNorm through the Euclidean norm: x * sqrt(d) / ||x|| (with eps) * w."""
    d = x.shape[-1]
    nrm = np.linalg.norm(x, axis=-1, keepdims=True)
    return x / np.sqrt(nrm ** 2 / d + eps) * w


def silu_t(x):
    return F.silu(torch.as_tensor(x)).numpy()


# ---------------------------------------------------------------------------
# Whole model, zero mixer: every residual block returns its input, so
# logits = RMSNorm_f(E[ids]) @ E^T.  Catches a residual that drops x, the final norm
# applied without norm_f.weight (or with a layer's), an untied head or E^T / E confusion.
def test_zero_mixer_closed_form():
    cfg, w = make(seed=1)
    for i in range(cfg.n_layer):
        w[f"layers.{i}.mixer.out_proj.weight"][:] = 0.0
    ref = RefModel(cfg, w)
    ids = np.random.default_rng(1).integers(0, cfg.vocab_size, (2, 9))
    E = w["embeddings.weight"]
    want = rms_np(E[ids], w["norm_f.weight"], cfg.rms_norm_eps) @ E.T
    got, convs, ssms = ref.prefill(ids)
    assert_close(got.numpy(), want, 1e-12, 1e-12, "prefill logits")
    got_last, _, _ = ref.prefill(ids, last_only=True)
    assert_close(got_last.numpy(), want[:, -1:], 1e-12, 1e-12, "last-only logits")
    tok = np.array([3, 17])
    st, _, _ = ref.step(tok, convs, ssms)
    want_st = rms_np(E[tok], w["norm_f.weight"], cfg.rms_norm_eps) @ E.T
    assert_close(st[:, 0].numpy(), want_st, 1e-12, 1e-12, "step logits")


# ---------------------------------------------------------------------------
# One block with B = C = 0 (the x_proj rows of B and C zeroed): the state contributes
# nothing and the block is out_proj(D * silu(conv(x)) * silu(z)), with the conv taken
# by torch's conv1d.  Catches x / z swapped in the in_proj split, a flipped or
# mis-padded conv, a missing conv bias, D or gate, B/C taken from the dt slice.
def _block_no_state(w, cfg, i, x):
    di = cfg.d_inner
    xz = x @ w[f"layers.{i}.mixer.in_proj.weight"].T
    xpre, z = xz[..., :di], xz[..., di:]
    L = x.shape[1]
    conv = F.conv1d(torch.as_tensor(xpre).transpose(1, 2), torch.as_tensor(w[f"layers.{i}.mixer.conv1d.weight"]),
                    torch.as_tensor(w[f"layers.{i}.mixer.conv1d.bias"]), padding=cfg.d_conv - 1,
                    groups=di)[..., :L].transpose(1, 2).numpy()
    y = w[f"layers.{i}.mixer.D"] * silu_t(conv) * silu_t(z)
    return y @ w[f"layers.{i}.mixer.out_proj.weight"].T


def test_block_zero_BC_closed_form():
    cfg, w = make(seed=2, n_layer=1)
    r, n = cfg.dt_rank, cfg.d_state
    w["layers.0.mixer.x_proj.weight"][r:r + 2 * n] = 0.0
    ref = RefModel(cfg, w)
    x = np.random.default_rng(2).standard_normal((2, 11, cfg.d_model))
    out, conv_state, ssm_state = ref._mixer_prefill(0, torch.as_tensor(x))
    assert_close(out.numpy(), _block_no_state(w, cfg, 0, x), 1e-12, 1e-12, "prefill block")
    assert np.all(ssm_state.numpy() == 0.0)
    # the decode step: same closed form at the next position
    xs = np.random.default_rng(3).standard_normal((2, cfg.d_model))
    out_s, _, _ = ref._mixer_step(0, torch.as_tensor(xs), conv_state, ssm_state)
    full = _block_no_state(w, cfg, 0, np.concatenate([x, xs[:, None]], 1))
    assert_close(out_s.numpy(), full[:, -1], 1e-12, 1e-12, "step block")


# ---------------------------------------------------------------------------
# One block with A = 0: exp(dt * A) = 1, so h_t = cumsum_s(dt_s * x_s * B_s) and
# y_t = sum_n C_t h_t + D x_t, times silu(z) -- a cumulative sum in place of the
# recurrence.  Catches B and C swapped, dt taken from the wrong slice of x_proj, the
# dt bias or softplus dropped, state written from the wrong step.
def _block_A0(w, cfg, x):
    di, r, n = cfg.d_inner, cfg.dt_rank, cfg.d_state
    xz = x @ w["layers.0.mixer.in_proj.weight"].T
    xpre, z = xz[..., :di], xz[..., di:]
    L = x.shape[1]
    conv = F.conv1d(torch.as_tensor(xpre).transpose(1, 2), torch.as_tensor(w["layers.0.mixer.conv1d.weight"]),
                    torch.as_tensor(w["layers.0.mixer.conv1d.bias"]), padding=cfg.d_conv - 1,
                    groups=di)[..., :L].transpose(1, 2).numpy()
    xc = silu_t(conv)                                                # (b, L, di)
    xdbl = xc @ w["layers.0.mixer.x_proj.weight"].T
    dt = F.softplus(torch.as_tensor(xdbl[..., :r] @ w["layers.0.mixer.dt_proj.weight"].T
                                    + w["layers.0.mixer.dt_proj.bias"])).numpy()
    Bm, Cm = xdbl[..., r:r + n], xdbl[..., r + n:]
    h = np.cumsum((dt * xc)[..., None] * Bm[:, :, None, :], axis=1)  # (b, L, di, n)
    y = np.einsum("bldn,bln->bld", h, Cm) + w["layers.0.mixer.D"] * xc
    y = y * silu_t(z)
    return y @ w["layers.0.mixer.out_proj.weight"].T, h[:, -1]


def test_block_zero_A_cumsum_closed_form():
    cfg = RefConfig(**{**CFG, "n_layer": 1})
    w = random_weights(cfg, 4, A_log=-1e4)          # A = -exp(-1e4) = -0
    ref = RefModel(cfg, w)
    x = np.random.default_rng(4).standard_normal((2, 13, cfg.d_model))
    want, h_last = _block_A0(w, cfg, x)
    out, conv_state, ssm_state = ref._mixer_prefill(0, torch.as_tensor(x))
    assert_close(out.numpy(), want, 1e-10, 1e-10, "prefill block (A = 0)")
    assert_close(ssm_state.numpy(), h_last, 1e-10, 1e-10, "final state (A = 0)")
    xs = np.random.default_rng(5).standard_normal((2, cfg.d_model))
    out_s, _, h_s = ref._mixer_step(0, torch.as_tensor(xs), conv_state, ssm_state)
    want_s, h_last_s = _block_A0(w, cfg, np.concatenate([x, xs[:, None]], 1))
    assert_close(out_s.numpy(), want_s[:, -1], 1e-10, 1e-10, "step block (A = 0)")
    assert_close(h_s.numpy(), h_last_s, 1e-10, 1e-10, "step state (A = 0)")


# ---------------------------------------------------------------------------
# The reference's invariants on RefModel itself.
@pytest.mark.parametrize("L", [1, 2, 3, 4, 5, 17])
def test_prefill_then_step_equals_longer_prefill(L):
    """prefill(L) + step == prefill(L + 1) at position L, then four more steps.  Covers
    L < d_conv (the left-padded conv state).  Catches a conv window shifted the wrong
    way, a state handed over from the wrong step, prefill/step softplus that disagree."""
    cfg, w = make(seed=10 + L)
    ref = RefModel(cfg, w)
    ids = np.random.default_rng(L).integers(0, cfg.vocab_size, (3, L + 5))
    full = ref.forward(ids).numpy()
    _, convs, ssms = ref.prefill(ids[:, :L])
    for t in range(L, L + 5):
        lg, convs, ssms = ref.step(ids[:, t], convs, ssms)
        assert_close(lg[:, 0].numpy(), full[:, t], 1e-10, 1e-10, f"step at {t}")


def test_conv_state_left_padding():
    """L < d_conv: the conv state is the pre-conv input left-padded with zeros
    (mamba_block.py:118-127); L >= d_conv: its last d_conv rows."""
    cfg, w = make(seed=20, n_layer=1)
    ref = RefModel(cfg, w)
    for L in (1, 2, 4, 7):
        x = np.random.default_rng(L).standard_normal((2, L, cfg.d_model))
        _, cs, _ = ref._mixer_prefill(0, torch.as_tensor(x))
        xpre = (x @ w["layers.0.mixer.in_proj.weight"].T)[..., :cfg.d_inner]
        want = np.zeros((2, cfg.d_inner, cfg.d_conv))
        k = min(L, cfg.d_conv)
        want[:, :, cfg.d_conv - k:] = xpre[:, L - k:].transpose(0, 2, 1)
        assert_close(cs.numpy(), want, 1e-12, 1e-12, f"conv state L={L}")


def test_causality():
    """experiments/11-mamba-block/test_block.py:42-61 on RefModel: logits before k do not
    depend on tokens from k on; logits from k on do."""
    cfg, w = make(seed=30)
    ref = RefModel(cfg, w)
    rng = np.random.default_rng(30)
    ids1 = rng.integers(0, cfg.vocab_size, (1, 24))
    ids2 = ids1.copy()
    ids2[:, 12:] = (ids1[:, 12:] + 1 + rng.integers(0, cfg.vocab_size - 1, (1, 12))) % cfg.vocab_size
    a, b = ref.forward(ids1).numpy(), ref.forward(ids2).numpy()
    assert np.max(np.abs(a[:, :12] - b[:, :12])) == 0.0
    assert np.max(np.abs(a[:, 12:] - b[:, 12:])) > 1e-3


def test_generate_fast_ids_is_argmax_of_steps():
    """Greedy ids are the argmax of each step's logits, and each step is fed the
    previous id (generate.py:89-107)."""
    cfg, w = make(seed=40)
    ref = RefModel(cfg, w)
    ids = np.random.default_rng(40).integers(0, cfg.vocab_size, (2, 6))
    toks, logits = ref.generate_fast_ids(ids, 5)
    seq = ids
    for s in range(5):
        nxt = ref.forward(seq).numpy()[:, -1]
        assert_close(logits[s].numpy(), nxt, 1e-10, 1e-10, f"logits {s}")
        assert np.array_equal(toks[:, s].numpy(), nxt.argmax(-1))
        seq = np.concatenate([seq, nxt.argmax(-1)[:, None]], 1)
