"""numpy restatement of the selective-scan inference path -- TEST INFRASTRUCTURE ONLY.

Written independently of ``scan_ref.c`` (vectorised over (batch, dim, dstate),
loop over time) so the two restatements check each other.  Every function cites
the reference code it restates; tests/test_oracle.py pins each one against
closed forms, invariants or a library routine:

  softplus_safe       selective_scan_chunked.metal:60-65, test_features.py:13-16
                      -- pinned: log(2) at 0, identity above 20, torch.nn.functional.softplus
  silu                test_features.py:19-20 -- pinned: torch.nn.functional.silu, silu(0)=0
  selective_scan      test_features.py:23-43, test_fp16.py:147-174, verify_state_out.py:13-26
                      -- pinned: closed forms (constant a,b; A=0 cumsum; L=1), linearity in u,
                         concatenation with h0, C one-hot == state, agreement with scan_ref.c
  pair_scan           pair_scan.metal:24-76, experiments/05-pair-scan/pair_scan.py:36-42
                      -- pinned: a=0.5,b=1 -> 2(1-0.5^(i+1)); a=1 -> cumsum
  causal_conv1d       mamba_block.py:45-52,72-78,115-130 (nn.Conv1d padding K-1, slice [:L])
                      -- pinned: torch.nn.functional.conv1d, impulse response
  decode_conv_step    mamba_block.py:170-177 -- pinned: equals causal_conv1d at the last position
  decode_ssm_step     mamba_block.py:183-195 -- pinned: equals selective_scan one step from h0
  rms_norm            mlx nn.RMSNorm used at mamba_model.py:40,69 -- pinned: torch rms_norm
"""

from __future__ import annotations

import numpy as np


def softplus_safe(x):
    """log(1 + exp(x)) for x <= 20, else x (the kernel's cutoff)."""
    x = np.asarray(x, dtype=np.float64)
    return np.where(x <= 20.0, np.log1p(np.exp(np.minimum(x, 20.0))), x)


def softplus(x):
    """MLX nn.softplus (logaddexp(x, 0)) used by MambaBlock.step (mamba_block.py:184)."""
    x = np.asarray(x, dtype=np.float64)
    return np.logaddexp(x, 0.0)


def silu(x):
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def selective_scan(u, delta, A, B, C, D=None, z=None, delta_softplus=False, h0=None):
    """Sequential scan in float64.  Shapes as mamba_metal/selective_scan.py:36-44.

    Returns (y (batch, dim, seqlen), state (batch, dim, dstate)), float64.
    """
    u = np.asarray(u, np.float64)
    delta = np.asarray(delta, np.float64)
    A = np.asarray(A, np.float64)
    B = np.asarray(B, np.float64)
    C = np.asarray(C, np.float64)
    batch, dim, seqlen = u.shape
    dstate = A.shape[1]
    if delta_softplus:
        delta = softplus_safe(delta)
    h = np.zeros((batch, dim, dstate)) if h0 is None else np.array(h0, np.float64)
    y = np.empty((batch, dim, seqlen))
    for t in range(seqlen):
        dt = delta[:, :, t][:, :, None]                       # (b, d, 1)
        a = np.exp(dt * A[None])                              # (b, d, n)
        bx = (dt * u[:, :, t][:, :, None]) * B[:, None, :, t]  # (b, d, n)
        h = a * h + bx
        y[:, :, t] = np.einsum("bdn,bn->bd", h, C[:, :, t])
    if D is not None:
        y = y + np.asarray(D, np.float64)[None, :, None] * u
    if z is not None:
        y = y * silu(z)
    return y, h


def pair_scan(a, b):
    """Inclusive scan of (a, b) pairs; returns (prod a, h)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    pa = np.cumprod(a)
    h = np.empty_like(b)
    acc = 0.0
    for i in range(a.size):
        acc = a[i] * acc + b[i]
        h[i] = acc
    return pa, h


def causal_conv1d(x, w, bias=None, apply_silu=True):
    """Causal depthwise conv over time for channels-last x (batch, L, D).

    w: (D, K) taps (torch/HF weight (D, 1, K) squeezed), oldest tap first.
    Returns (out (batch, L, D), conv_state (batch, D, K)) where conv_state holds the
    last K pre-conv inputs, left zero-padded when L < K (mamba_block.py:118-127).
    """
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    batch, L, D = x.shape
    K = w.shape[1]
    xp = np.concatenate([np.zeros((batch, K - 1, D)), x], axis=1)
    out = np.zeros((batch, L, D))
    for k in range(K):
        out += w[None, None, :, k] * xp[:, k:k + L, :]
    if bias is not None:
        out += np.asarray(bias, np.float64)[None, None, :]
    if apply_silu:
        out = silu(out)
    conv_state = np.transpose(xp[:, L - 1:L - 1 + K, :] if L >= 1 else xp[:, :K, :], (0, 2, 1))
    return out, np.ascontiguousarray(conv_state)


def decode_conv_step(conv_state, x, w, bias=None, apply_silu=True):
    """One decode step of the conv window (mamba_block.py:170-177).

    conv_state (batch, D, K) oldest->newest, x (batch, D).
    Returns (out (batch, D), new_conv_state)."""
    conv_state = np.asarray(conv_state, np.float64)
    new = np.concatenate([conv_state[:, :, 1:], np.asarray(x, np.float64)[:, :, None]], axis=2)
    out = (new * np.asarray(w, np.float64)[None]).sum(-1)
    if bias is not None:
        out = out + np.asarray(bias, np.float64)[None]
    if apply_silu:
        out = silu(out)
    return out, new


def decode_ssm_step(h, x, dt, A, B, C, D=None, z=None, dt_bias=None, dt_softplus=True):
    """One decode step of the SSM (mamba_block.py:183-195).

    h (batch, D, N), x/dt/z (batch, D), B/C (batch, N), A (D, N).
    dt is the dt_proj output; softplus is MLX's logaddexp form (no cutoff).
    Returns (y (batch, D), new_h)."""
    h = np.asarray(h, np.float64)
    x = np.asarray(x, np.float64)
    dt = np.asarray(dt, np.float64)
    if dt_bias is not None:
        dt = dt + np.asarray(dt_bias, np.float64)[None]
    if dt_softplus:
        dt = softplus(dt)
    A = np.asarray(A, np.float64)
    a = np.exp(dt[:, :, None] * A[None])
    bx = (dt * x)[:, :, None] * np.asarray(B, np.float64)[:, None, :]
    h = a * h + bx
    y = (h * np.asarray(C, np.float64)[:, None, :]).sum(-1)
    if D is not None:
        y = y + np.asarray(D, np.float64)[None] * x
    if z is not None:
        y = y * silu(z)
    return y, h


def rms_norm(x, weight, eps=1e-5):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(weight, np.float64)
