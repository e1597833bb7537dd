"""Seeded input generators shared by the tests and the golden-fixture script.

Distributions follow the reference's test scripts and BASELINE configs:
  - ``config0_inputs``: BASELINE config 0 -- u, B, C, z ~ N(0,1); delta_raw ~ N(-1, 0.5)
    (softplus on); A[d,n] = -(n+1); D = 1.
  - ``features_inputs``: experiments/09-features/test_features.py:46-56 -- delta ~ U(-1, 2),
    A = -U(0.1, 2), D, z ~ N(0,1) (seeded with a fixed seed, not the reference's
    per-process ``hash(name)``, test_features.py:60).
  - ``fp16_inputs``: experiments/10-fp16/test_fp16.py:177-186 -- u, B, C ~ 0.5 N(0,1),
    delta ~ U(0.01, 0.1).
  - ``plain_inputs``: experiments/07-chunked/selective_scan_chunked.py:114-120.
"""

from __future__ import annotations

import numpy as np


def config0_inputs(batch=1, dim=16, dstate=16, seqlen=4096, seed=0):
    rng = np.random.default_rng(seed)
    u = rng.standard_normal((batch, dim, seqlen)).astype(np.float32)
    delta = rng.normal(-1.0, 0.5, size=(batch, dim, seqlen)).astype(np.float32)
    B = rng.standard_normal((batch, dstate, seqlen)).astype(np.float32)
    C = rng.standard_normal((batch, dstate, seqlen)).astype(np.float32)
    z = rng.standard_normal((batch, dim, seqlen)).astype(np.float32)
    A = -np.broadcast_to(np.arange(1, dstate + 1, dtype=np.float32), (dim, dstate)).copy()
    D = np.ones(dim, np.float32)
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z)


def features_inputs(batch, dim, dstate, seqlen, seed=0):
    rng = np.random.default_rng(seed)
    u = rng.standard_normal((batch, dim, seqlen)).astype(np.float32)
    delta = rng.uniform(-1.0, 2.0, size=(batch, dim, seqlen)).astype(np.float32)
    A = -rng.uniform(0.1, 2.0, size=(dim, dstate)).astype(np.float32)
    B = rng.standard_normal((batch, dstate, seqlen)).astype(np.float32)
    C = rng.standard_normal((batch, dstate, seqlen)).astype(np.float32)
    D = rng.standard_normal((dim,)).astype(np.float32)
    z = rng.standard_normal((batch, dim, seqlen)).astype(np.float32)
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z)


def fp16_inputs(batch, dim, dstate, seqlen, seed=0):
    rng = np.random.default_rng(seed)
    u = rng.standard_normal((batch, dim, seqlen)).astype(np.float32) * 0.5
    delta = rng.uniform(0.01, 0.1, size=(batch, dim, seqlen)).astype(np.float32)
    A = -rng.uniform(0.1, 2.0, size=(dim, dstate)).astype(np.float32)
    B = rng.standard_normal((batch, dstate, seqlen)).astype(np.float32) * 0.5
    C = rng.standard_normal((batch, dstate, seqlen)).astype(np.float32) * 0.5
    D = rng.standard_normal((dim,)).astype(np.float32)
    z = rng.standard_normal((batch, dim, seqlen)).astype(np.float32)
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=D, z=z)


def plain_inputs(batch, dim, dstate, seqlen, seed=0):
    rng = np.random.default_rng(seed)
    u = rng.standard_normal((batch, dim, seqlen)).astype(np.float32)
    delta = rng.uniform(0.01, 0.1, size=(batch, dim, seqlen)).astype(np.float32)
    A = -rng.uniform(0.1, 2.0, size=(dim, dstate)).astype(np.float32)
    B = rng.standard_normal((batch, dstate, seqlen)).astype(np.float32)
    C = rng.standard_normal((batch, dstate, seqlen)).astype(np.float32)
    return dict(u=u, delta=delta, A=A, B=B, C=C, D=None, z=None)


def round_fp16(arrs, keys=("u", "delta", "B", "C", "z")):
    """fp16-round the activation inputs (what the GPU sees) but keep float32 arrays."""
    out = dict(arrs)
    for k in keys:
        if out.get(k) is not None:
            out[k] = out[k].astype(np.float16).astype(np.float32)
    return out


def assert_close(actual, expected, rtol, atol, what=""):
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    assert actual.shape == expected.shape, f"{what}: shape {actual.shape} != {expected.shape}"
    err = np.abs(actual - expected)
    tol = atol + rtol * np.abs(expected)
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} elements outside rtol={rtol} atol={atol}; "
            f"worst at {i}: got {actual[i]!r} expected {expected[i]!r} (max abs err {err.max():.3e})")


def check_greedy(got, gpu_logits, ref_logits, n, what, max_exempt_frac=0.05, tol=2e-2):
    """Teacher-forced logits within fp16 tolerance, and the GPU's greedy id equal to the
    oracle's argmax at every step where the oracle's top-2 margin exceeds twice the
    measured logit error of this run (there no error of that size can flip the argmax;
    below it a flip is possible and the step is counted as exempt, not hidden)."""
    errs = [float(np.abs(gpu_logits[s].cpu().numpy() - ref_logits[s].numpy()).max()) for s in range(n)]
    err = max(errs)
    exempt = []
    for s in range(n):
        g, r = gpu_logits[s].cpu().numpy(), ref_logits[s].numpy()
        assert_close(g, r, tol, tol, f"{what}: step {s} logits")
        for row in range(r.shape[0]):
            top2 = np.sort(r[row])[-2:]
            margin = float(top2[1] - top2[0])
            if margin > 2 * err:
                assert got[row, s] == int(np.argmax(r[row])), \
                    f"{what}: step {s} row {row}: margin {margin:.4f} > 2 x err {err:.2e}"
            else:
                exempt.append((s, row, margin))
    total = n * ref_logits[0].shape[0]
    scale = max(float(np.abs(ref_logits[s].numpy()).max()) for s in range(n))
    print(f"[greedy] {what}: per-step max logit error {[f'{e:.1e}' for e in errs]}, "
          f"max |logit| {scale:.2f}")
    print(f"[greedy] {what}: max logit error {err:.2e}; {len(exempt)} of {total} argmax checks "
          f"exempt (oracle top-2 margin <= {2 * err:.2e}): {exempt}")
    assert len(exempt) <= max_exempt_frac * total
