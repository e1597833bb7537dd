"""Writes the committed golden fixtures of the scan (run from the repo root:
``python tests/golden/make_golden.py``).

The reference commits no vectors for this path, so these come from the build's
float64 oracle (oracle/scan_ref.c), itself pinned by tests/test_oracle.py.
Inputs are NOT stored: they are regenerated from their seeds by
tests/helpers.py (numpy's PCG64 streams are stable); the first eight values of
u are stored to detect generator drift.

  scan_config0.npz  BASELINE config 0: fp32, B=1 D=16 N=16 L=4096, u,B,C,z ~ N(0,1),
                    delta_raw ~ N(-1, 0.5), softplus on, A[d,n] = -(n+1), D = 1.
  scan_edges.npz    short edge cases (L = 1, 33, 1025; N = 1, 5, 64; D = 1, 65).
"""

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path[:0] = [str(ROOT), str(ROOT / "tests")]

from helpers import config0_inputs, features_inputs  # noqa: E402
from oracle import cscan  # noqa: E402

EDGES = [  # (batch, dim, dstate, seqlen, seed)
    (1, 3, 16, 1, 11), (2, 3, 16, 33, 12), (1, 2, 16, 1025, 13),
    (2, 4, 1, 64, 14), (2, 4, 5, 64, 15), (1, 2, 64, 96, 16),
    (1, 1, 16, 200, 17), (1, 65, 16, 40, 18),
]


def run(inp):
    return cscan.selective_scan(inp["u"], inp["delta"], inp["A"], inp["B"], inp["C"],
                                D=inp["D"], z=inp["z"], delta_softplus=True, precision="f64")


def main():
    out = Path(__file__).resolve().parent
    inp = config0_inputs(1, 16, 16, 4096, seed=0)
    y, h = run(inp)
    np.savez_compressed(out / "scan_config0.npz", y=y, state=h, u_head=inp["u"][0, 0, :8])
    edges = {}
    for i, (b, d, n, L, seed) in enumerate(EDGES):
        e = features_inputs(b, d, n, L, seed=seed)
        y, h = run(e)
        edges[f"y{i}"], edges[f"state{i}"] = y, h
        edges[f"u_head{i}"] = e["u"].reshape(-1)[:8]
    edges["shapes"] = np.array(EDGES, dtype=np.int64)
    np.savez_compressed(out / "scan_edges.npz", **edges)
    print("wrote", out / "scan_config0.npz", out / "scan_edges.npz")


if __name__ == "__main__":
    main()
