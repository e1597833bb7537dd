"""Benchmark of the selective-scan inference path on one MI355X.

Prints ONE JSON line.  Headline (``value``): the fused chunked scan at BASELINE
config 4 -- fp16 B=4, D=5120, N=16, L=32768 with D skip, SiLU(z) gate, softplus
delta and final-state write -- in Mtok/s (batch*seqlen tokens per step), inputs
resident in HBM.  A step is one ``selective_scan`` call (B/C pack + scan kernel).

  roofline      algorithmic bytes of one call / its average duration measured with
                HIP events on the launch stream, against the 8 TB/s HBM peak;
                ``traffic`` = measured HBM bytes per launch from the committed
                rocprofv3 counter summary (profiles/scan_traffic.json) when present.
  cpu_baseline  the build's C restatement of the reference's sequential scan
                (oracle/scan_ref.c, fp32, OpenMP over channels) timed on this
                host on a bounded channel sample of the same workload and scaled
                to the whole workload.  The reference's MLX CPU path cannot run
                here (no MLX, no network).
  extra         config 2 scan, the copy-probe HBM peak, and decode tok/s for the
                130m (config 1) and 2.8b (config 3) random-init models.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-decode] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
METRIC = "scan prefill Mtok/s + HBM GB/s (% of peak); decode tok/s at 130m/2.8b"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def scan_bytes(batch, dim, dstate, seqlen, xs=2, bcs=2, has_z=True, has_D=True, state=True):
    """Algorithmic HBM bytes of one scan: every input read once, every output written once."""
    n = batch * dim * seqlen * (xs * (3 + (1 if has_z else 0)))      # u, delta, y (+ z)
    n += batch * dstate * seqlen * 2 * bcs                          # B, C
    n += dim * dstate * 4 + (dim * 4 if has_D else 0)               # A, D
    n += batch * dim * dstate * 4 if state else 0                   # final state
    return n


def make_scan_inputs(batch, dim, dstate, seqlen, seed, dev):
    import torch

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    f16 = torch.float16
    u = torch.randn((batch, dim, seqlen), generator=g, device=dev).to(f16)
    d = (torch.randn((batch, dim, seqlen), generator=g, device=dev) * 0.5 - 1.0).to(f16)
    z = torch.randn((batch, dim, seqlen), generator=g, device=dev).to(f16)
    B = torch.randn((batch, dstate, seqlen), generator=g, device=dev).to(f16)
    C = torch.randn((batch, dstate, seqlen), generator=g, device=dev).to(f16)
    A = -torch.arange(1, dstate + 1, device=dev, dtype=torch.float32).expand(dim, dstate).contiguous()
    D = torch.ones(dim, device=dev)
    return u, d, A, B, C, D, z


def time_scan(batch, dim, dstate, seqlen, steps, warmup, seed=0):
    import torch

    from mamba_metal_amd import selective_scan

    dev = torch.device("cuda:0")
    u, d, A, B, C, D, z = make_scan_inputs(batch, dim, dstate, seqlen, seed, dev)
    run = lambda: selective_scan(u, d, A, B, C, D=D, z=z, delta_softplus=True, return_state=True)
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    t0 = time.perf_counter()
    for e0, e1 in evs:
        e0.record(stream)
        run()
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ev_ms = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
    del u, d, z, B, C
    torch.cuda.empty_cache()
    return {"wall_ms_per_step": wall * 1e3 / steps, "event_ms_avg": sum(ev_ms) / len(ev_ms),
            "event_ms_median": ev_ms[len(ev_ms) // 2], "event_ms_min": ev_ms[0]}


def copy_probe_gbs():
    """Achievable HBM bandwidth: device-to-device copy of 2 GiB (read + write bytes)."""
    import torch

    n = 1 << 30
    src = torch.empty(n, dtype=torch.float16, device="cuda:0").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    reps = 10
    for _ in range(reps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del src, dst
    torch.cuda.empty_cache()
    return 2 * n * 2 / (ms * 1e-3) / 1e9


def cpu_baseline(batch, dim, dstate, seqlen, n_channels=5120):
    """C oracle (fp32 math, OpenMP) on n_channels of the workload -- a quarter of
    config 4, about 12 s of CPU work on 16 threads -- scaled to all B*D."""
    import numpy as np

    from oracle import cscan

    per_b = max(1, n_channels // batch)
    rng = np.random.default_rng(123)
    f = lambda *s: rng.standard_normal(s).astype(np.float16).astype(np.float32)
    u, z = f(batch, per_b, seqlen), f(batch, per_b, seqlen)
    d = (rng.standard_normal((batch, per_b, seqlen)) * 0.5 - 1.0).astype(np.float16).astype(np.float32)
    B, C = f(batch, dstate, seqlen), f(batch, dstate, seqlen)
    A = -np.broadcast_to(np.arange(1, dstate + 1, dtype=np.float32), (per_b, dstate)).copy()
    D = np.ones(per_b, np.float32)
    cscan.selective_scan(u[:, :1, :64], d[:, :1, :64], A[:1], B[:, :, :64], C[:, :, :64],
                         D=D[:1], z=z[:, :1, :64], delta_softplus=True, precision="f32")
    t0 = time.perf_counter()
    cscan.selective_scan(u, d, A, B, C, D=D, z=z, delta_softplus=True, precision="f32")
    dt = time.perf_counter() - t0
    scale = (batch * dim) / (batch * per_b)
    t_full = dt * scale
    return {"value": batch * seqlen / t_full / 1e6, "unit": "Mtok/s", "cores": cscan.num_threads(),
            "kind": "port",
            "sample": f"{batch * per_b} of {batch * dim} channels ({per_b} per batch row), "
                      f"L={seqlen}, N={dstate}, fp16-rounded inputs, D+z+softplus+state; "
                      f"{dt:.2f} s wall on {cscan.num_threads()} threads measured, scaled x{scale:.0f}",
            "sample_seconds": dt}


def decode_bench(name, cfg_kw, batch, prompt_len, n_decode, seed=0):
    """Random-init model: parallel prefill, then n_decode greedy steps (HIP graph)."""
    import torch

    from mamba_metal_amd import GraphDecoder, MambaConfig, MambaModel, init_weights_

    dev = torch.device("cuda:0")
    cfg = MambaConfig(**cfg_kw)
    with torch.device("meta"):
        model = MambaModel(cfg, dtype=torch.float16)
    model = init_weights_(model.to_empty(device=dev), seed=seed).eval()
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    ids = torch.randint(0, cfg.vocab_size, (batch, prompt_len), generator=g, device=dev)
    dec = GraphDecoder(model, batch, use_graph=True)
    dec.start(ids)                           # warm-up prefill + graph capture
    for _ in range(3):
        dec.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dec.start(ids)
    torch.cuda.synchronize()
    t_prefill = time.perf_counter() - t0
    t0 = time.perf_counter()
    for _ in range(n_decode):
        dec.step()
    torch.cuda.synchronize()
    t_dec = time.perf_counter() - t0
    res = {"prefill_s": t_prefill, "prefill_tok_s": batch * prompt_len / t_prefill,
           "decode_ms_per_step": t_dec * 1e3 / n_decode,
           "decode_tok_s": batch * n_decode / t_dec, "batch": batch, "prompt": prompt_len,
           "steps": n_decode}
    del model, dec
    torch.cuda.empty_cache()
    log(f"{name}: {res}")
    return res


def gemm_probe(calls=24, n_weights=12):
    """The decode GEMM at Mamba-2.8B's in_proj shape (M=64, K=2560, N=10240 fp16), weights
    rotated so each call streams its 52 MB from HBM; HIP-event average per call."""
    import torch

    from mamba_metal_amd.linear import decode_linear, packed_weight

    dev = torch.device("cuda:0")
    M, K, N = 64, 2560, 10240
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    ws = [(torch.randn((N, K), generator=g, device=dev) * 0.02).half() for _ in range(n_weights)]
    for w in ws:
        packed_weight(w)
    x = torch.randn((M, K), generator=g, device=dev).half()
    out = torch.empty((M, N), device=dev, dtype=torch.float16)
    for i in range(3):
        decode_linear(x, ws[i % n_weights], out=out)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(calls):
        decode_linear(x, ws[i % n_weights], out=out)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / calls
    return {"gemm": "decode in_proj M=64 K=2560 N=10240 fp16", "us_per_call": us,
            "weight_gbs": N * K * 2 / us / 1e3, "calls": calls}


def decode_roofline_bytes(d_model, n_layer, vocab, d_state, d_conv, dt_rank, batch):
    """Weights (fp16) once + fp32 SSM state r/w + fp16 conv state r/w per decode step."""
    di = 2 * d_model
    per_layer = (d_model * 2 * di + di * d_conv + di + di * (dt_rank + 2 * d_state)
                 + dt_rank * di + di + di * d_state + di + di * d_model + d_model)
    params = per_layer * n_layer + vocab * d_model + d_model
    w = params * 2
    ssm = batch * di * d_state * 4 * 2 * n_layer
    conv = batch * di * d_conv * 2 * 2 * n_layer
    return w + ssm + conv


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--copy-probe-only", action="store_true",
                    help="run only the 2 GiB device copy (HBM counter calibration)")
    ap.add_argument("--only-decode", choices=["130m", "2.8b"],
                    help="run one decode benchmark only (the command of the decode profiles)")
    ap.add_argument("--only-scan", action="store_true",
                    help="config-4 scan only (the command the committed rocprof summaries use)")
    ap.add_argument("--only-gemm", action="store_true",
                    help="the decode GEMM at the 2.8B in_proj shape only (counter profiles)")
    args = ap.parse_args()
    if args.only_scan:
        args.no_extra = args.no_decode = args.no_cpu = True
    if args.gpus != 1:
        print(f"bench.py runs on exactly one GPU (got --gpus {args.gpus}); the scan would shard "
              "over (batch, channel) with no exchange between GPUs, so one GPU's share is the "
              "measured unit", file=sys.stderr)
        sys.exit(2)

    import torch

    from mamba_metal_amd import _lib

    if args.only_gemm:
        _lib.load()
        print(json.dumps(gemm_probe()))
        return
    if args.only_decode:
        _lib.load()
        if args.only_decode == "130m":
            r = decode_bench("130m", dict(d_model=768, n_layer=24, vocab_size=50280, dt_rank=48),
                             1, 2048, 128)
        else:
            r = decode_bench("2.8b", dict(d_model=2560, n_layer=64, vocab_size=50280, dt_rank=160),
                             64, 512, 256)
        print(json.dumps(r))
        return
    if args.copy_probe_only:
        print(json.dumps({"copy_probe_gbs": copy_probe_gbs(), "bytes_per_copy": 2 * (1 << 30)}))
        return
    _lib.load()
    torch.backends.cuda.matmul.allow_tf32 = False
    B, D, N, L = 4, 5120, 16, 32768
    log(f"config 4 scan: B={B} D={D} N={N} L={L} fp16, steps={args.steps} warmup={args.warmup}")
    r = time_scan(B, D, N, L, args.steps, args.warmup)
    nbytes = scan_bytes(B, D, N, L)
    tokens = B * L
    achieved = nbytes / (r["event_ms_avg"] * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": tokens / (r["wall_ms_per_step"] * 1e-3) / 1e6,
        "unit": "Mtok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["wall_ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "io_dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "config4: fused chunked selective scan, fp16 B=4 D=5120 N=16 "
                               "L=32768, D skip + SiLU(z) + softplus + final state",
                   "batch": B, "dim": D, "dstate": N, "seqlen": L},
        "hbm_gbs": achieved,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": None,
                     "algorithmic_bytes": nbytes, "event_ms_avg": r["event_ms_avg"],
                     "event_ms_median": r["event_ms_median"], "event_ms_min": r["event_ms_min"]},
    }
    tf = ROOT / "profiles" / "scan_traffic.json"
    if tf.exists():
        try:
            out["roofline"]["traffic"] = json.loads(tf.read_text()).get("config4_bytes_per_launch")
        except Exception as e:  # noqa: BLE001
            log(f"traffic file unreadable: {e}")
    log(f"config 4: {out['value']:.1f} Mtok/s, {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%})")

    extra = {}
    if not args.no_extra:
        try:
            probe = copy_probe_gbs()
            extra["copy_probe_gbs"] = probe
            out["roofline"]["frac_of_copy_probe"] = achieved / probe
            r2 = time_scan(8, 1536, 16, 8192, args.steps, args.warmup, seed=2)
            b2 = scan_bytes(8, 1536, 16, 8192)
            extra["config2_scan"] = {"Mtok_s": 8 * 8192 / (r2["wall_ms_per_step"] * 1e-3) / 1e6,
                                     "gbs": b2 / (r2["event_ms_avg"] * 1e-3) / 1e9,
                                     "event_ms_avg": r2["event_ms_avg"]}
            log(f"config 2: {extra['config2_scan']}")
        except Exception as e:  # noqa: BLE001
            extra["error_scan_extra"] = repr(e)
    if not args.no_decode:
        try:
            extra["decode_130m"] = decode_bench(
                "130m", dict(d_model=768, n_layer=24, vocab_size=50280, dt_rank=48), 1, 2048, 128)
            rb = decode_roofline_bytes(2560, 64, 50280, 16, 4, 160, 64)
            c3 = decode_bench(
                "2.8b", dict(d_model=2560, n_layer=64, vocab_size=50280, dt_rank=160), 64, 512, 256)
            c3["roofline_bytes_per_step"] = rb
            c3["roofline_frac"] = (rb / (c3["decode_ms_per_step"] * 1e-3) / 1e9) / HBM_PEAK_GBS
            extra["decode_2p8b"] = c3
        except Exception as e:  # noqa: BLE001
            extra["error_decode"] = repr(e)
    out["extra"] = extra
    if not args.no_cpu:
        try:
            out["cpu_baseline"] = cpu_baseline(B, D, N, L)
            log(f"cpu baseline: {out['cpu_baseline']}")
        except Exception as e:  # noqa: BLE001
            out["cpu_baseline"] = {"error": repr(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
