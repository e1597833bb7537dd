"""Benchmark of the selective-scan inference path on one MI355X.

Prints ONE JSON line.  Headline (``value``): the fused chunked scan at BASELINE
config 4 -- fp16 B=4, D=5120, N=16, L=32768 with D skip, SiLU(z) gate, softplus
delta and final-state write -- in Mtok/s (batch*seqlen tokens per step), inputs
resident in HBM.  A step is one ``selective_scan`` call (B/C pack + scan kernel).

  roofline      algorithmic bytes of one call / its average duration measured with
                HIP events on the launch stream, against the 8 TB/s HBM peak;
                ``traffic`` = measured HBM bytes per launch from the committed
                rocprofv3 counter summary (profiles/scan_traffic.json) when present.
                ``valu_floor_frac`` = the recurrence's VALU issue floor (6 issue slots
                per state update on 256 CUs at 2.4 GHz) over the measured time.
  cpu_baseline  the build's C restatement of the reference's sequential scan
                (oracle/scan_ref.c, fp32, OpenMP over channels) timed on this
                host on a bounded channel sample of the same workload and scaled
                to the whole workload; ``scan_configs`` adds configs 0 / 2 / 4 on all
                threads and on one core plus the numpy restatement, ``decode`` the
                torch-CPU model restatement's decode step at 130m and 2.8b.  The
                reference's MLX CPU path cannot run here (no MLX, no network).
  extra         config 2 (with its roofline fraction and measured traffic), config 0,
                the reference's own benchmark shape (B=1 D=16 N=16 L=32768 fp32, y only,
                experiments/08-benchmark/bench.py:76-100), the copy-probe HBM peak,
                and decode tok/s with roofline fractions for the 130m (config 1) and 2.8b
                (config 3) random-init models.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-decode] [--no-cpu]
       python bench.py --only-scan [config4|config2|reference] | --only-gemm [store|conv|conv_xp]
                       | --only-decode {130m,2.8b} | --copy-probe-only   (profiling commands)
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


def make_reference_shape_inputs(batch, dim, dstate, seqlen, seed, dev):
    """The reference's own scan benchmark inputs (experiments/08-benchmark/bench.py:17-27):
    fp32, delta ~ U(0.01, 0.1), A = -U(0.1, 2), u, B, C ~ N(0, 1); no D, no z, no softplus."""
    import torch

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    u = torch.randn((batch, dim, seqlen), generator=g, device=dev)
    d = torch.rand((batch, dim, seqlen), generator=g, device=dev) * 0.09 + 0.01
    A = -(torch.rand((dim, dstate), generator=g, device=dev) * 1.9 + 0.1)
    B = torch.randn((batch, dstate, seqlen), generator=g, device=dev)
    C = torch.randn((batch, dstate, seqlen), generator=g, device=dev)
    return u, d, A, B, C


def time_scan(batch, dim, dstate, seqlen, steps, warmup, seed=0, kind="config"):
    """HIP-event and wall timing of one selective_scan call per step.  kind "config":
    BASELINE configs 2/4 inputs (fp16, D + z + softplus + final state); "config0": the
    same distributions in fp32; "reference": the reference's own
    benchmark inputs and call (fp32, y only)."""
    import torch

    from mamba_metal_amd import selective_scan

    dev = torch.device("cuda:0")
    if kind == "reference":
        u, d, A, B, C = make_reference_shape_inputs(batch, dim, dstate, seqlen, seed, dev)
        D = z = None
        run = lambda: selective_scan(u, d, A, B, C)
    else:
        u, d, A, B, C, D, z = make_scan_inputs(batch, dim, dstate, seqlen, seed, dev)
        if kind == "config0":
            u, d, B, C, z = (t.float() for t in (u, d, B, C, z))
        run = lambda: selective_scan(u, d, A, B, C, D=D, z=z, delta_softplus=True,
                                     return_state=True)
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
    del u, d, B, C
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


# VALU issue floor of the scan: one state update is a multiply (delta2 * A), v_exp_f32
# (two issue slots), a multiply (delta2 * u * B) and two fmas (state, C contraction) =
# 6 issue slots of a 64-lane wave; MI355X issues 256 CUs x 4 SIMDs x 16 lanes per clock at
# 2.4 GHz (packed fp32 is not used).  The floor ignores the per-(channel, step) work.
VALU_SLOTS_PER_UPDATE = 6
VALU_LANE_SLOTS_PER_S = 256 * 64 * 2.4e9


def valu_floor_ms(batch, dim, dstate, seqlen):
    return batch * dim * dstate * seqlen * VALU_SLOTS_PER_UPDATE / VALU_LANE_SLOTS_PER_S * 1e3


def _cpu_scan_inputs(batch, dim, dstate, seqlen, seed=123):
    import numpy as np

    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float16).astype(np.float32)
    u, z = f(batch, dim, seqlen), f(batch, dim, seqlen)
    d = (rng.standard_normal((batch, dim, seqlen)) * 0.5 - 1.0).astype(np.float16).astype(np.float32)
    B, C = f(batch, dstate, seqlen), f(batch, dstate, seqlen)
    A = -np.broadcast_to(np.arange(1, dstate + 1, dtype=np.float32), (dim, dstate)).copy()
    D = np.ones(dim, np.float32)
    return u, d, A, B, C, D, z


def _time_cscan(inp, threads=None, reps=1):
    from oracle import cscan

    u, d, A, B, C, D, z = inp
    n0 = cscan.num_threads()
    if threads:
        cscan.set_num_threads(threads)
    try:
        cscan.selective_scan(u[:, :1, :64], d[:, :1, :64], A[:1], B[:, :, :64], C[:, :, :64],
                             D=D[:1], z=z[:, :1, :64], delta_softplus=True, precision="f32")
        t0 = time.perf_counter()
        for _ in range(reps):
            cscan.selective_scan(u, d, A, B, C, D=D, z=z, delta_softplus=True, precision="f32")
        return (time.perf_counter() - t0) / reps, cscan.num_threads()
    finally:
        cscan.set_num_threads(n0)


def cpu_scan_extras():
    """The C restatement on all host threads and on one core at configs 0, 2 and 4 (channel
    samples scaled to the whole workload), and the numpy restatement (vectorised over
    channels, loop over time: the analogue of experiments/08-benchmark/bench.py:107-123)
    at config 0."""
    import numpy as np

    from oracle import numpy_ref

    out = {}
    # (channels per batch row timed, repetitions) on all threads and on one core, each
    # sized to ~0.2-0.5 s of wall time on a 16-thread host
    for name, (b, dim, n, L), allt, one in (
            ("config0", (1, 16, 16, 4096), (16, 40), (16, 10)),
            ("config2", (8, 1536, 16, 8192), (192, 1), (16, 1)),
            ("config4", (4, 5120, 16, 32768), None, (16, 1))):
        rows = {}
        for label, spec, thr in (("all_threads", allt, None), ("one_core", one, 1)):
            if spec is None:
                continue
            pb, reps = spec
            dt, used = _time_cscan(_cpu_scan_inputs(b, pb, n, L), thr, reps)
            scale = dim / pb
            rows[label] = {"Mtok_s": b * L / (dt * scale) / 1e6, "cores": used,
                           "sample": f"{b * pb} of {b * dim} channels, {dt * 1e3:.2f} ms per call "
                                     f"({reps} calls), scaled x{scale:.0f}"}
        out[name] = rows
    u, d, A, B, C, D, z = _cpu_scan_inputs(1, 16, 16, 4096)
    t0 = time.perf_counter()
    numpy_ref.selective_scan(u, d, A, B, C, D=D, z=z, delta_softplus=True)
    dt = time.perf_counter() - t0
    out["config0"]["numpy_float64"] = {"Mtok_s": 4096 / dt / 1e6, "cores": 1,
                                       "sample": f"whole config 0, {dt:.3f} s"}
    return out


def _random_ref_weights(cfg, layers, seed=0):
    import numpy as np
    import torch

    rng = np.random.default_rng(seed)
    g = lambda *s: torch.from_numpy((rng.standard_normal(s) * 0.02).astype(np.float32))
    di, r, n, K, dm = cfg.d_inner, cfg.dt_rank, cfg.d_state, cfg.d_conv, cfg.d_model
    w = {"embeddings.weight": g(cfg.vocab_size, dm), "norm_f.weight": torch.ones(dm)}
    for i in range(layers):
        p = f"layers.{i}."
        w.update({p + "norm.weight": torch.ones(dm), p + "mixer.in_proj.weight": g(2 * di, dm),
                  p + "mixer.conv1d.weight": g(di, 1, K), p + "mixer.conv1d.bias": torch.zeros(di),
                  p + "mixer.x_proj.weight": g(r + 2 * n, di), p + "mixer.dt_proj.weight": g(di, r),
                  p + "mixer.dt_proj.bias": torch.full((di,), -2.0),
                  p + "mixer.A_log": torch.log(torch.arange(1, n + 1, dtype=torch.float32)).expand(di, n).clone(),
                  p + "mixer.D": torch.ones(di), p + "mixer.out_proj.weight": g(dm, di)})
    return w


def cpu_decode_extras():
    """The torch-CPU float32 restatement of MambaModel.step (oracle/model_ref.py) timed per
    decode step: 130m at batch 1 (all 24 layers); 2.8b at batch 64 on 2 of its 64 layers
    plus the head, scaled to 64 layers."""
    import torch

    from oracle.model_ref import RefConfig, RefModel

    out = {}
    for name, dm, nl, vocab, r, batch, sample_layers in (("130m", 768, 24, 50280, 48, 1, 24),
                                                          ("2.8b", 2560, 64, 50280, 160, 64, 2)):
        cfg = RefConfig(dm, sample_layers, vocab, 16, 4, 2, r)
        model = RefModel(cfg, _random_ref_weights(cfg, sample_layers), dtype=torch.float32)
        convs = [torch.zeros(batch, cfg.d_inner, 4) for _ in range(sample_layers)]
        ssms = [torch.zeros(batch, cfg.d_inner, 16) for _ in range(sample_layers)]
        ids = torch.zeros(batch, dtype=torch.long)
        model.step(ids, convs, ssms)
        steps = 3 if name == "130m" else 1
        t0 = time.perf_counter()
        for _ in range(steps):
            model.step(ids, convs, ssms)
        dt = (time.perf_counter() - t0) / steps
        x = torch.zeros(batch, dm)
        t1 = time.perf_counter()
        x @ model.w["embeddings.weight"].T
        head = time.perf_counter() - t1
        per_step = head + (dt - head) * nl / sample_layers
        out[name] = {"ms_per_step": per_step * 1e3, "tok_s": batch / per_step,
                     "cores": torch.get_num_threads(), "batch": batch,
                     "sample": f"{sample_layers} of {nl} layers timed ({dt * 1e3:.1f} ms/step incl. "
                               f"the head), layers scaled x{nl / sample_layers:.0f}"}
        del model
    return out


def cpu_baseline(batch, dim, dstate, seqlen, n_channels=5120):
    """C oracle (fp32 math, OpenMP over channels) on n_channels of the workload -- a
    quarter of config 4: about 1 s of wall time on the GPU box's 16 host threads, i.e.
    ~15 thread-seconds of CPU work -- scaled to all B*D.  This is config 4's all-threads
    figure (``scan_configs`` adds its one-core figure)."""
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
    """Random-init model: parallel prefill, then n_decode greedy steps (HIP graph of 8 steps)."""
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
    dec = GraphDecoder(model, batch, use_graph=True, steps_per_graph=8)
    dec.start(ids)                           # warm-up prefill + graph capture (8 steps a replay)
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


def gemm_probe(calls=24, n_weights=12, mode="store"):
    """The decode GEMM at Mamba-2.8B's in_proj shape (M=64, K=2560, N=10240 fp16), weights
    rotated so each call streams its 52 MB from HBM; HIP-event average per call.  mode
    "store": the plain product (mm_decode_linear); "conv": in_proj + conv window
    (mm_decode_linear, CONV epilogue); "conv_xp": in_proj + conv window + x_proj
    (mm_decode_in_proj_xproj) exactly as the decode step runs it -- the in_proj kernel with
    the CONV and x_proj-partial epilogue, then the x_proj plane reduce."""
    import torch

    from mamba_metal_amd.linear import (decode_in_proj_conv, decode_in_proj_conv_xproj, decode_linear,
                                        packed_weight)

    dev = torch.device("cuda:0")
    M, K, N = 64, 2560, 10240
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    ws = [(torch.randn((N, K), generator=g, device=dev) * 0.02).half() for _ in range(n_weights)]
    for w in ws:
        packed_weight(w)
    x = torch.randn((M, K), generator=g, device=dev).half()
    out = torch.empty((M, N), device=dev, dtype=torch.float16)
    if mode != "store":
        di = N // 2
        conv_state = torch.zeros((M, di, 4), device=dev, dtype=torch.float16)
        conv_w = (torch.randn((di, 1, 4), generator=g, device=dev) * 0.5).half()
        conv_b = torch.zeros(di, device=dev, dtype=torch.float16)
        w_x = (torch.randn((160 + 32, di), generator=g, device=dev) * 0.02).half()
        packed_weight(w_x)
        if mode == "conv_xp":
            run = lambda i: decode_in_proj_conv_xproj(x, ws[i % n_weights], conv_state, conv_w, conv_b, w_x)
        else:
            run = lambda i: decode_in_proj_conv(x, ws[i % n_weights], conv_state, conv_w, conv_b)
    else:
        run = lambda i: decode_linear(x, ws[i % n_weights], out=out)
    for i in range(3):
        run(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(calls):
        run(i)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / calls
    name = {"store": "decode in_proj", "conv": "decode in_proj + conv",
            "conv_xp": "decode in_proj + conv + x_proj"}[mode]
    return {"gemm": f"{name} M=64 K=2560 N=10240 fp16", "us_per_call": us,
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
    ap.add_argument("--only-scan", nargs="?", const="config4",
                    choices=["config4", "config2", "reference"],
                    help="one scan only (the command the committed rocprof summaries use)")
    ap.add_argument("--only-gemm", nargs="?", const="store", choices=["store", "conv", "conv_xp"],
                    help="a decode GEMM at the 2.8B in_proj shape only (counter profiles): the "
                         "plain kernel, in_proj + conv window, or in_proj + conv window + x_proj "
                         "partials as decode runs it")
    args = ap.parse_args()
    if args.only_scan and args.only_scan != "config4":
        import torch

        from mamba_metal_amd import _lib

        _lib.load()
        shp, kind = ((8, 1536, 16, 8192), "config") if args.only_scan == "config2" else \
            ((1, 16, 16, 32768), "reference")
        r = time_scan(*shp, args.steps, args.warmup, seed=2, kind=kind)
        print(json.dumps({"scan": args.only_scan, "shape": shp, **r}))
        return
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
        print(json.dumps(gemm_probe(mode=args.only_gemm)))
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
                     "event_ms_median": r["event_ms_median"], "event_ms_min": r["event_ms_min"],
                     "valu_floor_ms": valu_floor_ms(B, D, N, L),
                     "valu_floor_frac": valu_floor_ms(B, D, N, L) / r["event_ms_avg"]},
    }
    tf = ROOT / "profiles" / "scan_traffic.json"
    traffic = {}
    if tf.exists():
        try:
            traffic = json.loads(tf.read_text())
            out["roofline"]["traffic"] = traffic.get("config4_bytes_per_launch")
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
            g2 = b2 / (r2["event_ms_avg"] * 1e-3) / 1e9
            extra["config2_scan"] = {"Mtok_s": 8 * 8192 / (r2["wall_ms_per_step"] * 1e-3) / 1e6,
                                     "gbs": g2, "roofline_frac": g2 / HBM_PEAK_GBS,
                                     "algorithmic_bytes": b2, "traffic": traffic.get("config2_bytes_per_launch"),
                                     "event_ms_avg": r2["event_ms_avg"],
                                     "valu_floor_frac": valu_floor_ms(8, 1536, 16, 8192) / r2["event_ms_avg"]}
            log(f"config 2: {extra['config2_scan']}")
            r0 = time_scan(1, 16, 16, 4096, args.steps, args.warmup, seed=0, kind="config0")
            extra["config0_scan"] = {"Mtok_s": 4096 / (r0["wall_ms_per_step"] * 1e-3) / 1e6,
                                     "event_ms_avg": r0["event_ms_avg"], "dtype": "f32"}
            rr = time_scan(1, 16, 16, 32768, args.steps, args.warmup, seed=0, kind="reference")
            extra["reference_shape_scan"] = {
                "shape": "B=1 D=16 N=16 L=32768 fp32, no D/z/softplus, y only "
                         "(experiments/08-benchmark/bench.py:76-100)",
                "Mtok_s": 32768 / (rr["wall_ms_per_step"] * 1e-3) / 1e6,
                "event_ms_avg": rr["event_ms_avg"],
                "reference_published_Mtok_s": 45.0, "reference_hardware": "Apple M4 Max (README.md:107)"}
            log(f"config 0: {extra['config0_scan']}; reference shape: {extra['reference_shape_scan']}")
        except Exception as e:  # noqa: BLE001
            extra["error_scan_extra"] = repr(e)
    if not args.no_decode:
        try:
            c1 = decode_bench(
                "130m", dict(d_model=768, n_layer=24, vocab_size=50280, dt_rank=48), 1, 2048, 128)
            r1 = decode_roofline_bytes(768, 24, 50280, 16, 4, 48, 1)
            c1["roofline_bytes_per_step"] = r1
            c1["roofline_frac"] = (r1 / (c1["decode_ms_per_step"] * 1e-3) / 1e9) / HBM_PEAK_GBS
            extra["decode_130m"] = c1
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
        if not args.no_extra:
            try:
                out["cpu_baseline"]["scan_configs"] = cpu_scan_extras()
                log(f"cpu scan configs: {out['cpu_baseline']['scan_configs']}")
            except Exception as e:  # noqa: BLE001
                out["cpu_baseline"]["scan_configs"] = {"error": repr(e)}
            if not args.no_decode:
                try:
                    out["cpu_baseline"]["decode"] = cpu_decode_extras()
                    log(f"cpu decode: {out['cpu_baseline']['decode']}")
                except Exception as e:  # noqa: BLE001
                    out["cpu_baseline"]["decode"] = {"error": repr(e)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
