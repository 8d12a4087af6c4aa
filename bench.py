#!/usr/bin/env python3
"""SVD-MLP layer benchmark on one MI355X (BASELINE.json metric).

One step = one SVD-MLP layer forward, y = xuv(gate_up(x)), over one batch:
the LLaMA3-8B-shape layer at T=1024 tokens, bf16.  The
value is algorithmic TFLOP/s, 2*T*3*r*(d+ff) per step, with inputs resident
in HBM.  Weights rotate over several synthetic layers so that consecutive
steps do not re-read factors out of the 256 MB Infinity Cache.

The JSON line also carries:
  roofline      the dominant kernel (the GEMM stage with the most time per
                layer) timed live with hipEvents on the launch stream:
                algorithmic FLOP per launch / average launch duration vs the
                2.5 PFLOP/s bf16 MFMA peak
  decode        T = 1, 8, 32, 64 decode layers: us/layer
                and GB/s of compulsory bytes vs the 8 TB/s HBM peak
  cpu_baseline  the numpy oracle (oracle/reference_cpu.py) timed on this
                host's cores on a bounded row sample of the same layer

    python bench.py [--gpus 1] [--steps 20] [--warmup 5]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "neuronmlp-on-tpu_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "SVD-MLP layer µs + TFLOP/s (% MFMA peak), LLaMA3-8B shape T=1024; T=1 GB/s"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
D, FF, R = 4096, 14336, 2816


def _args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--tokens", type=int, default=1024)
    p.add_argument("--layers", type=int, default=4, help="synthetic layers the steps rotate over")
    p.add_argument("--decode-steps", type=int, default=200)
    p.add_argument("--decode-tokens", type=int, nargs="*", default=[1, 8, 32, 64])
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only", choices=("prefill", "decode"), default=None,
                   help="run one part only (for profiler runs)")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--copy-check", type=int, default=0, metavar="MIB",
                   help="before the steps, copy a MIB-sized buffer 3 times (a plain copy kernel of known size "
                        "for calibrating rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    p.add_argument("--weights-layout", choices=("natural", "linear"), default="natural",
                   help="natural (in, out) factors as kernels/reference.py takes them, or PyTorch Linear "
                        "(out, in) storage passed as transposed views (test_speedup.py nki_mm)")
    return p.parse_args(argv)


def _layer_weights(torch, dev, seed, linear=False):
    """Synthetic factors of one layer: U ~ N(0, 1/d_in), V ~ N(0, 1/r), bf16,
    drawn on the device from a seeded generator (reference recipe
    test_speedup.py:803-808, device RNG instead of numpy)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def rnd(rows, cols):
        w = (torch.randn(rows, cols, generator=g, device=dev, dtype=torch.float32)
             / math.sqrt(rows)).to(torch.bfloat16)
        return w.t().contiguous().t() if linear else w

    uu, vu, ug, vg = rnd(D, R), rnd(R, FF), rnd(D, R), rnd(R, FF)
    ud, vd = rnd(FF, R), rnd(R, D)
    return ug, vg, uu, vu, ud, vd  # gate-first, kernels/reference.py order


def _stage_work(T):
    """Per-launch algorithmic FLOP, compulsory HBM bytes (bf16 operands read
    once, the stage's bf16 result written once) and a description of each
    GEMM stage of the prefill layer, keyed by the library's stage names."""
    return {
        "gate_up_xu": (2.0 * T * D * 2 * R, 2 * (T * D + 2 * D * R + 2 * T * R),
                       "big_gemm_kernel X.[Ug|Uu] (split-K fp32 slices)"),
        "gate_up_xuv_g": (2.0 * T * R * FF, 2 * (T * R + R * FF + T * FF),
                          "big_gemm_kernel XUg.Vg -> bf16 g"),
        "gate_up_xuv_swiglu": (2.0 * T * R * FF, 2 * (T * R + R * FF + 2 * T * FF),
                               "big_gemm_kernel XUu.Vu, SiLU(g)*u epilogue"),
        "down_xu": (2.0 * T * FF * R, 2 * (T * FF + FF * R + T * R),
                    "big_gemm_kernel h.Ud (split-K fp32 slices)"),
        "down_xuv": (2.0 * T * R * D, 2 * (T * R + R * D + T * D),
                     "big_gemm_kernel XUd.Vd (split-K fp32 slices)"),
    }


TRAFFIC_PROFILE = ROOT / "profiles" / "prefill_8b_T1024_traffic.md"


def _profiled_traffic(stage):
    """HBM bytes per launch of a stage from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, calibrated against a copy kernel of known size),
    or None when the summary has no line for it."""
    try:
        for line in TRAFFIC_PROFILE.read_text().splitlines():
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic_bytes" and parts[1] == stage:
                return int(parts[2])
    except OSError:
        pass
    return None


def _time_steps(torch, fn, steps, warmup, stream):
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / steps, wall


def _cpu_baseline(layer0, x, T, seconds):
    """Time the numpy oracle on a row sample of the same layer."""
    import numpy as np

    import oracle as O

    try:
        from threadpoolctl import threadpool_info

        threads = max((i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"),
                      default=1)
    except Exception:  # pragma: no cover - threadpoolctl is optional
        threads = len(os.sched_getaffinity(0))
    rows = min(128, T)
    f = [w.float().cpu().numpy() for w in layer0]
    xs = x[:rows].float().cpu().numpy()
    O.svd_mlp_ref(xs[:8], *f, dtype="bfloat16")  # warm BLAS
    reps, t0 = 0, time.perf_counter()
    while True:
        y = O.svd_mlp_ref(xs, *f, dtype="bfloat16")
        reps += 1
        el = time.perf_counter() - t0
        if (el >= seconds and reps >= 2) or el >= 3 * seconds:
            break
    flops = O.layer_flops(rows, D, FF, R) * reps
    return {
        "value": round(flops / el / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": int(threads),
        "kind": "port",
        "sample": f"oracle svd_mlp_ref (numpy fp32 GEMMs, bf16 rounding) on {rows} of {T} rows of layer 0, "
                  f"{reps} reps in {el:.1f} s",
    }, y


def main(argv=None) -> int:
    args = _args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); this build runs the SVD-MLP path on a "
              "single MI355X and has no multi-GPU mode.", file=sys.stderr)
        return 2
    import torch

    import svdmlp
    from svdmlp import _lib

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    svdmlp.load()
    stream = torch.cuda.current_stream(dev)
    T = args.tokens
    linear = args.weights_layout == "linear"
    layers = [_layer_weights(torch, dev, args.seed + i, linear) for i in range(args.layers)]
    gx = torch.Generator(device=dev)
    gx.manual_seed(args.seed + 1000)
    x = torch.randn(T, D, generator=gx, device=dev, dtype=torch.float32).to(torch.bfloat16)
    flops = 2.0 * T * 3 * R * (D + FF)
    if args.copy_check > 0:
        n = args.copy_check << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    factor_bytes = 2 * (2 * R * (D + FF) + R * (FF + D))
    record: dict = {}

    if args.only in (None, "prefill"):
        ws = svdmlp.svd_mlp_workspace(x, r=R, ff=FF)
        out = torch.empty(T, D, dtype=torch.bfloat16, device=dev)

        def step(i):
            svdmlp.svd_mlp(x, *layers[i % len(layers)], workspace=ws, out=out)

        ms, wall = _time_steps(torch, step, args.steps, args.warmup, stream)
        with _lib.StageProfile() as prof:
            ms_prof, _ = _time_steps(torch, step, args.steps, 0, stream)
        stages = {k: v[0] / v[1] for k, v in prof.result.items()}
        # Each GEMM stage is one kernel launch; the roofline line is for the
        # one with the most time per layer.
        stage_work = _stage_work(T)
        gemm_stages = {k: v for k, v in stages.items() if k in stage_work}
        dom = max(gemm_stages, key=gemm_stages.get) if gemm_stages else None
        dom_ms = gemm_stages.get(dom)
        dom_flops, dom_bytes, dom_desc = stage_work.get(dom, (None, None, None))
        achieved = dom_flops / (dom_ms * 1e-3) / 1e12 if dom_ms else None
        tflops = flops / (ms * 1e-3) / 1e12
        record.update({
            "metric": METRIC,
            "value": round(tflops, 2),
            "unit": "TFLOP/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(ms, 4),
            "us_per_layer": round(ms * 1e3, 1),
            "pct_mfma_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": "bf16",
            "data": "synthetic (seeded device RNG; U~N(0,1/d_in), V~N(0,1/r), X~N(0,1))",
            "config": {"workload": "LLaMA3-8B SVD-MLP layer, prefill", "T": T, "d": D, "ff": FF, "r": R,
                       "layers_rotated": len(layers), "flop_per_step": flops,
                       "weights_layout": args.weights_layout},
            "wall_s_timed": round(wall, 4),
            "roofline": {
                "kernel": f"{dom}: {dom_desc}" if dom else None,
                "bound": "mfma",
                "achieved": round(achieved, 2) if achieved else None,
                "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4) if achieved else None,
                "traffic": _profiled_traffic(dom) if (T, args.weights_layout) == (1024, "natural") else None,
                "traffic_source": "profiles/prefill_8b_T1024_traffic.md: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE "
                                  "per dispatch, calibrated on a 256 MiB copy",
                "algorithmic_flop_per_launch": dom_flops,
                "algorithmic_bytes_per_launch": dom_bytes,
                "avg_launch_us": round(dom_ms * 1e3, 2) if dom_ms else None,
            },
            "stages_us": {k: round(v * 1e3, 2) for k, v in stages.items()},
            "ms_per_step_with_stage_events": round(ms_prof, 4),
        })
        # in-bench parity on a row sample (oracle is the checker only)
        if not args.no_cpu_baseline:
            base, y_ref = _cpu_baseline(layers[0], x, T, args.cpu_seconds)
            y = svdmlp.svd_mlp(x, *layers[0], workspace=ws, out=out)
            import oracle as O

            got = y[: y_ref.shape[0]].float().cpu().numpy()
            record["parity_rel_l2_vs_oracle"] = round(O.relative_l2(got, y_ref), 6)
            record["cpu_baseline"] = base

    if args.only in (None, "decode"):
        dec = {}
        for Td in args.decode_tokens:
            xd = x[:Td].contiguous()
            wsd = svdmlp.svd_mlp_workspace(xd, r=R, ff=FF)
            outd = torch.empty(Td, D, dtype=torch.bfloat16, device=dev)

            def dstep(i, xd=xd, wsd=wsd, outd=outd):
                svdmlp.svd_mlp(xd, *layers[i % len(layers)], workspace=wsd, out=outd)

            msd, _ = _time_steps(torch, dstep, args.decode_steps, 10, stream)
            with _lib.StageProfile() as prof:
                _time_steps(torch, dstep, min(args.decode_steps, 50), 0, stream)
            nbytes = factor_bytes + 2 * Td * D * 2
            gbs = nbytes / (msd * 1e-3) / 1e9
            dec[f"T={Td}"] = {
                "us_per_layer": round(msd * 1e3, 2),
                "GB/s": round(gbs, 1),
                "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
                "TFLOP/s": round(2.0 * Td * 3 * R * (D + FF) / (msd * 1e-3) / 1e12, 3),
                "stages_us": {k: round(v[0] / v[1] * 1e3, 2) for k, v in prof.result.items()},
            }
        record["decode"] = dec
        if args.only == "decode":
            t1 = dec.get("T=1") or next(iter(dec.values()))
            record.update({"metric": METRIC, "value": t1["GB/s"], "unit": "GB/s", "n_gpus": 1,
                           "steps": args.decode_steps, "warmup": 10, "ms_per_step": t1["us_per_layer"] / 1e3,
                           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                           "data": "synthetic", "config": {"workload": "LLaMA3-8B SVD-MLP layer, decode"}})
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
