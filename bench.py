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
                and GB/s of compulsory bytes vs the 8 TB/s HBM peak and vs
                this box's measured copy and streaming-read rates; block_us
                is the MLP block (RMSNorm, layer, residual) at the same T
  cpu_baseline  the numpy oracle (oracle/reference_cpu.py) timed on this
                host's cores on a bounded row sample of the same layer

    python bench.py [--gpus 1] [--steps 50] [--warmup 100]
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
    p.add_argument("--steps", type=int, default=50)
    # the clocks take some tens of milliseconds of load to settle; the prefill
    # line is timed after the other sections (see main), and the first W + K
    # steps of the run are reported beside it as cold_start
    p.add_argument("--warmup", type=int, default=100)
    p.add_argument("--tokens", type=int, default=1024)
    p.add_argument("--layers", type=int, default=4, help="synthetic layers the steps rotate over")
    p.add_argument("--decode-steps", type=int, default=200)
    p.add_argument("--decode-tokens", type=int, nargs="*", default=[1, 2, 8, 32, 64])
    p.add_argument("--no-decode-extra", action="store_true",
                   help="decode: the padded-layout lines only (no dense-layout, launcher or two-rank lines), "
                        "for profiler runs")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only", choices=("prefill", "decode", "stack", "fp8"), default=None,
                   help="run one part only (for profiler runs)")
    p.add_argument("--stack-layers", type=int, default=32)
    p.add_argument("--stack-tokens", type=int, default=4096)
    p.add_argument("--stack-steps", type=int, default=3)
    p.add_argument("--fp8-tokens", type=int, default=2048)
    p.add_argument("--fp8-steps", type=int, default=10)
    # ~2.2 ms per 70B layer: 10 steps are ~22 ms of load, which the clocks
    # need to settle (the first 1 + 5 steps are reported as cold_start)
    p.add_argument("--fp8-warmup", type=int, default=10)
    p.add_argument("--parity-rows", type=int, default=8)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--copy-check", type=int, default=0, metavar="MIB",
                   help="before the steps, copy a MIB-sized buffer 3 times (a plain copy kernel of known size "
                        "for calibrating rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    p.add_argument("--weights-layout", choices=("natural", "padded", "linear"), default="padded",
                   help="natural (in, out) factors as kernels/reference.py takes them; padded: natural with the "
                        "V factors' rows 64 elements longer in memory than their length (read in place); or PyTorch "
                        "Linear (out, in) storage passed as transposed views (test_speedup.py nki_mm)")
    return p.parse_args(argv)


def _layer_weights(torch, dev, seed, linear=False, pad_v=0):
    """Synthetic factors of one layer: U ~ N(0, 1/d_in), V ~ N(0, 1/r), bf16,
    drawn on the device from a seeded generator (reference recipe
    test_speedup.py:803-808, device RNG instead of numpy).  ``pad_v`` > 0
    stores the V factors with rows that many elements wider (the same
    values, read in place through the layered entry points)."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def rnd(rows, cols):
        w = (torch.randn(rows, cols, generator=g, device=dev, dtype=torch.float32)
             / math.sqrt(rows)).to(torch.bfloat16)
        return w.t().contiguous().t() if linear else w

    uu, vu, ug, vg = rnd(D, R), rnd(R, FF), rnd(D, R), rnd(R, FF)
    ud, vd = rnd(FF, R), rnd(R, D)
    if pad_v:
        from svdmlp.ops import pad_rows

        vu, vg, vd = (pad_rows(v, pad_v) for v in (vu, vg, vd))
    return ug, vg, uu, vu, ud, vd  # gate-first, kernels/reference.py order


def _stage_work(T):
    """Per-launch algorithmic FLOP, compulsory HBM bytes (bf16 operands read
    once, the stage's bf16 result written once) and a description of each
    GEMM stage of the prefill layer, keyed by the library's stage names."""
    return {
        "gate_up_xu": (2.0 * T * D * 2 * R, 2 * (T * D + 2 * D * R + 2 * T * R),
                       "big_gemm_kernel X.[Ug|Uu] (1024 tokens: 128x192 K-group tiles, no K split)"),
        "gate_up_xuv_g": (2.0 * T * R * FF, 2 * (T * R + R * FF + T * FF),
                          "big_gemm_kernel XUg.Vg -> bf16 g"),
        "gate_up_xuv_swiglu": (2.0 * T * R * FF, 2 * (T * R + R * FF + 2 * T * FF),
                               "big_gemm_kernel XUu.Vu, SiLU(g)*u epilogue"),
        "gate_up_xuv_dual": (2 * 2.0 * T * R * FF, 2 * (2 * T * R + 2 * R * FF + T * FF),
                             "big_gemm_kernel, one launch: every block XUg.Vg -> bf16 g, then XUu.Vu with the "
                             "SiLU(g)*u epilogue (g's round trip not counted)"),
        "down_xu": (2.0 * T * FF * R, 2 * (T * FF + FF * R + T * R),
                    "big_gemm_kernel h.Ud (split-K fp32 slices)"),
        "down_xuv": (2.0 * T * R * D, 2 * (T * R + R * D + T * D),
                     "big_gemm_kernel XUd.Vd (1024 tokens: 128x128 K-group tiles, no K split)"),
    }


TRAFFIC_PROFILE = ROOT / "profiles" / "prefill_8b_T1024_traffic.md"
MFMA_PROFILE = ROOT / "profiles" / "prefill_8b_T1024_mfma.md"
TRAFFIC_LAYOUT = "padded"   # the weights layout the PMC summaries were taken with
DECODE_TRAFFIC_PROFILE = ROOT / "profiles" / "decode_8b_traffic.md"


def _profiled(key, stage, path):
    """A per-stage figure from a committed rocprofv3 summary: the value of its
    machine-readable line ``<key> <stage> <value>``, or None."""
    try:
        for line in path.read_text().splitlines():
            parts = line.split()
            if len(parts) == 3 and parts[0] == key and parts[1] == stage:
                return float(parts[2])
    except OSError:
        pass
    return None


def _profiled_traffic(stage, path=TRAFFIC_PROFILE):
    """HBM bytes per launch of a stage (FETCH_SIZE + WRITE_SIZE, calibrated
    against a copy kernel of known size), or None."""
    v = _profiled("traffic_bytes", stage, path)
    return int(v) if v is not None else None


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
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(flops / el / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": int(threads),
        "cpu_model": model,
        "kind": "port",
        "sample": f"oracle svd_mlp_ref (numpy fp32 GEMMs, bf16 rounding) on {rows} of {T} rows of layer 0, "
                  f"{reps} reps in {el:.1f} s",
    }, y


def _read_rate(torch, stream, buf, blocks=8192, groups=3, per_group=5):
    """Streaming-read rate (GB/s) of `buf` (a device tensor, whole 16-byte
    words) by the probe library libhbmread.so (csrc/probe/hbm_read.hip,
    built with libsvdmlp.so): `per_group` back-to-back launches between one
    pair of events on `stream` (the launch stream), as the decode lines are
    timed, so one launch's dispatch gap does not count against the rate;
    the best of `groups` such averages."""
    import ctypes

    path = ROOT / "neuronmlp-on-tpu_amd" / "svdmlp" / "libhbmread.so"
    if not path.exists():
        raise RuntimeError(f"{path} is missing: run __graft_entry__.build() first")
    lib = ctypes.CDLL(str(path))
    lib.hbm_read_words.restype = ctypes.c_int
    lib.hbm_read_words.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                   ctypes.c_int32, ctypes.c_void_p]
    nbytes = buf.numel() * buf.element_size()
    out = torch.empty(blocks * 256, dtype=torch.int32, device=buf.device)
    best = None
    for _ in range(groups):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(per_group):
            rc = lib.hbm_read_words(buf.data_ptr(), nbytes, out.data_ptr(), out.numel() * 4, blocks,
                                    stream.cuda_stream)
            if rc != 0:
                raise RuntimeError(f"hbm_read_words failed ({rc})")
        e1.record(stream)
        torch.cuda.synchronize()
        t = e0.elapsed_time(e1) * 1e-3 / per_group
        best = t if best is None else min(best, t)
    return nbytes / best / 1e9


def _bench_decode(torch, dev, stream, args, layers, x, factor_bytes, tokens=None, rates=None, layout=None):
    """the 8B layer at decode token counts (GPU only).
    `rates` (copy, read GB/s) reuses the HBM rates of an earlier call;
    `layout` names the factors' storage when it differs from
    args.weights_layout (no committed traffic profile applies then)."""
    import svdmlp
    from svdmlp import _lib

    if rates is None:
        # measured HBM ceiling for the decode fractions: a 1 GiB device-to-device
        # copy (read + write bytes over its time), best of 5
        n = 1 << 30
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        best = None
        for _ in range(6):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            dst.copy_(src)
            e1.record(stream)
            torch.cuda.synchronize()
            t = e0.elapsed_time(e1) * 1e-3
            best = t if best is None else min(best, t)
        copy_gbs = 2 * n / best / 1e9
        # ... and a streaming read of the same 1 GiB (the decode layers read their
        # factors and write almost nothing): libhbmread.so
        read_gbs = _read_rate(torch, stream, src)
        del src, dst
    else:
        copy_gbs, read_gbs = rates
    layout = layout or args.weights_layout
    dec = {"hbm_copy_GBps": round(copy_gbs, 1), "hbm_read_GBps": round(read_gbs, 1), "weights_layout": layout}
    for Td in (tokens or args.decode_tokens):
        xd = x[:Td].contiguous()
        wsd = svdmlp.svd_mlp_workspace(xd, r=R, ff=FF)
        outd = torch.empty(Td, D, dtype=torch.bfloat16, device=dev)

        def dstep(i, xd=xd, wsd=wsd, outd=outd):
            svdmlp.svd_mlp(xd, *layers[i % len(layers)], workspace=wsd, out=outd)

        msd, _ = _time_steps(torch, dstep, args.decode_steps, max(10, args.warmup), stream)
        # the MLP block around the layer (RMSNorm and residual inside the decode layer's launch)
        gain = torch.ones(D, dtype=torch.float32, device=dev)

        def bstep(i, xd=xd, wsd=wsd, outd=outd, gain=gain):
            svdmlp.svd_mlp_block(xd, gain, *layers[i % len(layers)], workspace=wsd, out=outd)

        msb, _ = _time_steps(torch, bstep, args.decode_steps, 10, stream)
        with _lib.StageProfile() as prof:
            _time_steps(torch, dstep, min(args.decode_steps, 50), 0, stream)
        nbytes = factor_bytes + 2 * Td * D * 2
        gbs = nbytes / (msd * 1e-3) / 1e9
        # measured HBM bytes of the decode layer's launch: the contracted layer at
        # 1-3 tokens (its slices grow with T), else the MFMA layer by 16-row token tiles
        mt = 1 if Td <= 16 else (2 if Td <= 32 else (4 if Td <= 64 else 8))
        kernel = "decode_layer_contracted" if "decode_layer_contracted" in prof.result else "decode_layer"
        key = f"decode_layer_contracted_T{Td}" if kernel == "decode_layer_contracted" else f"decode_layer_mt{mt}"
        traffic = (_profiled_traffic(key, DECODE_TRAFFIC_PROFILE)
                   if layout == TRAFFIC_LAYOUT and Td <= 128 else None)
        dec[f"T={Td}"] = {
            "us_per_layer": round(msd * 1e3, 2),
            "GB/s": round(gbs, 1),
            "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
            "frac_measured_copy": round(gbs / copy_gbs, 4),
            "frac_measured_read": round(gbs / read_gbs, 4),
            "traffic": traffic,
            "traffic_GB/s": round(traffic / (msd * 1e-3) / 1e9, 1) if traffic else None,
            "TFLOP/s": round(2.0 * Td * 3 * R * (D + FF) / (msd * 1e-3) / 1e12, 3),
            "stages_us": {k: round(v[0] / v[1] * 1e3, 2) for k, v in prof.result.items()},
            "kernel": kernel,
            "block_us": round(msb * 1e3, 2),
        }
        if svdmlp.workspace_status(wsd):
            raise RuntimeError(f"decode T={Td}: a grid-barrier wait gave up (the device was shared?)")
    return dec


# BASELINE config 4 draws the gate, up and down ranks of a layer
# independently from {2048, ..., 3072}; one such draw, at decode shapes
TWO_RANKS = (2304, 3072, 2560)


def _bench_decode_ranks(torch, dev, stream, args, x, rates):
    """The 8B layer at decode token counts with a gate, an up and a down rank
    of their own (TWO_RANKS): each branch at its rank inside the decode
    layer's launch (GPU only)."""
    import svdmlp
    from svdmlp import _lib

    r_g, r_u, r_d = TWO_RANKS

    def layer(seed):
        g = torch.Generator(device=dev)
        g.manual_seed(seed)

        def rnd(rows, cols):
            return (torch.randn(rows, cols, generator=g, device=dev, dtype=torch.float32)
                    / math.sqrt(rows)).to(torch.bfloat16)

        return rnd(D, r_g), rnd(r_g, FF), rnd(D, r_u), rnd(r_u, FF), rnd(FF, r_d), rnd(r_d, D)

    layers = [layer(args.seed + 50 + i) for i in range(args.layers)]
    nbytes_w = 2 * (D * r_g + r_g * FF + D * r_u + r_u * FF + FF * r_d + r_d * D)
    out = {"ranks_gate_up_down": list(TWO_RANKS), "factor_bytes": nbytes_w}
    for Td in [t for t in (1, 8, 64) if t <= x.shape[0]]:
        xd = x[:Td].contiguous()
        wsd = svdmlp.svd_mlp_workspace(xd, r=max(TWO_RANKS), ff=FF)
        outd = torch.empty(Td, D, dtype=torch.bfloat16, device=dev)
        gain = torch.ones(D, dtype=torch.float32, device=dev)

        def dstep(i, xd=xd, wsd=wsd, outd=outd):
            svdmlp.svd_mlp(xd, *layers[i % len(layers)], workspace=wsd, out=outd)

        def bstep(i, xd=xd, wsd=wsd, outd=outd, gain=gain):
            svdmlp.svd_mlp_block(xd, gain, *layers[i % len(layers)], workspace=wsd, out=outd)

        msd, _ = _time_steps(torch, dstep, args.decode_steps, 10, stream)
        msb, _ = _time_steps(torch, bstep, args.decode_steps, 10, stream)
        with _lib.StageProfile() as prof:
            _time_steps(torch, dstep, 20, 0, stream)
        gbs = (nbytes_w + 2 * Td * D * 2) / (msd * 1e-3) / 1e9
        out[f"T={Td}"] = {"us_per_layer": round(msd * 1e3, 2), "GB/s": round(gbs, 1),
                          "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
                          "frac_measured_read": round(gbs / rates[1], 4),
                          "launches": {k: v[1] // 20 for k, v in prof.result.items()},
                          "block_us": round(msb * 1e3, 2)}
        if svdmlp.workspace_status(wsd):
            raise RuntimeError(f"two-rank decode T={Td}: a grid-barrier wait gave up (the device was shared?)")
    return out


# The reference's own standalone TPU launchers at its headline shape
# (results/kernel_optimizations_1_4_20260916/real_layer0_S128.json, TPU v5e,
# median host wall time of the optimized kernels): 8B factors, r=2816, S=128.
REF_TPU_US_S128 = {"fused_mlp_up_T": 503.6, "fused_three_mm_XTUV": 339.3, "svd_mlp_with_fused_kernel": 698.1}


def _bench_launchers(torch, dev, stream, args, layers, x, S=128):
    """compat.fused_mlp_up_T ((I, S) output) and compat.fused_three_mm_XTUV
    ((I, S) input) -- test_speedup.py:500-544 -- and their composition
    (test_speedup.py:631-655) on the 8B factors at S=128, timed back to back
    like the other lines (GPU only), with the factors rotating over the layers
    (1.25 GB) so that no call finds them in the memory-side cache; the
    reference's TPU figures beside them for context."""
    from svdmlp import compat

    xs = x[:S].contiguous()
    hT = compat.fused_mlp_up_T(xs, *layers[0][:4])
    out = {"S": S, "d": D, "ff": FF, "r": R, "layers_rotated": len(layers), "reference_tpu_us": REF_TPU_US_S128}
    n = len(layers)
    calls = {
        "fused_mlp_up_T": lambda i: compat.fused_mlp_up_T(xs, *layers[i % n][:4]),
        "fused_three_mm_XTUV": lambda i: compat.fused_three_mm_XTUV(hT, *layers[i % n][4:]),
        "svd_mlp_with_fused_kernel": lambda i: compat.svd_mlp_with_fused_kernel(
            xs, layers[i % n][2], layers[i % n][3], layers[i % n][0], layers[i % n][1], *layers[i % n][4:]),
    }
    flops = {"fused_mlp_up_T": 2.0 * S * 2 * R * (D + FF), "fused_three_mm_XTUV": 2.0 * S * R * (FF + D),
             "svd_mlp_with_fused_kernel": 2.0 * S * 3 * R * (D + FF)}
    for name, fn in calls.items():
        ms, _ = _time_steps(torch, fn, 100, 20, stream)
        out[name] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(flops[name] / (ms * 1e-3) / 1e12, 2)}
    return out


def _stack_inputs(torch, dev, args):
    from svdmlp import stack

    layers = stack.make_stack(args.stack_layers, D, FF, seed=args.seed + 4, device=dev)
    gx = torch.Generator(device=dev)
    gx.manual_seed(args.seed + 4000)
    x = torch.randn(args.stack_tokens, D, generator=gx, device=dev, dtype=torch.float32).to(torch.bfloat16)
    return layers, x


def _time_stack(torch, dev, stream, args, layers, x):
    """the 32-layer LLaMA3-8B MLP stack, x <- x +
    svd_mlp(RMSNorm(x) * gain) per layer, T=4096, per-branch ranks drawn from
    {2048, ..., 3072}, eps 1e-5, gains ~ U(0.9, 1.1) (GPU only)."""
    from svdmlp import stack

    T = x.shape[0]
    ws = stack.stack_workspace(x, layers)
    bufs = (torch.empty_like(x), torch.empty_like(x))
    ms, _ = _time_steps(torch, lambda i: stack.run_stack(x, layers, eps=1e-5, workspace=ws, buffers=bufs),
                        args.stack_steps, 1, stream)
    flops = stack.stack_flops(T, D, FF, layers)
    # FLOPs at the ranks the kernels run (each branch at its drawn rank: 0 padding)
    padded = sum(2 * T * ((l.factors[0].shape[1] + l.factors[2].shape[1]) * (D + FF) + l.factors[4].shape[1] * (FF + D))
                 for l in layers)
    tflops = flops / (ms * 1e-3) / 1e12
    return ws, {
        "workload": f"LLaMA3-8B MLP stack, {len(layers)} layers of RMSNorm + SVD-MLP + residual, non-uniform ranks",
        "T": T, "layers": len(layers), "ms_per_stack": round(ms, 3),
        "us_per_layer": round(ms * 1e3 / len(layers), 1), "TFLOP/s": round(tflops, 2),
        "pct_mfma_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "flop_per_stack": flops, "padded_flop_fraction": round(padded / flops - 1, 4),
        "ranks_first_layers": [l.ranks for l in layers[:4]],
    }


def _stack_parity(torch, args, layers, x, ws):
    """Rows are independent through the whole stack: on a row subset, each
    layer's block output against the oracle's block fed with the GPU's own
    input rows, and the whole chain against the unrounded float64 chain, for
    the GPU and for the oracle's own bf16 chain (two correct bf16 chains drift
    apart through the residual stream; a measured comparison, not a
    tolerance)."""
    import numpy as np

    import oracle as O
    from svdmlp import ops

    # rows spread evenly over the whole token range (first and last included)
    rows = min(max(args.parity_rows, 16), x.shape[0])
    idx = torch.linspace(0, x.shape[0] - 1, rows, device=x.device).round().long().unique()
    rows = int(idx.numel())
    bufs = (torch.empty_like(x), torch.empty_like(x))
    cur = x
    chain = x[idx].float().cpu().numpy()
    chain64 = chain.astype(np.float64)
    worst = 0.0
    first = None
    for i, l in enumerate(layers):
        out = ops.svd_mlp_block(cur, l.gain, *l.factors, eps=1e-5, workspace=ws, out=bufs[i % 2])
        xin, yout = cur[idx].float().cpu().numpy(), out[idx].float().cpu().numpy()
        f = [a.float().cpu().numpy() for a in l.factors]
        gain = l.gain.cpu().numpy()
        err = O.relative_l2(yout, O.mlp_block_ref(xin, gain, f, eps=1e-5, dtype="bfloat16"))
        worst = max(worst, err)
        first = err if first is None else first
        chain = O.mlp_block_ref(chain, gain, f, eps=1e-5, dtype="bfloat16")
        chain64 = O.mlp_block_f64(chain64, gain, f, eps=1e-5)
        cur = out
    got = cur[idx].float().cpu().numpy()
    exact = chain64.astype(np.float32)
    return {
        "parity_rows": rows,
        "parity_row_indices": [int(i) for i in idx.tolist()],
        "parity_rel_l2_first_layer": round(first, 6),
        "parity_rel_l2_worst_layer": round(worst, 6),
        "after_all_layers_rel_l2_gpu_vs_float64": round(O.relative_l2(got, exact), 6),
        "after_all_layers_rel_l2_oracle_bf16_vs_float64": round(O.relative_l2(chain, exact), 6),
        "after_all_layers_rel_l2_gpu_vs_oracle_bf16": round(O.relative_l2(got, chain), 6),
        "parity_note": "per layer: the GPU block vs the oracle block on the GPU's input rows; after all layers: "
                       "both bf16 chains against the unrounded float64 chain",
    }


def _fp8_inputs(torch, dev, args):
    from svdmlp import fp8

    T, d, ff, r = args.fp8_tokens, 8192, 28672, 5632
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed + 5)

    def q(rows, cols):
        w = torch.randn(rows, cols, generator=g, device=dev, dtype=torch.float32) / math.sqrt(rows)
        return fp8.quantize_per_channel(w)

    fs = [q(d, r), q(r, ff), q(d, r), q(r, ff), q(ff, r), q(r, d)]
    x = torch.randn(T, d, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    return fs, x


def _time_fp8(torch, dev, stream, args, fs, x):
    """the LLaMA3-70B-shape layer (T=2048, d=8192,
    ff=28672, r=5632) with fp8 e4m3fn factors and per-output-channel fp32
    scales (amax/448), bf16 activations, fp32 accumulation (GPU only)."""
    import svdmlp
    from svdmlp import _lib

    T, d = x.shape
    ff, r = fs[1].data.shape[1], fs[0].data.shape[1]
    ws = svdmlp.svd_mlp_workspace(x, r=r, ff=ff, w_code=2)
    out = torch.empty(T, d, dtype=torch.bfloat16, device=dev)
    run = lambda i: svdmlp.svd_mlp(x, *fs, workspace=ws, out=out)
    cold, _ = _time_steps(torch, run, 5, 1, stream)  # the section's first steps, clocks still ramping
    ms, _ = _time_steps(torch, run, args.fp8_steps, args.fp8_warmup, stream)
    flops = 2.0 * T * 3 * r * (d + ff)
    tflops = flops / (ms * 1e-3) / 1e12
    fbytes = sum(f.data.numel() + 4 * f.scale.numel() for f in fs)
    # SVDMLP_FP8_ACT: h quantised to e4m3 per token row, h . Ud on the fp8 MFMA
    out8 = torch.empty_like(out)
    ms8, _ = _time_steps(torch, lambda i: svdmlp.svd_mlp(x, *fs, workspace=ws, out=out8, fp8_activations=True),
                         args.fp8_steps, args.fp8_warmup, stream)
    stages = {}
    prof_steps = 2
    for name, kw in (("bf16_activations", {}), ("fp8_activations_h", {"fp8_activations": True})):
        with _lib.StageProfile() as prof:
            _time_steps(torch, lambda i: svdmlp.svd_mlp(x, *fs, workspace=ws, out=out8, **kw), prof_steps, 0, stream)
        # per layer: a stage may take more than one launch (the fp8 h.Ud's unsplit head and split tail)
        stages[name] = {k: round(v[0] / prof_steps * 1e3, 1) for k, v in prof.result.items()}
    tflops8 = flops / (ms8 * 1e-3) / 1e12
    return (out, out8), {
        "workload": "LLaMA3-70B-shape SVD-MLP layer, fp8 e4m3 factors with per-column scales, bf16 activations",
        "T": T, "d": d, "ff": ff, "r": r, "us_per_layer": round(ms * 1e3, 1), "TFLOP/s": round(tflops, 2),
        "cold_start_us_per_layer": round(cold * 1e3, 1),
        "steps": args.fp8_steps, "warmup": args.fp8_warmup,
        "pct_fp8_mfma_peak": round(100 * tflops / 5000.0, 2),
        "pct_bf16_mfma_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "compute": "factors widened exactly to bf16 in registers, bf16 MFMA (activations stay bf16: e4m3 "
                   "activations in more than one GEMM would exceed the 3e-2 tolerance, tests/test_fp8_budget.py)",
        "factor_bytes": fbytes,
        "stages_us_per_layer": stages,
        "fp8_activations_h": {
            "us_per_layer": round(ms8 * 1e3, 1), "TFLOP/s": round(tflops8, 2),
            "pct_fp8_mfma_peak": round(100 * tflops8 / 5000.0, 2),
            "compute": "SVDMLP_FP8_ACT: h quantised to e4m3 per token row (amax/448), h . Ud as fp8 x fp8 "
                       "v_mfma_scale_f32_16x16x128_f8f6f4 (unit block scales), fp32 accumulation; the other "
                       "GEMMs as above",
        },
    }


def _fp8_parity(args, fs, x, y):
    import numpy as np

    import oracle as O

    # 64 rows spread evenly over the token range (first and last included)
    idx = np.unique(np.linspace(0, x.shape[0] - 1, min(64, x.shape[0])).round().astype(np.int64))
    table = O.e4m3_decode(np.arange(256, dtype=np.uint8))
    deq = [table[f.data.view(__import__("torch").uint8).cpu().numpy()] * f.scale.cpu().numpy()[None, :] for f in fs]
    ref = O.svd_mlp_ref(x.float().cpu().numpy()[idx], *deq, dtype="bfloat16")
    y, y8 = y
    return {"parity_rows": int(idx.size),
            "parity_rel_l2_vs_oracle": round(O.relative_l2(y.float().cpu().numpy()[idx], ref), 6),
            "fp8_activations_h_parity_rel_l2_vs_oracle": round(O.relative_l2(y8.float().cpu().numpy()[idx], ref), 6)}


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
    pad_v = 64 if args.weights_layout == "padded" else 0
    layers = [_layer_weights(torch, dev, args.seed + i, linear, pad_v) for i in range(args.layers)]
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
    prefill = args.only in (None, "prefill")
    ws = svdmlp.svd_mlp_workspace(x, r=R, ff=FF)
    out = torch.empty(T, D, dtype=torch.bfloat16, device=dev)

    def step(i):
        svdmlp.svd_mlp(x, *layers[i % len(layers)], workspace=ws, out=out)

    # The prefill line is timed after the other GPU sections, with the clocks
    # at their steady state under load; the same W + K steps as the first GPU
    # work of the run (the GPU ramping up from idle) are reported beside it.
    cold = _time_steps(torch, step, args.steps, args.warmup, stream)[0] if prefill else None

    if args.only in (None, "decode"):
        record["decode"] = _bench_decode(torch, dev, stream, args, layers, x, factor_bytes)
        if args.weights_layout == "padded" and not args.no_decode_extra:
            # the dense natural-layout factors kernels/reference.py takes, at the
            # config-3 token counts, on the same box and HBM rates
            dense = [_layer_weights(torch, dev, args.seed + i) for i in range(args.layers)]
            rates = (record["decode"]["hbm_copy_GBps"], record["decode"]["hbm_read_GBps"])
            record["decode_dense"] = _bench_decode(torch, dev, stream, args, dense, x, factor_bytes,
                                                   tokens=[t for t in (1, 8, 32, 64) if t <= x.shape[0]],
                                                   rates=rates, layout="natural")
            if x.shape[0] >= 128:
                record["launchers_s128"] = _bench_launchers(torch, dev, stream, args, dense, x)
            del dense
            record["decode_two_ranks"] = _bench_decode_ranks(torch, dev, stream, args, x, rates)
    if args.only in (None, "stack"):
        s_layers, s_x = _stack_inputs(torch, dev, args)
        s_ws, record["stack"] = _time_stack(torch, dev, stream, args, s_layers, s_x)
    if args.only in (None, "fp8"):
        f_fs, f_x = _fp8_inputs(torch, dev, args)
        f_out, record["fp8_70b"] = _time_fp8(torch, dev, stream, args, f_fs, f_x)

    if prefill:
        ms, wall = _time_steps(torch, step, args.steps, args.warmup, stream)
        with _lib.StageProfile() as prof:
            ms_prof, _ = _time_steps(torch, step, args.steps, 0, stream)
        stages = {k: v[0] / v[1] for k, v in prof.result.items()}
        # per-step distribution: each step between its own pair of events
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
        for i, (e0, e1) in enumerate(evs):
            e0.record(stream)
            step(i)
            e1.record(stream)
        torch.cuda.synchronize()
        per_step = sorted(e0.elapsed_time(e1) * 1e3 for e0, e1 in evs)
        pct = lambda q: per_step[min(len(per_step) - 1, int(q * (len(per_step) - 1) + 0.5))]
        # Each GEMM stage is one kernel launch; the roofline line is for the
        # one with the most time per layer.
        stage_work = _stage_work(T)
        gemm_stages = {k: v for k, v in stages.items() if k in stage_work}
        dom = max(gemm_stages, key=gemm_stages.get) if gemm_stages else None
        dom_ms = gemm_stages.get(dom)
        dom_flops, dom_bytes, dom_desc = stage_work.get(dom, (None, None, None))
        achieved = dom_flops / (dom_ms * 1e-3) / 1e12 if dom_ms else None
        tflops = flops / (ms * 1e-3) / 1e12
        profiled = (T, args.weights_layout) == (1024, TRAFFIC_LAYOUT)
        busy = _profiled("mfma_busy", dom, MFMA_PROFILE) if profiled and dom else None
        clock = _profiled("shader_clock_ghz", dom, MFMA_PROFILE) if profiled and dom else None
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
            "cold_start": {"ms_per_step": round(cold, 4), "us_per_layer": round(cold * 1e3, 1),
                           "note": "the same warmup and timed steps as the first GPU work of the run"},
            "roofline": {
                "kernel": f"{dom}: {dom_desc}" if dom else None,
                "bound": "mfma",
                "achieved": round(achieved, 2) if achieved else None,
                "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_BF16_TFLOPS, 4) if achieved else None,
                "traffic": _profiled_traffic(dom) if profiled else None,
                "traffic_source": "profiles/prefill_8b_T1024_traffic.md: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE "
                                  "per dispatch, calibrated on a 256 MiB copy",
                "mfma_busy": busy,
                "shader_clock_ghz": clock,
                "mfma_source": "profiles/prefill_8b_T1024_mfma.md: rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES, "
                               "SQ_BUSY_CYCLES; MFMA-busy share of the SIMD cycles at the measured shader clock",
                "algorithmic_flop_per_launch": dom_flops,
                "algorithmic_bytes_per_launch": dom_bytes,
                "avg_launch_us": round(dom_ms * 1e3, 2) if dom_ms else None,
            },
            "stages_us": {k: round(v * 1e3, 2) for k, v in stages.items()},
            # per layer: a stage may take more than one launch per layer (the split-K reductions, "finalize")
            "stages_us_per_layer": {k: round(v[0] / args.steps * 1e3, 2) for k, v in prof.result.items()},
            "ms_per_step_with_stage_events": round(ms_prof, 4),
            "step_us_p10_p50_p90": [round(pct(0.1), 1), round(pct(0.5), 1), round(pct(0.9), 1)],
        })

    # CPU work last (the oracle is the checker only; nothing below is timed
    # on the GPU)
    if prefill and not args.no_cpu_baseline:
        base, y_ref = _cpu_baseline(layers[0], x, T, args.cpu_seconds)
        y = svdmlp.svd_mlp(x, *layers[0], workspace=ws, out=out)
        import oracle as O

        got = y[: y_ref.shape[0]].float().cpu().numpy()
        record["parity_rel_l2_vs_oracle"] = round(O.relative_l2(got, y_ref), 6)
        record["cpu_baseline"] = base
    if args.only in (None, "stack"):
        record["stack"].update(_stack_parity(torch, args, s_layers, s_x, s_ws))
    if args.only in (None, "fp8"):
        record["fp8_70b"].update(_fp8_parity(args, f_fs, f_x, f_out))
    if args.only == "decode":
        t1 = record["decode"].get("T=1") or next(v for v in record["decode"].values() if isinstance(v, dict))
        record.update({"metric": METRIC, "value": t1["GB/s"], "unit": "GB/s", "n_gpus": 1,
                       "steps": args.decode_steps, "warmup": max(10, args.warmup), "ms_per_step": t1["us_per_layer"] / 1e3,
                       "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
                       "data": "synthetic", "config": {"workload": "LLaMA3-8B SVD-MLP layer, decode"}})
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
