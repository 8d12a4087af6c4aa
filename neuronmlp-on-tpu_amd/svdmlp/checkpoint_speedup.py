"""Per-layer verification and timing on an SVD checkpoint: the ``--model-path``
mode of the reference's synthetic benchmark (test_speedup.py:752-835, with its
runner bench/checkpoint_speedup.py), on MI355X.

Each selected layer is loaded alone, run on a seeded synthetic input that all
layers share (a layer never sees another layer's output), and compared in
three arms:

* ``fused``: ``compat.svd_mlp_with_fused_kernel`` (the HIP layer);
* ``unfused_low_rank``: torch/hipBLASLt GEMMs at the input dtype
  (test_speedup.py:690-696);
* the fp32 arm (test_speedup.py:681-687), the reference for both.

A record per (layer, S) holds both arms' errors against the fp32 arm
(relative L2, max abs error, reference RMS; a NaN or Inf fails loudly), the
pass verdict and, when it passed, the median per-call time of each arm.  The
two arms are sampled alternately, call by call, so clock drift and cache
state weigh on both alike.  Per S, a summary divides the summed unfused
medians by the summed fused ones.  The report is rewritten after every record
(JSON, plus a CSV next to it) with the reference's keys, so a partial run
leaves a readable report marked incomplete.

    python -m svdmlp.checkpoint_speedup --model-path CKPT --layers 0 1 --seq-lens 1 128 512 --output out.json
"""

from __future__ import annotations

import argparse
import csv
import json
import math
import statistics
import sys
import time
from pathlib import Path

import numpy as np

CSV_COLUMNS = ("layer", "S", "rank", "dtype", "down_backend", "passed", "fused_ms", "unfused_low_rank_ms",
               "speedup_vs_unfused", "fused_relative_l2", "unfused_relative_l2", "max_abs_error")


def _errors(actual, expected) -> dict:
    """Relative L2 (norm of the difference over the reference norm, floored at
    1e-12), max abs error and reference RMS, in float64 (the metric of
    bench/checkpoint_speedup.py:20-31).  NaN/Inf -> FloatingPointError."""
    import torch

    a = torch.as_tensor(actual).double()
    e = torch.as_tensor(expected).double().to(a.device)
    if a.shape != e.shape:
        raise ValueError(f"output shape mismatch: {tuple(a.shape)} != {tuple(e.shape)}")
    if not (bool(torch.isfinite(a).all()) and bool(torch.isfinite(e).all())):
        raise FloatingPointError("MLP output or reference contains NaN/Inf")
    d = a - e
    return {"relative_l2": float(d.norm() / max(float(e.norm()), 1e-12)),
            "max_abs_error": float(d.abs().max()) if d.numel() else 0.0,
            "reference_rms": float(e.pow(2).mean().sqrt()) if e.numel() else 0.0}


def summarize(records, selected_layers, seq_lens) -> list[dict]:
    """One summary per S: how many of the selected layers have a record, whether
    all passed, the worst fused error, and (when every layer was timed) the
    speedup as a ratio of summed medians (bench/checkpoint_speedup.py:34-53)."""
    want = set(selected_layers)
    out = []
    for S in seq_lens:
        rows = [r for r in records if r["S"] == S]
        have = {r["layer"] for r in rows}
        summary = {"S": S, "layers_completed": len(rows), "layers_expected": len(selected_layers),
                   "complete": len(rows) == len(selected_layers) and have == want}
        summary["passed"] = summary["complete"] and all(r["passed"] for r in rows)
        summary["failed_layers"] = [r["layer"] for r in rows if not r["passed"]]
        if rows:
            summary["max_fused_relative_l2"] = max(r["fused_vs_fp32"]["relative_l2"] for r in rows)
        timed = [r for r in rows if "fused_ms" in r and "unfused_low_rank_ms" in r]
        if summary["passed"] and len(timed) == len(rows):
            f = math.fsum(r["fused_ms"] for r in timed)
            u = math.fsum(r["unfused_low_rank_ms"] for r in timed)
            summary.update(fused_ms_sum=f, unfused_low_rank_ms_sum=u, speedup_vs_unfused=u / f)
        out.append(summary)
    return out


class RunReport:
    """The report of one run: header fields, records, summaries; written to
    ``path`` (JSON) and ``path`` with a .csv suffix after every change."""

    def __init__(self, path, header: dict, selected_layers, seq_lens):
        self.path = Path(path) if path else None
        self.data = dict(header, complete=False, records=[], summaries=[])
        self.layers, self.seq_lens = list(selected_layers), list(seq_lens)

    def add(self, record: dict) -> None:
        self.data["records"].append(record)
        self.data["summaries"] = summarize(self.data["records"], self.layers, self.seq_lens)
        self.save()

    def finish(self) -> dict:
        self.data["complete"] = True
        self.save()
        return self.data

    def save(self) -> None:
        if self.path is None:
            return
        self.path.parent.mkdir(parents=True, exist_ok=True)
        self.path.write_text(json.dumps(self.data, indent=2, allow_nan=False), encoding="utf-8")
        with self.path.with_suffix(".csv").open("w", newline="", encoding="utf-8") as fh:
            w = csv.writer(fh)
            w.writerow(CSV_COLUMNS)
            for r in self.data["records"]:
                extra = {"fused_relative_l2": r["fused_vs_fp32"]["relative_l2"],
                         "unfused_relative_l2": r["unfused_vs_fp32"]["relative_l2"],
                         "max_abs_error": r["fused_vs_fp32"]["max_abs_error"]}
                w.writerow([extra.get(c, r.get(c, "")) for c in CSV_COLUMNS])


def _sample_alternately(torch, arms: dict, args: tuple, warmup: int, repeats: int) -> dict:
    """Median milliseconds per call of each arm.  After ``warmup`` untimed
    rounds, every round times one call of each arm (hipEvents on the current
    stream, each call waited for, as test_speedup.py:739-749 times a call),
    the arms in turn, so that both see the same clocks and caches."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup + 1):
        for fn in arms.values():
            fn(*args)
    torch.cuda.synchronize()
    samples = {name: [] for name in arms}
    for _ in range(repeats):
        for name, fn in arms.items():
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            fn(*args)
            stop.record(stream)
            stop.synchronize()
            samples[name].append(start.elapsed_time(stop))
    return {name: statistics.median(v) for name, v in samples.items()}


def _check_args(args) -> None:
    if len(set(args.seq_lens)) != len(args.seq_lens):
        raise ValueError("sequence lengths must not contain duplicates")
    for name, value in (("input-scale", args.input_scale), ("max-relative-l2", args.max_relative_l2)):
        if value is not None and not (np.isfinite(value) and value > 0):
            raise ValueError(f"{name} must be finite and positive")


def run(args) -> dict:
    """Inspect the checkpoint, then verify and time every (layer, S)."""
    from . import checkpoint, compat

    meta = checkpoint.inspect_mlp_checkpoint(args.model_path, args.layers)
    _check_args(args)
    mode = ("checkpoint_inspection" if args.inspect_only else
            "gpu_correctness_only" if args.check_only else "gpu_benchmark")
    report = RunReport(args.output, {
        "mode": mode, "down_backend": args.down_backend, "checkpoint": meta, "seq_lens": args.seq_lens,
        "input": {"kind": "synthetic_standard_normal", "scale": args.input_scale, "seed": args.seed,
                  "shared_across_layers": True, "chain_layers": False},
        "requested_dtype": args.dtype or "checkpoint",
        "timing": {"statistic": "median_ms", "warmup": args.warmup, "repeats": args.repeats,
                   "load_and_compile_included": False, "sampling": "arms alternated call by call",
                   "aggregation": "sum_unfused_layer_medians / sum_fused_layer_medians"},
    }, meta["selected_layers"], args.seq_lens)
    print(json.dumps({"checkpoint": meta["model_path"], "shards": len(meta["shards"]),
                      "selected_layers": meta["selected_layers"], "H": meta["hidden_size"],
                      "I": meta["intermediate_size"], "ranks": sorted({l["rank"] for l in meta["layers"]}),
                      "mode": mode}), flush=True)
    if args.inspect_only:
        return report.finish()

    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("real-checkpoint runs need the GPU; use --inspect-only on a host without one")
    dev = torch.device("cuda:0")
    report.data["devices"] = [torch.cuda.get_device_name(dev)]
    report.save()
    draw = np.random.default_rng(args.seed)
    xs = {S: draw.normal(size=(S, meta["hidden_size"])).astype(np.float32) * args.input_scale for S in args.seq_lens}
    cast = {None: None, "bf16": torch.bfloat16, "fp32": torch.float32}[args.dtype]

    for info in meta["layers"]:
        print(f"Layer {info['layer']}: loading six SVD factors (rank={info['rank']})...", flush=True)
        ug, vg, uu, vu, ud, vd = checkpoint.load_mlp_factors(args.model_path, [info["layer"]], device=dev,
                                                             dtype=cast)[0]
        up_first = (uu, vu, ug, vg, ud, vd)   # the argument order of test_speedup.py's arms
        dtype = ug.dtype
        bf16 = dtype == torch.bfloat16
        arms = {
            "fused_ms": lambda x, *f: compat.svd_mlp_with_fused_kernel(x, *f, mixed_precision=bf16,
                                                                       down_backend=args.down_backend),
            "unfused_low_rank_ms": compat._unfused_low_rank,
        }
        for S in args.seq_lens:
            limit = args.max_relative_l2 or (0.12 if bf16 else 0.001)
            call = (torch.from_numpy(xs[S]).to(dev).to(dtype), *up_first)
            t0 = time.perf_counter()
            gold = compat._unfused_reference(*call).float()
            outs = {name: fn(*call).float() for name, fn in arms.items()}
            err_f, err_u = _errors(outs["fused_ms"], gold), _errors(outs["unfused_low_rank_ms"], gold)
            rec = {"layer": info["layer"], "S": S, "rank": info["rank"], "dtype": str(dtype).split(".")[-1],
                   "down_backend": args.down_backend, "fused_vs_fp32": err_f, "unfused_vs_fp32": err_u,
                   "fused_vs_unfused": _errors(outs["fused_ms"], outs["unfused_low_rank_ms"]),
                   "max_relative_l2": limit,
                   "passed": err_f["relative_l2"] <= limit and err_u["relative_l2"] <= limit,
                   "compile_and_verify_seconds": time.perf_counter() - t0}
            if rec["passed"] and not args.check_only:
                rec.update(_sample_alternately(torch, arms, call, args.warmup, args.repeats))
                rec["speedup_vs_unfused"] = rec["unfused_low_rank_ms"] / rec["fused_ms"]
            report.add(rec)
            print(json.dumps(rec, allow_nan=False), flush=True)
        del ug, vg, uu, vu, ud, vd, up_first
    data = report.finish()
    for summary in data["summaries"]:
        print(json.dumps({"summary": summary}), flush=True)
    failed = [(r["layer"], r["S"]) for r in data["records"] if not r["passed"]]
    if failed:
        raise RuntimeError(f"numerical verification failed for (layer, S) {failed}; the report lists every record")
    return data


def _parser() -> argparse.ArgumentParser:
    """The flags of test_speedup.py:752-774 that its --model-path mode uses."""
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--model-path", required=True, help="offline SVD checkpoint directory; test real layers")
    p.add_argument("--layers", type=int, nargs="+", help="layer indices; defaults to all checkpoint layers")
    p.add_argument("--output", help="real-layer JSON report path; also writes a sibling CSV")
    p.add_argument("--inspect-only", action="store_true", help="validate checkpoint headers without loading tensors")
    p.add_argument("--input-scale", type=float, default=1.0)
    p.add_argument("--max-relative-l2", type=float)
    p.add_argument("--seq-lens", type=int, nargs="+", default=[1, 128, 512])
    p.add_argument("--dtype", choices=("bf16", "fp32"), help="defaults to the checkpoint dtype")
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--repeats", type=int, default=10)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--check-only", action="store_true")
    p.add_argument("--down-backend", choices=("pallas", "jax"), default="pallas",
                   help="'pallas': the fused HIP layer; 'jax': HIP Gate/Up then the vendor Down")
    return p


def main(argv=None) -> int:
    run(_parser().parse_args(argv))
    return 0


if __name__ == "__main__":
    sys.exit(main())
