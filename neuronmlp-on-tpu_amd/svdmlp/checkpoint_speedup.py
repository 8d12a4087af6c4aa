"""Per-layer measurements on a real SVD checkpoint (bench/checkpoint_speedup.py:1-222,
the ``--model-path`` branch of test_speedup.py:752-835), on MI355X.

Layers share one seeded synthetic input and never each other's output; only
one layer's factors are on the device at a time.  For every (layer, T):

* ``fused``: ``svdmlp.compat.svd_mlp_with_fused_kernel`` (the HIP layer);
* ``unfused_low_rank``: the vendor arm, torch/hipBLASLt GEMMs at the input
  dtype (test_speedup.py:690-696);
* ``reference``: the fp32 arm (test_speedup.py:681-687);

errors of both arms against the fp32 arm (relative L2, max abs error,
reference RMS; NaN/Inf rejected), medians of hipEvent-timed calls and a
summary per T as the ratio of summed layer medians.  The report (JSON and a
sibling CSV) keeps the reference's keys.

    python -m svdmlp.checkpoint_speedup --model-path CKPT --layers 0 1 --seq-lens 1 128 512 --output out.json
"""

from __future__ import annotations

import argparse
import csv
import json
import statistics
import sys
import time
from pathlib import Path

import numpy as np


def _errors(actual, expected) -> dict:
    actual = np.asarray(actual, dtype=np.float32)
    expected = np.asarray(expected, dtype=np.float32)
    if actual.shape != expected.shape:
        raise ValueError(f"output shape mismatch: {actual.shape} != {expected.shape}")
    if not np.isfinite(actual).all() or not np.isfinite(expected).all():
        raise FloatingPointError("MLP output or reference contains NaN/Inf")
    diff = actual - expected
    return {
        "relative_l2": float(np.linalg.norm(diff) / max(np.linalg.norm(expected), 1e-12)),
        "max_abs_error": float(np.max(np.abs(diff))),
        "reference_rms": float(np.sqrt(np.mean(expected ** 2))),
    }


def summarize(records, selected_layers, seq_lens) -> list[dict]:
    """Per T: completeness, pass state and the ratio of summed layer medians
    (not the mean of per-layer speedups), bench/checkpoint_speedup.py:35-55."""
    out = []
    for S in seq_lens:
        rows = [r for r in records if r["S"] == S]
        complete = len(rows) == len(selected_layers) and {r["layer"] for r in rows} == set(selected_layers)
        passed = complete and all(r["passed"] for r in rows)
        res = {"S": S, "layers_completed": len(rows), "layers_expected": len(selected_layers), "complete": complete,
               "passed": passed, "failed_layers": [r["layer"] for r in rows if not r["passed"]]}
        if rows:
            res["max_fused_relative_l2"] = max(r["fused_vs_fp32"]["relative_l2"] for r in rows)
        if passed and all("fused_ms" in r and "unfused_low_rank_ms" in r for r in rows):
            fused = sum(r["fused_ms"] for r in rows)
            unfused = sum(r["unfused_low_rank_ms"] for r in rows)
            res.update(fused_ms_sum=fused, unfused_low_rank_ms_sum=unfused, speedup_vs_unfused=unfused / fused)
        out.append(res)
    return out


def _save_report(report, path) -> None:
    if not path:
        return
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(json.dumps(report, indent=2, allow_nan=False), encoding="utf-8")
    columns = ("layer", "S", "rank", "dtype", "down_backend", "passed", "fused_ms", "unfused_low_rank_ms",
               "speedup_vs_unfused", "fused_relative_l2", "unfused_relative_l2", "max_abs_error")
    with path.with_suffix(".csv").open("w", newline="", encoding="utf-8") as handle:
        writer = csv.DictWriter(handle, fieldnames=columns)
        writer.writeheader()
        for rec in report["records"]:
            row = {k: rec[k] for k in columns if k in rec}
            row.update(fused_relative_l2=rec["fused_vs_fp32"]["relative_l2"],
                       unfused_relative_l2=rec["unfused_vs_fp32"]["relative_l2"],
                       max_abs_error=rec["fused_vs_fp32"]["max_abs_error"])
            writer.writerow(row)


def _time_ms(torch, fn, args, warmup, repeats) -> float:
    """Median of hipEvent-timed calls after one untimed call and `warmup`
    more (test_speedup.py:739-749 times each call after waiting for it)."""
    stream = torch.cuda.current_stream()
    fn(*args)
    for _ in range(warmup):
        fn(*args)
    torch.cuda.synchronize()
    samples = []
    for _ in range(repeats):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn(*args)
        b.record(stream)
        b.synchronize()
        samples.append(a.elapsed_time(b))
    return statistics.median(samples)


def run(args) -> dict:
    """The per-layer loop of bench/checkpoint_speedup.py:75-222."""
    from . import checkpoint, compat

    metadata = checkpoint.inspect_mlp_checkpoint(args.model_path, args.layers)
    if len(set(args.seq_lens)) != len(args.seq_lens):
        raise ValueError("sequence lengths must not contain duplicates")
    if args.input_scale <= 0 or not np.isfinite(args.input_scale):
        raise ValueError("input-scale must be finite and positive")
    if args.max_relative_l2 is not None and (args.max_relative_l2 <= 0 or not np.isfinite(args.max_relative_l2)):
        raise ValueError("max-relative-l2 must be finite and positive")
    mode = "checkpoint_inspection" if args.inspect_only else ("gpu_correctness_only" if args.check_only else
                                                              "gpu_benchmark")
    report = {
        "mode": mode, "complete": False, "down_backend": args.down_backend, "checkpoint": metadata,
        "seq_lens": args.seq_lens,
        "input": {"kind": "synthetic_standard_normal", "scale": args.input_scale, "seed": args.seed,
                  "shared_across_layers": True, "chain_layers": False},
        "requested_dtype": args.dtype or "checkpoint",
        "timing": {"statistic": "median_ms", "warmup": args.warmup, "repeats": args.repeats,
                   "load_and_compile_included": False,
                   "aggregation": "sum_unfused_layer_medians / sum_fused_layer_medians"},
        "records": [], "summaries": [],
    }
    H, I = metadata["hidden_size"], metadata["intermediate_size"]
    print(json.dumps({"checkpoint": metadata["model_path"], "shards": len(metadata["shards"]),
                      "selected_layers": metadata["selected_layers"], "H": H, "I": I,
                      "ranks": sorted({row["rank"] for row in metadata["layers"]}), "mode": mode}), flush=True)
    if args.inspect_only:
        report["complete"] = True
        _save_report(report, args.output)
        return report

    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("real-checkpoint runs need the GPU; use --inspect-only on a host without one")
    dev = torch.device("cuda:0")
    report["devices"] = [torch.cuda.get_device_name(dev)]
    _save_report(report, args.output)
    rng = np.random.default_rng(args.seed)
    inputs = {S: rng.normal(size=(S, H)).astype(np.float32) * args.input_scale for S in args.seq_lens}

    for info in metadata["layers"]:
        layer = info["layer"]
        print(f"Layer {layer}: loading six SVD factors (rank={info['rank']})...", flush=True)
        want = None if args.dtype is None else (torch.bfloat16 if args.dtype == "bf16" else torch.float32)
        (loaded,) = checkpoint.load_mlp_factors(args.model_path, [layer], device=dev, dtype=want)
        ug, vg, uu, vu, ud, vd = loaded
        factors = (uu, vu, ug, vg, ud, vd)  # test_speedup.py order: up, gate, down
        dtype = ug.dtype
        for S in args.seq_lens:
            mixed = dtype == torch.bfloat16
            tolerance = args.max_relative_l2 or (0.12 if mixed else 0.001)
            x = torch.from_numpy(inputs[S]).to(dev).to(dtype)
            call = (x, *factors)

            def fused(*a):
                return compat.svd_mlp_with_fused_kernel(*a, mixed_precision=mixed, down_backend=args.down_backend)

            started = time.perf_counter()
            expected = compat._unfused_reference(*call).float().cpu().numpy()
            unfused_out = compat._unfused_low_rank(*call).float().cpu().numpy()
            fused_out = fused(*call).float().cpu().numpy()
            fused_err, unfused_err = _errors(fused_out, expected), _errors(unfused_out, expected)
            passed = fused_err["relative_l2"] <= tolerance and unfused_err["relative_l2"] <= tolerance
            rec = {"layer": layer, "S": S, "rank": info["rank"], "dtype": str(dtype).replace("torch.", ""),
                   "down_backend": args.down_backend, "fused_vs_fp32": fused_err, "unfused_vs_fp32": unfused_err,
                   "fused_vs_unfused": _errors(fused_out, unfused_out), "max_relative_l2": tolerance,
                   "passed": passed, "compile_and_verify_seconds": time.perf_counter() - started}
            if passed and not args.check_only:
                jobs = [("fused_ms", fused), ("unfused_low_rank_ms", compat._unfused_low_rank)]
                if layer % 2:  # alternate the order between layers to reduce systematic bias
                    jobs.reverse()
                for name, fn in jobs:
                    rec[name] = _time_ms(torch, fn, call, args.warmup, args.repeats)
                rec["speedup_vs_unfused"] = rec["unfused_low_rank_ms"] / rec["fused_ms"]
            report["records"].append(rec)
            report["summaries"] = summarize(report["records"], metadata["selected_layers"], args.seq_lens)
            _save_report(report, args.output)
            print(json.dumps(rec, allow_nan=False), flush=True)
            del x, call
        del loaded, factors, ug, vg, uu, vu, ud, vd
    report["complete"] = True
    _save_report(report, args.output)
    for summary in report["summaries"]:
        print(json.dumps({"summary": summary}), flush=True)
    if not all(r["passed"] for r in report["records"]):
        raise RuntimeError("some layers failed numerical verification; see the saved per-layer report")
    return report


def _parser() -> argparse.ArgumentParser:
    """The flags of test_speedup.py:752-774 that the --model-path branch uses."""
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
