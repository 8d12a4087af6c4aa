"""Three-way SVD-MLP benchmark on synthetic factors (the synthetic branch of
test_speedup.py:752-900), on MI355X.

For every sequence length S, on one seeded set of factors:

* ``fused``: ``compat.svd_mlp_with_fused_kernel`` (the HIP layer, or HIP
  Gate/Up plus the vendor Down with ``--down-backend jax``);
* ``dense``: ``compat.nki_baseline`` on the dense weights rebuilt as
  (U.V)^T in fp32 outside the timing (test_speedup.py:818-821);
* ``unfused``: ``compat._unfused_low_rank_pallas``, six plain GEMMs;

the fused output is checked against the fp32 arm ``compat._unfused_reference``
(relative L2 <= 0.12 for bf16, 1e-3 for fp32, as the reference) before
anything is timed.  Records keep the reference's keys (``S``, ``relative_l2``,
``max_abs_error``, ``fused_ms``, ``dense_ms``, ``unfused_low_rank_ms``,
``speedup_vs_dense``, ``speedup_vs_unfused`` ...); times are medians of
hipEvent-timed calls.  The dense and unfused arms run on the vendor library
(hipBLASLt): they are comparison arms, not part of the SVD-MLP path.

``--model-path`` runs the per-layer real-checkpoint runner instead
(:mod:`svdmlp.checkpoint_speedup`), as the reference does.

    python -m svdmlp.speedup --model llama3-8b --seq-lens 1 128 512 1024
"""

from __future__ import annotations

import argparse
import json
import math
import sys

import numpy as np

_BASE = {"llama3-3b": (3072, 8192, 1792), "llama3-8b": (4096, 14336, 2560)}


def _parser() -> argparse.ArgumentParser:
    """The flags of test_speedup.py:752-774."""
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--model-path", help="offline SVD checkpoint directory; test real layers")
    p.add_argument("--layers", type=int, nargs="+", help="layer indices; defaults to all checkpoint layers")
    p.add_argument("--output", help="real-layer JSON report path; also writes a sibling CSV")
    p.add_argument("--inspect-only", action="store_true", help="validate real checkpoint headers without loading tensors")
    p.add_argument("--input-scale", type=float, default=1.0)
    p.add_argument("--max-relative-l2", type=float)
    p.add_argument("--model", choices=tuple(_BASE), default="llama3-3b")
    p.add_argument("--seq-lens", type=int, nargs="+", default=[1, 128, 512])
    p.add_argument("--hidden", type=int)
    p.add_argument("--intermediate", type=int)
    p.add_argument("--rank", type=int)
    p.add_argument("--dtype", choices=("bf16", "fp32"), help="defaults to checkpoint dtype, or bf16 for synthetic tests")
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--repeats", type=int, default=10)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--interpret", action="store_true", help="the Pallas CPU emulator: no MI355X counterpart")
    p.add_argument("--check-only", action="store_true")
    p.add_argument("--down-backend", choices=("pallas", "jax"), default="pallas",
                   help="'pallas': the fused HIP layer; 'jax': HIP Gate/Up then the vendor Down")
    p.add_argument("--sync-dma", action="store_true", help="accepted; the HIP kernels always prefetch")
    p.add_argument("--profile-dir", default=None, help="not supported: profile with rocprofv3 --kernel-trace")
    return p


def synthetic_factors(rng, H: int, I: int, R: int):
    """Factors in the reference's draw order uu, vu, ug, vg, ud, vd, each
    N(0, 1/rows) (test_speedup.py:810-815), as float32 numpy arrays."""
    def random_matrix(rows, cols):
        return rng.normal(size=(rows, cols)).astype(np.float32) / math.sqrt(rows)
    return (random_matrix(H, R), random_matrix(R, I), random_matrix(H, R), random_matrix(R, I),
            random_matrix(I, R), random_matrix(R, H))


def _time_ms(torch, fn, args, warmup: int, repeats: int) -> float:
    """Median hipEvent time of single calls (each call waited for, as
    test_speedup.py:739-749 times a call), after warmup calls."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup + 1):
        fn(*args)
    torch.cuda.synchronize()
    times = []
    for _ in range(repeats):
        begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        begin.record(stream)
        fn(*args)
        end.record(stream)
        end.synchronize()
        times.append(begin.elapsed_time(end))
    times.sort()
    return times[len(times) // 2] if len(times) % 2 else 0.5 * (times[len(times) // 2 - 1] + times[len(times) // 2])


def run(args) -> list[dict]:
    from . import compat

    if args.warmup < 0 or args.repeats <= 0:
        raise ValueError("warmup must be >= 0 and repeats must be > 0")
    for s in args.seq_lens:
        compat._positive("sequence length", s)
    if args.model_path:
        if any(v is not None for v in (args.hidden, args.intermediate, args.rank)):
            raise ValueError("real-checkpoint dimensions come from the tensors; omit --hidden/--intermediate/--rank")
        from . import checkpoint_speedup
        return checkpoint_speedup.run(args)["records"]
    if args.layers is not None or args.inspect_only or args.output or args.max_relative_l2 is not None:
        raise ValueError("--layers/--inspect-only/--output/--max-relative-l2 require --model-path")
    if args.interpret:
        raise ValueError("--interpret (the Pallas CPU emulator) has no MI355X counterpart")
    if args.profile_dir is not None:
        raise ValueError("--profile-dir is not supported; run under rocprofv3 --kernel-trace --stats instead")

    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("the benchmark needs the GPU")
    dev = torch.device("cuda:0")
    dtype_name = args.dtype or "bf16"
    dtype = torch.bfloat16 if dtype_name == "bf16" else torch.float32
    mixed = dtype_name == "bf16"
    H, I, R = (v if v is not None else d for v, d in zip((args.hidden, args.intermediate, args.rank), _BASE[args.model]))
    for name, value in zip(("hidden", "intermediate", "rank"), (H, I, R)):
        compat._positive(name, value)
    rng = np.random.default_rng(args.seed)
    host = synthetic_factors(rng, H, I, R)
    factors = tuple(torch.from_numpy(f).to(dev).to(dtype) for f in host)
    uu, vu, ug, vg, ud, vd = factors
    weights = tuple((u.float() @ v.float()).to(dtype).t().contiguous() for u, v in ((uu, vu), (ug, vg), (ud, vd)))
    print(json.dumps({"torch": torch.__version__, "devices": [torch.cuda.get_device_name(dev)], "mode": "gpu",
                      "shape": {"H": H, "I": I, "R": R}, "dtype": dtype_name, "down_backend": args.down_backend}),
          flush=True)
    records = []
    for S in args.seq_lens:
        x = torch.from_numpy(rng.normal(size=(S, H)).astype(np.float32)).to(dev).to(dtype)
        up_params = compat.get_fused_mlp_up_T_params(S)
        down_params = compat.get_fused_three_mm_XTUV_params(S)

        def fused(x, *f):
            return compat.svd_mlp_with_fused_kernel(x, *f, up_params, down_params, mixed_precision=mixed,
                                                    async_dma=not args.sync_dma, down_backend=args.down_backend)

        def dense(x, *w):
            return compat.nki_baseline(x, *w, mixed_precision=mixed)

        def unfused(x, *f):
            return compat._unfused_low_rank_pallas(x, *f, mixed_precision=mixed)

        call_args = (x, *factors)
        expected = compat._unfused_reference(*call_args).cpu().numpy()
        got = fused(*call_args).float().cpu().numpy()
        if not np.isfinite(got).all():
            raise AssertionError("fused output contains NaN/Inf")
        rel_l2 = float(np.linalg.norm(got - expected) / max(np.linalg.norm(expected), 1e-12))
        tolerance = 0.12 if mixed else 0.001
        if rel_l2 > tolerance:
            raise AssertionError(f"S={S}: relative L2 error {rel_l2:.6g} > {tolerance}")
        record = {"S": S, "async_dma": not args.sync_dma, "down_backend": args.down_backend,
                  "up_params": up_params, "down_params": down_params if args.down_backend == "pallas" else None,
                  "relative_l2": rel_l2, "max_abs_error": float(np.max(np.abs(got - expected)))}
        if not args.check_only:
            print(f"S={S}: correctness passed; timing the dense and unfused baselines.", flush=True)
            fused_ms = _time_ms(torch, fused, call_args, args.warmup, args.repeats)
            dense_ms = _time_ms(torch, dense, (x, *weights), args.warmup, args.repeats)
            unfused_ms = _time_ms(torch, unfused, call_args, args.warmup, args.repeats)
            record.update(fused_ms=fused_ms, dense_ms=dense_ms, unfused_low_rank_ms=unfused_ms,
                          speedup_vs_dense=dense_ms / fused_ms, speedup_vs_unfused=unfused_ms / fused_ms)
        records.append(record)
        print(json.dumps(record), flush=True)
    return records


def main(argv=None) -> int:
    parser = _parser()
    args = parser.parse_args(argv)
    try:
        run(args)
    except ValueError as exc:
        parser.error(str(exc))
    return 0


if __name__ == "__main__":
    sys.exit(main())
