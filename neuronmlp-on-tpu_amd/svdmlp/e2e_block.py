"""Whole-model N-layer transformer prefill: fused SVD MLP vs unfused SVD MLP
(bench/e2e_block.py:1-439), on MI355X.

Every layer is RMSNorm -> GQA attention -> residual -> RMSNorm -> MLP ->
residual (bench/e2e_block.py:229-278), with RMSNorm eps 1e-6 and the
reference's synthetic weights (unit norm gains, N(0, 1/fan_in) projections,
X ~ 0.02 N(0, 1)).  The arms differ only in how the SVD MLP runs:

* ``fused_block``: the library's block entry point ``ops.svd_mlp_block``
  (RMSNorm, the fused SVD-MLP layer and the residual add, all HIP kernels);
* ``unfused_block``: RMSNorm and six plain GEMMs with an fp32 SiLU
  (``compat._unfused_low_rank_pallas``, the reference's
  ``nki_matmul_fully_optimized_`` arm, on the vendor library);
* ``dense_block`` (``--dense-arm``, not in the reference's report): the
  dense SwiGLU (``compat.nki_baseline``) on weights rebuilt as U.V.

Attention is the same in all arms and is not the subject of the comparison:
torch's scaled_dot_product_attention, restricted to its flash and
memory-efficient kernels (non-causal, as ``jax.nn.dot_product_attention`` is
called at bench/e2e_block.py:222), with the KV heads repeated per group.
Times are hipEvent-timed whole-model forward passes; the report keeps the
reference's keys (bench/e2e_block.py:338-352, 399-413).

    python -m svdmlp.e2e_block --model llama3-8b --seq-lens 128 512 1024 --layers 4
"""

from __future__ import annotations

import argparse
import json
import math
import statistics
import sys

_SHAPES = {
    "llama3-3b": dict(hidden=3072, intermediate=8192, heads=24, kv_heads=8, layers=28),
    "llama3-8b": dict(hidden=4096, intermediate=14336, heads=32, kv_heads=8, layers=32),
}
_DEFAULT_COMPRESS_RATIO = 0.8
RMS_EPS = 1e-6
_WEIGHT_KEYS = ("norm1_w", "norm2_w", "wq", "wk", "wv", "wo", "ug", "vg", "uu", "vu", "ud", "vd")


def rmsnorm(x, w, eps: float = RMS_EPS):
    """bench/e2e_block.py:72-75: fp32 x / sqrt(mean(x^2) + eps) * w, cast back."""
    import torch

    x32 = x.float()
    rms = torch.sqrt(torch.mean(x32 * x32, dim=-1, keepdim=True) + eps)
    return (x32 / rms * w.float()).to(x.dtype)


def attention(x, wq, wk, wv, wo, num_heads: int, num_kv_heads: int):
    """Grouped-query attention over one sequence (bench/e2e_block.py:205-226):
    q, k, v projections, KV heads repeated per group, non-causal softmax
    attention with scale 1/sqrt(head_dim), output projection."""
    import torch
    from torch.nn.attention import SDPBackend, sdpa_kernel

    S, H = x.shape
    head_dim = H // num_heads
    groups = num_heads // num_kv_heads
    q = (x @ wq).view(S, num_heads, head_dim).transpose(0, 1)
    k = (x @ wk).view(S, num_kv_heads, head_dim).transpose(0, 1).repeat_interleave(groups, dim=0)
    v = (x @ wv).view(S, num_kv_heads, head_dim).transpose(0, 1).repeat_interleave(groups, dim=0)
    if x.device.type == "cuda":
        # flash / memory-efficient kernels only: the math fallback runs batched
        # bf16 products on transposed views
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            out = torch.nn.functional.scaled_dot_product_attention(q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0))[0]
    else:
        scores = (q.float() @ k.float().transpose(-1, -2)) / math.sqrt(head_dim)
        out = (torch.softmax(scores, dim=-1) @ v.float()).to(x.dtype)
    return out.transpose(0, 1).reshape(S, H) @ wo


def make_layer_weights(gen, device, H: int, I: int, R: int, num_heads: int, num_kv_heads: int, dtype):
    """Synthetic weights of one layer (bench/e2e_block.py:88-115): unit norm
    gains, N(0, 1/fan_in) projections and SVD factors, drawn from ``gen``."""
    import torch

    kv_dim = num_kv_heads * (H // num_heads)

    def rand(shape, fan_in):
        return (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) / math.sqrt(fan_in)).to(dtype)

    return dict(
        norm1_w=torch.ones(H, device=device, dtype=dtype), norm2_w=torch.ones(H, device=device, dtype=dtype),
        wq=rand((H, H), H), wk=rand((H, kv_dim), H), wv=rand((H, kv_dim), H), wo=rand((H, H), H),
        ug=rand((H, R), H), vg=rand((R, I), R), uu=rand((H, R), H), vu=rand((R, I), R),
        ud=rand((I, R), I), vd=rand((R, H), R))


def load_checkpoint_weights(model_path, layer_indices, device, dtype):
    """Real weights of the selected layers (bench/e2e_block.py:118-197):
    attention projections and norm gains straight from the safetensors
    shards (2-D Linear weights transposed to (in, out)), MLP factors through
    :func:`svdmlp.checkpoint.load_mlp_factors`."""
    from contextlib import ExitStack
    from pathlib import Path

    from safetensors import safe_open

    from . import checkpoint

    model_path = Path(model_path)
    _, index = checkpoint.checkpoint_metadata(model_path)
    weight_map = index["weight_map"]
    attn = ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
            "self_attn.o_proj.weight", "input_layernorm.weight", "post_attention_layernorm.weight")
    keys = [f"model.layers.{layer}.{suffix}" for layer in layer_indices for suffix in attn]
    missing = [k for k in keys if k not in weight_map]
    if missing:
        raise KeyError(f"checkpoint missing key: {missing[0]}")
    raw = {}
    with ExitStack() as stack:
        shards = {name: stack.enter_context(safe_open(str(model_path / name), framework="pt"))
                  for name in sorted({weight_map[k] for k in keys})}
        for k in keys:
            t = shards[weight_map[k]].get_tensor(k)
            raw[k] = (t.t() if t.dim() == 2 else t).contiguous().to(device=device, dtype=dtype)
    factors = checkpoint.load_mlp_factors(model_path, layer_indices, device=device, dtype=dtype)
    out = []
    for layer, (ug, vg, uu, vu, ud, vd) in zip(layer_indices, factors):
        p = f"model.layers.{layer}."
        out.append(dict(norm1_w=raw[p + "input_layernorm.weight"], norm2_w=raw[p + "post_attention_layernorm.weight"],
                        wq=raw[p + "self_attn.q_proj.weight"], wk=raw[p + "self_attn.k_proj.weight"],
                        wv=raw[p + "self_attn.v_proj.weight"], wo=raw[p + "self_attn.o_proj.weight"],
                        ug=ug, vg=vg, uu=uu, vu=vu, ud=ud, vd=vd))
    return out


def unfused_block(x, w, num_heads: int, num_kv_heads: int):
    """bench/e2e_block.py:229-253: attention, then six plain GEMMs."""
    from . import compat

    x = x + attention(rmsnorm(x, w["norm1_w"]), w["wq"], w["wk"], w["wv"], w["wo"], num_heads, num_kv_heads)
    h = rmsnorm(x, w["norm2_w"])
    return x + compat._unfused_low_rank_pallas(h, w["uu"], w["vu"], w["ug"], w["vg"], w["ud"], w["vd"])


def fused_block(x, w, num_heads: int, num_kv_heads: int, workspace=None):
    """bench/e2e_block.py:256-278: attention, then the library's MLP block
    (RMSNorm, fused SVD MLP and residual in HIP kernels)."""
    from . import ops

    x = x + attention(rmsnorm(x, w["norm1_w"]), w["wq"], w["wk"], w["wv"], w["wo"], num_heads, num_kv_heads)
    return ops.svd_mlp_block(x, w["norm2_w"].float(), w["ug"], w["vg"], w["uu"], w["vu"], w["ud"], w["vd"],
                             eps=RMS_EPS, workspace=workspace)


def dense_block(x, w, dense, num_heads: int, num_kv_heads: int):
    """Dense comparison arm: attention, then the dense SwiGLU
    (test_speedup.py:669-678) on ``dense`` = (up_proj, gate_proj, down_proj)."""
    from . import compat

    x = x + attention(rmsnorm(x, w["norm1_w"]), w["wq"], w["wk"], w["wv"], w["wo"], num_heads, num_kv_heads)
    return x + compat.nki_baseline(rmsnorm(x, w["norm2_w"]), *dense)


def _stats(samples) -> dict:
    """The latency keys of bench/e2e_block.py:281-302."""
    samples = sorted(samples)
    return dict(latency_ms_avg=statistics.fmean(samples), latency_ms_p50=statistics.median(samples),
                latency_ms_p90=samples[math.ceil(0.90 * len(samples)) - 1], latency_ms_min=samples[0],
                latency_ms_max=samples[-1], iterations=len(samples))


def _time_model(torch, fn, x, warmup: int, repeats: int) -> dict:
    for _ in range(warmup):
        fn(x)
    torch.cuda.synchronize()
    samples = []
    stream = torch.cuda.current_stream()
    for _ in range(repeats):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn(x)
        b.record(stream)
        b.synchronize()
        samples.append(a.elapsed_time(b))
    return _stats(samples)


def bench_model(S: int, cfg: dict, args) -> dict:
    """One sequence length (bench/e2e_block.py:305-356)."""
    import torch

    from . import compat, ops

    compat._positive("S", S)
    H, I, n_heads, kv_heads = cfg["hidden"], cfg["intermediate"], cfg["heads"], cfg["kv_heads"]
    n_layers = args.layers if args.layers is not None else cfg["layers"]
    dev = torch.device("cuda:0")
    dtype = torch.bfloat16
    if args.model_path:
        print(f"S={S}: loading real checkpoint weights for {n_layers} layers...", flush=True)
        weights = load_checkpoint_weights(args.model_path, list(range(n_layers)), dev, dtype)
        R = weights[0]["ug"].shape[1]
        compress_ratio = R / ops.low_rank_dim(H, I, 1.0)
    else:
        R = ops.low_rank_dim(H, I, args.compress_ratio)
        compress_ratio = args.compress_ratio
        gen = torch.Generator(device=dev)
        gen.manual_seed(args.seed)
        weights = [make_layer_weights(gen, dev, H, I, R, n_heads, kv_heads, dtype) for _ in range(n_layers)]
    xgen = torch.Generator(device=dev)
    xgen.manual_seed(args.seed ^ 0xDEAD)
    x = (torch.randn((S, H), generator=xgen, device=dev, dtype=torch.float32) * 0.02).to(dtype)
    r_max = max(max(w["ug"].shape[1], w["ud"].shape[1]) for w in weights)  # checkpoint ranks may differ per layer
    workspace = ops.svd_mlp_workspace(x, r=r_max, ff=I)

    def unfused_model(x):
        for w in weights:
            x = unfused_block(x, w, n_heads, kv_heads)
        return x

    def fused_model(x):
        for w in weights:
            x = fused_block(x, w, n_heads, kv_heads, workspace)
        return x

    # both arms first agree on the output (same weights, same rounding points
    # up to accumulation order)
    got, want = fused_model(x).float(), unfused_model(x).float()
    agreement = float(torch.linalg.norm(got - want) / torch.clamp(torch.linalg.norm(want), min=1e-12))
    if not bool(torch.isfinite(got).all()):
        raise FloatingPointError("fused model output contains NaN/Inf")
    unfused_stats = _time_model(torch, unfused_model, x, args.warmup, args.repeats)
    fused_stats = _time_model(torch, fused_model, x, args.warmup, args.repeats)
    rec = dict(seq_len=S, hidden=H, intermediate=I, rank=R, compress_ratio=compress_ratio, num_layers=n_layers,
               num_heads=n_heads, num_kv_heads=kv_heads, weights="checkpoint" if args.model_path else "synthetic",
               unfused_block=unfused_stats, fused_block=fused_stats,
               speedup_fused_vs_unfused=unfused_stats["latency_ms_avg"] / fused_stats["latency_ms_avg"],
               fused_vs_unfused_relative_l2=agreement)
    if args.dense_arm:
        dense = [tuple((w[u].float() @ w[v].float()).to(dtype).t().contiguous()
                       for u, v in (("uu", "vu"), ("ug", "vg"), ("ud", "vd"))) for w in weights]

        def dense_model(x):
            for w, dw in zip(weights, dense):
                x = dense_block(x, w, dw, n_heads, kv_heads)
            return x

        rec["dense_block"] = _time_model(torch, dense_model, x, args.warmup, args.repeats)
        rec["speedup_fused_vs_dense"] = rec["dense_block"]["latency_ms_avg"] / fused_stats["latency_ms_avg"]
        del dense
    del weights
    return rec


def _parser() -> argparse.ArgumentParser:
    """The flags of bench/e2e_block.py:363-394, plus --dense-arm."""
    p = argparse.ArgumentParser(description="Whole-model N-layer transformer E2E: fused vs unfused SVD MLP.")
    p.add_argument("--model", choices=list(_SHAPES), default="llama3-3b")
    p.add_argument("--seq-lens", type=int, nargs="+", default=[128, 512, 1024], metavar="S")
    p.add_argument("--layers", type=int, default=None, help="Override layer count (default: model depth)")
    p.add_argument("--model-path", type=str, default=None, metavar="PATH",
                   help="Path to an SVD-decomposed HF checkpoint directory. If omitted, synthetic random weights are used.")
    p.add_argument("--compress-ratio", type=float, default=_DEFAULT_COMPRESS_RATIO)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--repeats", type=int, default=10)
    p.add_argument("--seed", type=int, default=42)
    p.add_argument("--output", type=str, default=None, help="Write full JSON report to this path")
    p.add_argument("--dense-arm", action="store_true", help="also time the dense SwiGLU block (weights rebuilt as U.V)")
    return p


def main(argv=None) -> int:
    args = _parser().parse_args(argv)
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("E2E block benchmark requires a ROCm GPU")
    cfg = _SHAPES[args.model]
    results = []
    for S in args.seq_lens:
        rec = bench_model(S, cfg, args)
        results.append(rec)
        print(json.dumps(rec, indent=2), flush=True)
    report = dict(model=args.model, backend="rocm", torch_version=torch.__version__,
                  devices=[torch.cuda.get_device_name(0)], compress_ratio=args.compress_ratio, cases=results)
    if args.output:
        with open(args.output, "w", encoding="utf-8") as fh:
            json.dump(report, fh, indent=2)
            fh.write("\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
