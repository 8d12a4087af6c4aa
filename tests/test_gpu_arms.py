"""The pallas_ops-style API, the comparison arms and the benchmark runners on
the GPU, against the oracle (bf16: relative Frobenius error <= 1e-2).

The dense and unfused arms run on the vendor library; the SVD-MLP entry
points run the HIP kernels through the C ABI."""

import argparse

import numpy as np
import pytest
import torch

import oracle as O
from svdmlp import compat, e2e_block, inputs, pallas_ops, speedup
from svdmlp.config import GateUpBlocks

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
SHAPE = inputs.LayerShape(512, 1024, 256)


def _layer(T, seed):
    x, f = inputs.make_layer(SHAPE, T=T, seed=seed)
    xb, *fb = (inputs.as_float32(a, torch.bfloat16) for a in (x, *f))
    return xb, fb


def _dev(arrs, gpu):
    return [inputs.to_torch(a, torch.bfloat16, gpu) for a in arrs]


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("T", [7, 300])
def test_pallas_ops_svd_entry_points(gpu, T):
    xb, fb = _layer(T, 40 + T)
    t = _dev((xb, *fb), gpu)
    want = O.svd_mlp_ref(xb, *fb, dtype="bfloat16")
    blocks = GateUpBlocks(128, 1024, 512, 512)
    for fn in (pallas_ops.svd_mlp, pallas_ops.contracted_svd_mlp):
        got = _np(fn(*t, gate_up_blocks=blocks))
        assert O.relative_l2(got, want) < BF16_TOL, fn.__name__
    h = _np(pallas_ops.fused_gate_up(*t[:5], blocks=blocks))
    assert O.relative_l2(h, O.fused_gate_up_ref(xb, *fb[:4], dtype="bfloat16")) < BF16_TOL
    hb = inputs.as_float32(h, torch.bfloat16)
    y = _np(pallas_ops.xuv_matmul(inputs.to_torch(hb, torch.bfloat16, gpu), t[5], t[6]))
    assert O.relative_l2(y, O.fused_xuv_ref(hb, fb[4], fb[5], "bfloat16")) < BF16_TOL


def test_dense_arms_match_dense_mlp_ref(gpu):
    """pallas_ops.dense_mlp (natural (H, I) weights) and compat.nki_baseline
    (Linear (out, in) weights) against kernels/reference.py:96-106 on dense
    weights rebuilt from the factors as U.V."""
    xb, (ug, vg, uu, vu, ud, vd) = _layer(64, 9)
    wg, wu, wd = (inputs.as_float32(u @ v, torch.bfloat16) for u, v in ((ug, vg), (uu, vu), (ud, vd)))
    want = O.dense_mlp_ref(xb, wg, wu, wd, dtype="bfloat16")
    x, twg, twu, twd = _dev((xb, wg, wu, wd), gpu)
    assert O.relative_l2(_np(pallas_ops.dense_mlp(x, twg, twu, twd)), want) < BF16_TOL
    got = compat.nki_baseline(x, twu.t().contiguous(), twg.t().contiguous(), twd.t().contiguous())
    assert O.relative_l2(_np(got), want) < BF16_TOL


def test_unfused_arm_on_the_plain_matmul(gpu):
    xb, fb = _layer(130, 11)
    x, ug, vg, uu, vu, ud, vd = _dev((xb, *fb), gpu)
    got = compat._unfused_low_rank_pallas(x, uu, vu, ug, vg, ud, vd)
    assert O.relative_l2(_np(got), O.svd_mlp_ref(xb, *fb, dtype="bfloat16")) < BF16_TOL
    # lhsT^T . rhs with the transposed operand
    a = x[:, :256].t().contiguous()
    np.testing.assert_allclose(_np(compat.nki_matmul_fully_optimized_(a, ug[:256])),
                               _np((x[:, :256].float() @ ug[:256].float()).to(torch.bfloat16)), rtol=2e-2, atol=2e-2)


def _args(**kw):
    base = dict(layers=2, model_path=None, compress_ratio=0.8, warmup=1, repeats=2, seed=3, dense_arm=True)
    base.update(kw)
    return argparse.Namespace(**base)


def test_e2e_block_model_matches_a_cpu_fp32_chain(gpu):
    """Two layers of RMSNorm -> GQA attention -> residual -> RMSNorm -> SVD MLP
    -> residual: the fused model on the GPU against the same chain in fp32 on
    the CPU (attention and RMSNorm restated per head in float64 in the CPU
    tests; the MLP is the oracle's)."""
    cfg = dict(hidden=512, intermediate=1024, heads=8, kv_heads=2, layers=2)
    H, I = cfg["hidden"], cfg["intermediate"]
    R = O.low_rank_dim(H, I, 0.8)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(5)
    weights = [e2e_block.make_layer_weights(gen, gpu, H, I, R, 8, 2, torch.bfloat16) for _ in range(2)]
    x = (torch.randn((96, H), generator=gen, device=gpu) * 0.02).to(torch.bfloat16)
    got = x
    for w in weights:
        got = e2e_block.fused_block(got, w, 8, 2)
    ref = x.float().cpu()
    for w in weights:
        c = {k: v.float().cpu() for k, v in w.items()}
        ref = ref + e2e_block.attention(e2e_block.rmsnorm(ref, c["norm1_w"]), c["wq"], c["wk"], c["wv"], c["wo"], 8, 2)
        h = e2e_block.rmsnorm(ref, c["norm2_w"]).numpy()
        ref = ref + torch.from_numpy(O.svd_mlp_ref(h, *(c[k].numpy() for k in ("ug", "vg", "uu", "vu", "ud", "vd"))))
    assert O.relative_l2(_np(got), ref.numpy()) < 2e-2


def test_e2e_bench_record(gpu):
    cfg = dict(hidden=512, intermediate=1024, heads=8, kv_heads=2, layers=2)
    rec = e2e_block.bench_model(64, cfg, _args())
    for key in ("seq_len", "hidden", "intermediate", "rank", "compress_ratio", "num_layers", "num_heads",
                "num_kv_heads", "weights", "unfused_block", "fused_block", "speedup_fused_vs_unfused",
                "dense_block", "speedup_fused_vs_dense"):
        assert key in rec, key
    assert rec["rank"] == 256 and rec["num_layers"] == 2 and rec["weights"] == "synthetic"
    assert rec["fused_vs_unfused_relative_l2"] < 2e-2
    for arm in ("unfused_block", "fused_block", "dense_block"):
        s = rec[arm]
        assert s["iterations"] == 2 and 0 < s["latency_ms_min"] <= s["latency_ms_avg"] <= s["latency_ms_max"]


def test_speedup_runner_check_only(gpu):
    args = speedup._parser().parse_args(["--hidden", "512", "--intermediate", "1024", "--rank", "256",
                                         "--seq-lens", "1", "64", "--check-only", "--seed", "4"])
    recs = speedup.run(args)
    assert [r["S"] for r in recs] == [1, 64]
    assert all(r["relative_l2"] < BF16_TOL for r in recs)
    args = speedup._parser().parse_args(["--hidden", "512", "--intermediate", "1024", "--rank", "256",
                                         "--seq-lens", "32", "--warmup", "1", "--repeats", "2",
                                         "--down-backend", "jax"])
    (rec,) = speedup.run(args)
    assert rec["down_params"] is None and rec["speedup_vs_dense"] > 0 and rec["speedup_vs_unfused"] > 0
