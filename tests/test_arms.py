"""Host-side contract of the pallas_ops-style API, the comparison arms
(test_speedup.py:545-735) and the benchmark runners (test_speedup.py's
synthetic branch, bench/e2e_block.py): argument validation that raises before
any GPU work, and the e2e block's attention and RMSNorm against independent
float64 restatements."""

import math

import numpy as np
import pytest
import torch

from svdmlp import compat, e2e_block, inputs, pallas_ops, speedup
from svdmlp.config import GateUpBlocks


def _cpu(*shapes, dtype=torch.bfloat16):
    return [torch.zeros(s, dtype=dtype) for s in shapes]


def test_pallas_ops_reject_interpret_and_bad_blocks():
    x, ug, vg, uu, vu, ud, vd = _cpu((8, 64), (64, 32), (32, 96), (64, 32), (32, 96), (96, 32), (32, 64))
    with pytest.raises(NotImplementedError, match="CPU emulator"):
        pallas_ops.svd_mlp(x, ug, vg, uu, vu, ud, vd, interpret=True)
    with pytest.raises(NotImplementedError):
        pallas_ops.xuv_matmul(x, ug, vg, interpret=True)
    with pytest.raises(ValueError, match="gate_up_blocks.br must be a positive integer"):
        pallas_ops.svd_mlp(x, ug, vg, uu, vu, ud, vd, gate_up_blocks=GateUpBlocks(128, 1024, 0, 512))
    with pytest.raises(ValueError, match="blocks must have the four fields"):
        pallas_ops.fused_gate_up(x, ug, vg, uu, vu, blocks=(128, 1024, 512))
    # valid blocks pass validation; the kernels then refuse CPU tensors
    with pytest.raises(ValueError, match="ROCm GPU"):
        pallas_ops.contracted_svd_mlp(x, ug, vg, uu, vu, ud, vd, gate_up_blocks=GateUpBlocks(128, 1024, 512, 512))


def test_dense_mlp_validation():
    x, wg, wu, wd = _cpu((8, 64), (64, 96), (64, 96), (96, 64))
    with pytest.raises(ValueError, match="dense MLP weight shapes"):
        pallas_ops.dense_mlp(x, wg, wu, wd[:, :32])
    with pytest.raises(TypeError, match="same dtype"):
        pallas_ops.dense_mlp(x, wg.float(), wu, wd)
    with pytest.raises(ValueError, match="ROCm GPU"):
        pallas_ops.dense_mlp(x, wg, wu, wd)


def test_nki_matmul_validation_follows_the_reference():
    a, b = _cpu((64, 16), (64, 32))
    with pytest.raises(ValueError, match="same contraction dimension"):
        compat.nki_matmul_fully_optimized_(a, b[:32])
    with pytest.raises(ValueError, match="TILES_IN_BLOCK_K must be a positive integer"):
        compat.nki_matmul_fully_optimized_(a, b, TILES_IN_BLOCK_K=0)
    with pytest.raises(NotImplementedError):
        compat.nki_matmul_fully_optimized_(a, b, interpret=True)
    # Mp * BLOCK_N * 2 bytes alone is over the 12.8 MiB budget for M = 8000
    big = torch.zeros((64, 8000), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="Estimated VMEM"):
        compat.nki_matmul_fully_optimized_(big, b)
    with pytest.raises(ValueError, match="ROCm GPU"):
        compat.nki_matmul_fully_optimized_(a, b)


def _attention_f64(x, wq, wk, wv, wo, nh, nkv):
    """Per-head loop in float64: head h reads KV head h // (nh / nkv)
    (jnp.repeat of the KV heads along the head axis)."""
    S, H = x.shape
    hd = H // nh
    q, k, v = x @ wq, x @ wk, x @ wv
    out = np.zeros((S, H))
    for h in range(nh):
        g = h // (nh // nkv)
        qh, kh, vh = q[:, h * hd:(h + 1) * hd], k[:, g * hd:(g + 1) * hd], v[:, g * hd:(g + 1) * hd]
        s = qh @ kh.T / math.sqrt(hd)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h * hd:(h + 1) * hd] = (p / p.sum(axis=1, keepdims=True)) @ vh
    return out @ wo


@pytest.mark.parametrize("nh,nkv", [(8, 2), (4, 4), (6, 1)])
def test_e2e_attention_matches_per_head_float64(nh, nkv):
    rng = np.random.default_rng(nh * 10 + nkv)
    S, H = 24, 48
    kv = nkv * (H // nh)
    x = rng.normal(size=(S, H))
    ws = [rng.normal(size=s) / math.sqrt(s[0]) for s in ((H, H), (H, kv), (H, kv), (H, H))]
    got = e2e_block.attention(*(torch.from_numpy(a).float() for a in (x, *ws)), nh, nkv)
    want = _attention_f64(x, *ws, nh, nkv)
    assert np.abs(got.numpy() - want).max() < 1e-5 * max(1.0, np.abs(want).max())


def test_e2e_rmsnorm_matches_float64():
    rng = np.random.default_rng(7)
    x = rng.normal(size=(5, 64)) * 0.02
    w = rng.uniform(0.5, 1.5, size=64)
    got = e2e_block.rmsnorm(torch.from_numpy(x).float(), torch.from_numpy(w).float()).numpy()
    want = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + 1e-6) * w
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-7)
    # eps 1e-6 matters at this scale: without it the result differs
    assert e2e_block.RMS_EPS == 1e-6


def test_runner_parsers_keep_the_reference_defaults():
    a = e2e_block._parser().parse_args([])
    assert (a.model, a.seq_lens, a.layers, a.compress_ratio, a.warmup, a.repeats, a.seed) == (
        "llama3-3b", [128, 512, 1024], None, 0.8, 3, 10, 42)
    b = speedup._parser().parse_args([])
    assert (b.model, b.seq_lens, b.warmup, b.repeats, b.seed, b.down_backend) == (
        "llama3-3b", [1, 128, 512], 3, 10, 0, "pallas")
    assert speedup._BASE == {"llama3-3b": (3072, 8192, 1792), "llama3-8b": (4096, 14336, 2560)}


def test_speedup_runner_rejects_before_touching_the_gpu():
    p = speedup._parser()
    with pytest.raises(ValueError, match="require --model-path"):
        speedup.run(p.parse_args(["--layers", "0"]))
    with pytest.raises(ValueError, match="no MI355X counterpart"):
        speedup.run(p.parse_args(["--interpret"]))
    with pytest.raises(ValueError, match="positive integer"):
        speedup.run(p.parse_args(["--seq-lens", "0"]))
    with pytest.raises(SystemExit):
        speedup.main(["--interpret"])


def test_synthetic_factors_follow_the_reference_draw_order():
    """uu, vu, ug, vg, ud, vd each N(0, 1/rows) from one generator
    (test_speedup.py:810-815): the same draws as the oracle-side recipe."""
    H, I, R = 64, 96, 32
    got = speedup.synthetic_factors(np.random.default_rng(5), H, I, R)
    ug, vg, uu, vu, ud, vd = inputs.make_factors(inputs.LayerShape(H, I, R), rng=np.random.default_rng(5))
    for g, w in zip(got, (uu, vu, ug, vg, ud, vd)):
        np.testing.assert_array_equal(g, w)
