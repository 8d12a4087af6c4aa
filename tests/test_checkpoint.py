"""The safetensors SVD-checkpoint loader (models/hf_svd.py:1-196) on synthetic
checkpoints written by the tests: orientation (transpose + v/u name swap),
sharding, inspection without payloads, and the reference's errors."""

import json

import numpy as np
import pytest
import torch

from svdmlp import checkpoint as C

D, FF, R = 64, 96, 32


def _factors(seed, dtype=torch.bfloat16, r=R):
    g = torch.Generator().manual_seed(seed)
    shapes = [(D, r), (r, FF), (D, r), (r, FF), (FF, r), (r, D)]
    return tuple((torch.randn(s, generator=g) / s[0] ** 0.5).to(dtype) for s in shapes)


@pytest.fixture()
def ckpt(tmp_path):
    layers = [_factors(1), _factors(2), _factors(3)]
    C.save_mlp_checkpoint(tmp_path, layers, hidden_size=D, intermediate_size=FF, shard_layers=2)
    return tmp_path, layers


def test_keys_follow_the_reference_names():
    assert C.factor_keys(7) == tuple(f"model.layers.7.mlp.{s}" for s in (
        "gate_v_proj.weight", "gate_u_proj.weight", "up_v_proj.weight", "up_u_proj.weight",
        "down_v_proj.weight", "down_u_proj.weight"))
    with pytest.raises(ValueError, match="non-negative"):
        C.factor_keys(-1)


def test_stored_tensors_are_linear_weights_with_swapped_names(ckpt):
    """gate_v_proj is the first projection, stored (out, in) = (r, d): the
    natural Ug (d, r) transposed; gate_u_proj is Vg (r, ff) transposed."""
    from safetensors import safe_open

    path, layers = ckpt
    index = json.loads((path / "model.safetensors.index.json").read_text())["weight_map"]
    key = "model.layers.0.mlp.gate_v_proj.weight"
    with safe_open(str(path / index[key]), framework="pt") as f:
        stored = f.get_tensor(key)
        assert tuple(stored.shape) == (R, D)
        assert torch.equal(stored, layers[0][0].t())
        assert tuple(f.get_tensor("model.layers.0.mlp.gate_u_proj.weight").shape) == (FF, R)
    assert len(set(index.values())) == 2  # three layers, two per shard


@pytest.mark.parametrize("layout", ["natural", "padded", "linear"])
def test_load_returns_gate_first_natural_operands(ckpt, layout):
    path, layers = ckpt
    loaded = C.load_mlp_factors(path, [2, 0], device="cpu", layout=layout)
    assert len(loaded) == 2
    for got, want in zip(loaded, (layers[2], layers[0])):
        for i, (g, w) in enumerate(zip(got, want)):
            assert g.shape == w.shape and g.dtype == w.dtype
            assert torch.equal(g, w)
            if layout == "padded" and i % 2:   # V factors: rows 64 elements longer in memory
                assert g.stride() == (w.shape[1] + 64, 1)
            else:
                assert g.is_contiguous() == (layout != "linear")


def test_load_converts_dtype(ckpt):
    path, layers = ckpt
    (f,) = C.load_mlp_factors(path, [1], device="cpu", dtype=torch.float32)
    assert all(t.dtype == torch.float32 for t in f)
    assert torch.equal(f[3], layers[1][3].float())


def test_inspect_reads_headers_only(ckpt):
    path, _ = ckpt
    meta = C.inspect_mlp_checkpoint(path)
    assert meta["selected_layers"] == [0, 1, 2]
    assert meta["hidden_size"] == D and meta["intermediate_size"] == FF
    assert [row["rank"] for row in meta["layers"]] == [R, R, R]
    assert meta["layers"][0]["factor_bytes"] == 2 * 3 * R * (D + FF)
    assert meta["layers"][0]["dtype"] == "BF16"
    assert meta["layers"][0]["tensors"][0]["shape"] == [R, D]
    assert C.inspect_mlp_checkpoint(path, [1])["selected_layers"] == [1]


def test_errors_match_the_reference(tmp_path, ckpt):
    path, _ = ckpt
    with pytest.raises(FileNotFoundError, match="missing checkpoint config"):
        C.checkpoint_metadata(tmp_path / "nowhere")
    empty = tmp_path / "noindex"
    empty.mkdir()
    (empty / "config.json").write_text("{}")
    with pytest.raises(FileNotFoundError, match="missing safetensors index"):
        C.checkpoint_metadata(empty)
    (empty / "model.safetensors.index.json").write_text("{}")
    with pytest.raises(ValueError, match="no weight_map"):
        C.checkpoint_metadata(empty)
    with pytest.raises(KeyError, match="missing MLP factors"):
        C.load_mlp_factors(path, [5], device="cpu")
    with pytest.raises(ValueError, match="at least one layer"):
        C.load_mlp_factors(path, [], device="cpu")
    with pytest.raises(ValueError, match="layer indices must be in"):
        C.inspect_mlp_checkpoint(path, [3])
    with pytest.raises(ValueError, match="without duplicates"):
        C.inspect_mlp_checkpoint(path, [0, 0])
    (path / "model-00002.safetensors").unlink()
    with pytest.raises(FileNotFoundError, match="shards required"):
        C.load_mlp_factors(path, [2], device="cpu")


def test_shape_and_dtype_validation():
    f = list(_factors(4))
    assert C.validate_factor_shapes(f, hidden_size=D, intermediate_size=FF) == R
    with pytest.raises(ValueError, match="six MLP factors"):
        C.validate_factor_shapes(f[:5], hidden_size=D, intermediate_size=FF)
    with pytest.raises(ValueError, match="invalid transposed MLP factor shapes"):
        C.validate_factor_shapes(f, hidden_size=D, intermediate_size=FF + 1)
    g = f[:]
    g[5] = g[5].float()
    with pytest.raises(TypeError, match="dtypes differ"):
        C.validate_factor_shapes(g, hidden_size=D, intermediate_size=FF)


def test_bias_or_non_silu_checkpoints_are_rejected(tmp_path):
    C.save_mlp_checkpoint(tmp_path, [_factors(5)], hidden_size=D, intermediate_size=FF,
                          extra_config={"hidden_act": "gelu"})
    with pytest.raises(ValueError, match="bias-free SwiGLU"):
        C.inspect_mlp_checkpoint(tmp_path)


def test_non_uniform_ranks_per_layer(tmp_path):
    layers = [_factors(6, r=32), _factors(7, r=48)]
    C.save_mlp_checkpoint(tmp_path, layers, hidden_size=D, intermediate_size=FF)
    meta = C.inspect_mlp_checkpoint(tmp_path)
    assert [row["rank"] for row in meta["layers"]] == [32, 48]
    a, b = C.load_mlp_factors(tmp_path, [0, 1], device="cpu")
    assert a[0].shape == (D, 32) and b[0].shape == (D, 48)
    assert np.array_equal(b[5].float().numpy(), layers[1][5].float().numpy())


# ---------------------------------------------------------------------------
# the per-layer runner (bench/checkpoint_speedup.py)
# ---------------------------------------------------------------------------

def test_runner_errors_and_summary():
    from svdmlp import checkpoint_speedup as CS

    e = CS._errors(np.ones((2, 3)), np.ones((2, 3)) * 2)
    assert e["relative_l2"] == pytest.approx(0.5) and e["max_abs_error"] == 1.0 and e["reference_rms"] == 2.0
    with pytest.raises(FloatingPointError):
        CS._errors(np.array([[np.nan]]), np.array([[1.0]]))
    with pytest.raises(ValueError, match="shape mismatch"):
        CS._errors(np.ones((2, 2)), np.ones((2, 3)))
    ok = {"fused_vs_fp32": {"relative_l2": 0.01}, "passed": True}
    recs = [dict(ok, layer=0, S=1, fused_ms=1.0, unfused_low_rank_ms=3.0),
            dict(ok, layer=1, S=1, fused_ms=2.0, unfused_low_rank_ms=3.0),
            dict(ok, layer=0, S=8, passed=False)]
    s1, s8 = CS.summarize(recs, [0, 1], [1, 8])
    assert s1["complete"] and s1["passed"] and s1["speedup_vs_unfused"] == pytest.approx(2.0)
    assert not s8["complete"] and not s8["passed"] and s8["failed_layers"] == [0]


def test_runner_inspect_only_writes_report(ckpt, tmp_path):
    from svdmlp import checkpoint_speedup as CS

    path, _ = ckpt
    out = tmp_path / "report" / "r.json"
    report = CS.run(CS._parser().parse_args(["--model-path", str(path), "--layers", "0", "2", "--inspect-only",
                                             "--output", str(out)]))
    assert report["complete"] and report["mode"] == "checkpoint_inspection"
    saved = json.loads(out.read_text())
    assert saved["checkpoint"]["selected_layers"] == [0, 2]
    assert out.with_suffix(".csv").read_text().startswith("layer,S,rank")
    with pytest.raises(ValueError, match="duplicates"):
        CS.run(CS._parser().parse_args(["--model-path", str(path), "--seq-lens", "1", "1"]))
