"""Host-side contract of the package (no GPU): the reference's validation
messages and exception types, block-parameter tables, VMEM budget checks,
rank helpers and seeded generators."""

import numpy as np
import pytest
import torch

import oracle as O
from svdmlp import compat, config, inputs, ops


def _t(shape, dtype=torch.float32):
    return torch.zeros(shape, dtype=dtype)


# ---------------------------------------------------------------------------
# validation (test_speedup.py:37-49,508-509,530-533;
# tests_test_speedup_migration.py.before:122-132)
# ---------------------------------------------------------------------------

def test_invalid_configuration_rejected_before_launch():
    a = _t((8, 128))
    b = _t((128, 128))
    with pytest.raises(ValueError, match="positive integer"):
        compat.fused_mlp_up_T(a, b, b, b, b, M_tiles_in_block=0)
    with pytest.raises(ValueError, match="VMEM"):
        compat.fused_mlp_up_T(a, b, b, b, b, M_tiles_in_block=1024)
    with pytest.raises(ValueError, match="matching shapes"):
        compat.fused_mlp_up_T(a, b, b, b[:, :64], b)
    with pytest.raises(TypeError, match="same dtype"):
        compat.fused_three_mm_XTUV(a.T, b, b.to(torch.bfloat16))


def test_validation_messages_of_the_operator_api():
    x, u, v = _t((4, 16)), _t((16, 8)), _t((8, 32))
    with pytest.raises(ValueError, match="nonempty 2D array"):
        ops.fused_xuv(_t((0, 16)), u, v)
    with pytest.raises(ValueError, match="nonempty 2D array"):
        ops.fused_xuv(_t((4, 16, 1)), u, v)
    with pytest.raises(TypeError, match="supported dtypes are bfloat16 and float32"):
        ops.fused_xuv(x.half(), u.half(), v.half())
    with pytest.raises(ValueError, match="contraction dimensions do not match"):
        ops.fused_xuv(x, _t((15, 8)), v)
    with pytest.raises(ValueError, match="contraction dimensions do not match"):
        ops.fused_gate_up(x, u, _t((7, 32)), u, v)
    with pytest.raises(ValueError, match="gate/up factors must have matching shapes"):
        ops.fused_gate_up(x, u, v, u, _t((8, 31)))


def test_cpu_tensors_are_refused_not_computed():
    x, u, v = _t((4, 16)), _t((16, 8)), _t((8, 32))
    with pytest.raises(ValueError, match="ROCm GPU"):
        ops.fused_xuv(x, u, v)


def test_interpret_mode_has_no_cpu_fallback():
    a = _t((8, 128))
    b = _t((128, 128))
    with pytest.raises(NotImplementedError, match="GPU only"):
        compat.fused_mlp_up_T(a, b, b, b, b, interpret=True)


def test_down_backend_validated():
    a = _t((8, 128))
    b = _t((128, 128))
    with pytest.raises(ValueError, match="down_backend"):
        compat.svd_mlp_with_fused_kernel(a, b, b, b, b, b, b, down_backend="xla")


def test_fp8_factors_require_bf16_activations():
    q = ops.QuantizedFactor(torch.zeros((16, 8), dtype=torch.float8_e4m3fn), torch.ones(8))
    qv = ops.QuantizedFactor(torch.zeros((8, 32), dtype=torch.float8_e4m3fn), torch.ones(32))
    with pytest.raises(TypeError, match="bfloat16"):
        ops.fused_xuv(_t((4, 16)), q, qv)
    with pytest.raises(TypeError, match="same dtype"):
        ops.fused_xuv(_t((4, 16), torch.bfloat16), q, _t((8, 32), torch.bfloat16))


# ---------------------------------------------------------------------------
# block parameters and the VMEM budget (test_speedup.py:169-317)
# ---------------------------------------------------------------------------

def test_block_param_tables():
    assert compat.get_fused_mlp_up_T_params(128) == dict(
        M_tiles_in_block=4, r_tiles_in_block=2, K_tiles_in_block=1, N_tiles_in_block=2)
    assert compat.get_fused_mlp_up_T_params(1024) == dict(
        M_tiles_in_block=2, r_tiles_in_block=2, K_tiles_in_block=4, N_tiles_in_block=1)
    assert compat.get_fused_mlp_up_T_params(600)["K_tiles_in_block"] == 2
    assert compat.get_fused_three_mm_XTUV_params(1024)["K_tiles_in_block"] == 2
    assert compat.get_fused_three_mm_XTUV_params(2048)["K_tiles_in_block"] == 4
    with pytest.raises(ValueError, match="positive integer"):
        compat.get_fused_mlp_up_T_params(0)
    with pytest.raises(ValueError, match="positive integer"):
        compat.get_fused_three_mm_XTUV_params(True)


@pytest.mark.parametrize("S", [1, 8, 13, 127, 128, 129, 512, 1024])
def test_default_vmem_for_target_models(S):
    # tests_test_speedup_migration.py.before:110-119
    for H, I, R in [(3072, 8192, 1792), (4096, 14336, 2560)]:
        for gate, M, N, params in [(True, H, I, compat.get_fused_mlp_up_T_params(S)),
                                   (False, I, H, compat.get_fused_three_mm_XTUV_params(S))]:
            shape = compat._fusion_shape(M, R, S, N, torch.bfloat16, params["M_tiles_in_block"],
                                         params["r_tiles_in_block"], params["K_tiles_in_block"],
                                         params["N_tiles_in_block"], gate)
            assert shape.vmem_bytes < compat.VMEM_LIMIT * compat.VMEM_HEADROOM


def test_async_vmem_budget_includes_second_weight_slot():
    # tests_test_speedup_migration.py.before:236-240
    args = (513, 513, 257, 1025, torch.float32, 2, 2, 2, 2, True)
    compat._fusion_shape(*args, async_dma=False)
    with pytest.raises(ValueError, match="VMEM"):
        compat._fusion_shape(*args, async_dma=True)


def test_fusion_shape_padding():
    s = compat._fusion_shape(4096, 2816, 1024, 14336, torch.bfloat16, 2, 2, 4, 1, True)
    assert (s.M_block, s.r_block, s.K_block, s.N_block) == (512, 512, 512, 512)
    assert (s.M_padded, s.r_padded, s.K_padded, s.N_padded) == (4096, 2816, 1024, 14336)


# ---------------------------------------------------------------------------
# model tables and ranks
# ---------------------------------------------------------------------------

def test_models_and_rank_for():
    m = config.MODELS["llama-3.1-8b"]
    assert (m.hidden_size, m.intermediate_size, m.num_layers) == (4096, 14336, 32)
    assert m.rank_at_080 == 2560
    assert config.rank_for(m, 0.9) == 2816
    assert config.MODELS["llama-3.2-3b"].rank_at_080 == 1792
    with pytest.raises(ValueError, match="compress-ratio"):
        config.rank_for(m, 0.0)
    for H, I, c in [(2048, 8192, 0.8), (4096, 14336, 0.9), (640, 640, 1.0), (896, 896, 1.0)]:
        assert ops.low_rank_dim(H, I, c) == O.low_rank_dim(H, I, c)


def test_gate_up_blocks_namedtuple():
    b = config.GateUpBlocks(bs=128, bh=1024, br=512, bn=512)
    assert b._asdict() == dict(bs=128, bh=1024, br=512, bn=512)


# ---------------------------------------------------------------------------
# seeded inputs (test_speedup.py:803-835)
# ---------------------------------------------------------------------------

def test_generator_order_and_scale():
    shape = inputs.LayerShape(64, 96, 32)
    ug, vg, uu, vu, ud, vd = inputs.make_factors(shape, seed=5)
    rng = np.random.default_rng(5)
    first = rng.normal(size=(64, 32)).astype(np.float32) / np.float32(8.0)
    np.testing.assert_array_equal(uu, first)          # u_up is drawn first
    assert ug.shape == (64, 32) and vg.shape == (32, 96) and ud.shape == (96, 32) and vd.shape == (32, 64)
    big = inputs.make_factors(inputs.LayerShape(1024, 1024, 512), seed=0)
    assert abs(big[0].std() - 1 / 32) < 1e-3            # N(0, 1/d_in)
    assert abs(big[1].std() - 1 / np.sqrt(512)) < 1e-3  # N(0, 1/r)


def test_quantizer_matches_oracle_codec():
    from svdmlp import fp8

    w = (np.random.default_rng(2).normal(size=(256, 64)) / 16).astype(np.float32)
    q = fp8.quantize_per_channel(torch.from_numpy(w))
    q_ref, s_ref = O.quantize_per_channel(w, axis=0)
    np.testing.assert_allclose(q.scale.numpy(), s_ref, rtol=1e-6)
    np.testing.assert_array_equal(q.data.view(torch.uint8).numpy(), q_ref)


# ---------------------------------------------------------------------------
# MLP stack helpers
# ---------------------------------------------------------------------------

def test_stack_rank_draw_is_seeded_and_in_choices():
    from svdmlp import stack

    a = stack.draw_ranks(32, seed=7)
    assert a == stack.draw_ranks(32, seed=7)
    assert a != stack.draw_ranks(32, seed=8)
    assert all(r in stack.RANK_CHOICES for row in a for r in row)
    # gate, up and down are drawn independently: some layer has unequal ranks
    assert any(len(set(row)) > 1 for row in a)


def test_stack_rank_padding_is_exact():
    """Zero-padding U columns / V rows leaves x.U.V unchanged (checked with
    the oracle's float64-free fp32 math on CPU tensors)."""
    import torch

    from svdmlp import ops

    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 16, generator=g)
    u, v = torch.randn(16, 6, generator=g), torch.randn(6, 12, generator=g)
    up, vp = ops.pad_rank(u, v, 10)
    assert up.shape == (16, 10) and vp.shape == (10, 12)
    assert torch.equal(up[:, 6:], torch.zeros(16, 4)) and torch.equal(vp[6:], torch.zeros(4, 12))
    np.testing.assert_allclose(O.fused_xuv_ref(x.numpy(), up.numpy(), vp.numpy()),
                               O.fused_xuv_ref(x.numpy(), u.numpy(), v.numpy()), rtol=1e-6, atol=1e-6)


def test_pad_rank_fp8_and_branches():
    """fp8 factors pad with zero data (and unit U scales): the dequantized
    product is unchanged; _pad_branches brings gate and up to one rank."""
    import torch

    from svdmlp import fp8, ops

    g = torch.Generator().manual_seed(1)
    u = fp8.quantize_per_channel(torch.randn(16, 6, generator=g) / 4)
    v = fp8.quantize_per_channel(torch.randn(6, 12, generator=g) / 4)
    up, vp = ops.pad_rank(ops.QuantizedFactor(u.data, u.scale), ops.QuantizedFactor(v.data, v.scale), 10)
    assert up.shape == (16, 10) and vp.shape == (10, 12) and up.data.dtype == u.data.dtype
    assert torch.equal(up.data[:, :6].view(torch.uint8), u.data.view(torch.uint8))
    assert not up.data[:, 6:].view(torch.uint8).any() and not vp.data[6:].view(torch.uint8).any()
    assert torch.equal(up.scale[6:], torch.ones(4)) and torch.equal(vp.scale, v.scale)
    torch.testing.assert_close(up.dequantize() @ vp.dequantize(),
                               ops.QuantizedFactor(u.data, u.scale).dequantize() @ ops.QuantizedFactor(v.data, v.scale).dequantize())
    ug, vg, uu, vu = (torch.randn(16, 6), torch.randn(6, 12), torch.randn(16, 9), torch.randn(9, 12))
    pg, pvg, pu, pvu = ops._pad_branches(ug, vg, uu, vu)
    assert pg.shape == pu.shape == (16, 9) and pvg.shape == pvu.shape == (9, 12)
    assert pu is uu and pvu is vu   # the larger branch is passed through


def test_stack_flops_uses_drawn_ranks():
    from svdmlp import stack

    class L:
        def __init__(self, ranks):
            self.ranks = ranks

    layers = [L((2048, 3072, 2560)), L((2816, 2816, 2816))]
    T, d, ff = 4096, 4096, 14336
    want = sum(2 * T * ((rg + ru) * (d + ff) + rd * (ff + d)) for rg, ru, rd in (l.ranks for l in layers))
    assert stack.stack_flops(T, d, ff, layers) == want
    assert stack.stack_flops(T, d, ff, layers[1:]) == O.layer_flops(T, d, ff, 2816)


def test_padded_branches_are_cached_per_layer():
    """The zero-padding fallback (shapes whose kernels take one gate/up rank)
    reuses a layer's padded copies on the next call, and makes new ones once
    a factor is written in place (its version counter moves)."""
    ops._PAD_CACHE.clear()
    ug, vg, uu, vu = (torch.randn(16, 6), torch.randn(6, 12), torch.randn(16, 9), torch.randn(9, 12))
    first = ops._pad_branches(ug, vg, uu, vu)
    again = ops._pad_branches(ug, vg, uu, vu)
    assert all(a is b for a, b in zip(first, again))
    ug.mul_(2.0)   # in-place write: the cached padded copy is stale
    fresh = ops._pad_branches(ug, vg, uu, vu)
    assert fresh[0] is not first[0] and torch.equal(fresh[0][:, :6], ug)
    for i in range(ops._PAD_CACHE_LAYERS + 3):   # bounded: the oldest layers are dropped
        ops._pad_branches(torch.randn(16, 6), torch.randn(6, 12), uu, vu)
    assert len(ops._PAD_CACHE) == ops._PAD_CACHE_LAYERS
    ops._PAD_CACHE.clear()


def test_outlier_layer_generator():
    """inputs.make_outlier_layer: seeded; the listed hidden channels of x are
    scaled by their factors; factor columns carry log-normal scales (a few
    columns far above the median norm); shapes as make_layer."""
    shape = inputs.LayerShape(512, 1024, 128)
    x, f = inputs.make_outlier_layer(shape, 64, seed=5)
    x2, f2 = inputs.make_outlier_layer(shape, 64, seed=5)
    assert np.array_equal(x, x2) and all(np.array_equal(a, b) for a, b in zip(f, f2))
    xb, fb = inputs.make_layer(shape, 64, seed=5)
    assert x.shape == xb.shape and [a.shape for a in f] == [a.shape for a in fb]
    col_rms = np.sqrt((x ** 2).mean(axis=0))
    assert col_rms[17] > 1000 and col_rms[3] > 300 and col_rms[250] > 30
    assert np.median(col_rms) < 2
    for a in f:
        norms = np.sqrt((a ** 2).sum(axis=0))
        assert norms.max() > 5 * np.median(norms)
