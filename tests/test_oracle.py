"""Pins the CPU oracle (oracle/reference_cpu.py) against checks that do not
restate its formulas: independent implementations (torch casts), float64
brute force, closed forms, invariants and the reference's own known answers.
Each group is chosen so that a plausible slip (dropped term, wrong sign or
index, transposed operand, wrong rounding) fails at least one assertion."""

import math

import numpy as np
import pytest
import torch

import oracle as O

rng = np.random.default_rng(1234)


# ---------------------------------------------------------------------------
# bf16 rounding vs torch's cast
# ---------------------------------------------------------------------------

def _torch_bf16(a):
    return torch.from_numpy(np.asarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def test_round_bf16_matches_torch_on_random_and_edge_values():
    vals = [rng.normal(size=100_000).astype(np.float32),
            (rng.normal(size=10_000) * 1e30).astype(np.float32),
            (rng.normal(size=10_000) * 1e-38).astype(np.float32)]
    # ties: low 16 bits exactly 0x8000, with even and odd upper parts
    base = rng.integers(0, 0x7F7F, size=4096, dtype=np.uint32) << 16  # finite patterns only
    base |= rng.integers(0, 2, size=4096, dtype=np.uint32) << 31
    ties = (base | 0x8000).view(np.float32)
    near = np.concatenate([(base | 0x7FFF), (base | 0x8001)]).view(np.float32)
    special = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 3.3895314e38, 3.4028235e38,
                        1.0e-45, -1.0e-45, 65504.0], np.float32)
    for v in vals + [ties, near, special]:
        np.testing.assert_array_equal(O.round_bf16(v).view(np.uint32), _torch_bf16(v).view(np.uint32))


def test_round_bf16_nan_stays_nan():
    v = np.array([np.nan, -np.nan], np.float32)
    assert np.isnan(O.round_bf16(v)).all()
    assert O.bf16_bits(np.array([np.nan], np.float32))[0] & 0x7F80 == 0x7F80


def test_bf16_bits_roundtrip_all_finite_patterns():
    bits = np.arange(0, 2**16, dtype=np.uint32).astype(np.uint16)
    f = O.bf16_from_bits(bits)
    finite = np.isfinite(f)
    np.testing.assert_array_equal(O.bf16_bits(f[finite]), bits[finite])


# ---------------------------------------------------------------------------
# fp8 e4m3fn codec
# ---------------------------------------------------------------------------

def test_e4m3_decode_closed_form_and_torch():
    codes = np.arange(256, dtype=np.uint8)
    got = O.e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert nan.sum() == 2 and np.isnan(got[nan]).all()
    np.testing.assert_array_equal(got[~nan], ref[~nan])
    # spot values from the format definition
    assert got[0x7E] == 448.0 and got[0xFE] == -448.0
    assert got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6
    assert got[0x38] == 1.0 and got[0x3C] == 1.5


def test_e4m3_encode_matches_torch_rne_within_range():
    codes = np.arange(0, 0x7F, dtype=np.uint8)
    vals = O.e4m3_decode(codes).astype(np.float64)
    mids = (vals[:-1] + vals[1:]) / 2
    grid = np.concatenate([vals, mids, mids * (1 + 1e-6), mids * (1 - 1e-6),
                           rng.uniform(0, 448, 20000)])
    grid = np.concatenate([grid, -grid]).astype(np.float32)
    grid = grid[np.abs(grid) <= 448]
    got = O.e4m3_encode(grid)
    ref = torch.from_numpy(grid).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(got, ref)


def test_e4m3_encode_saturates_and_roundtrips():
    assert O.e4m3_encode(np.array([1e6], np.float32))[0] == 0x7E
    assert O.e4m3_encode(np.array([-1e6], np.float32))[0] == 0xFE
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    np.testing.assert_array_equal(O.e4m3_encode(O.e4m3_decode(codes)), codes)


def test_quantize_per_channel_scale_and_error_bound():
    w = (rng.normal(size=(512, 96)) / math.sqrt(512)).astype(np.float32)
    q, s = O.quantize_per_channel(w, axis=0)
    assert q.shape == w.shape and s.shape == (96,)
    np.testing.assert_allclose(s, np.abs(w).max(axis=0) / 448, rtol=1e-6)
    deq = O.e4m3_decode(q) * s
    # the column max maps exactly to 448 -> exact reconstruction there
    cols = np.arange(96)
    rows = np.abs(w).argmax(axis=0)
    np.testing.assert_allclose(deq[rows, cols], w[rows, cols], rtol=1e-6)
    # normal range: relative error <= 2^-4 (half an ulp of 3 mantissa bits)
    big = np.abs(w / s) >= 2.0 ** -6
    assert np.all(np.abs(deq - w)[big] <= np.abs(w)[big] * 2.0 ** -4 * 1.0001)


def test_quantize_rows_e4m3_codes_scale_and_zero_rows():
    a = (rng.normal(size=(64, 300)) * rng.uniform(0.01, 50, size=(64, 1))).astype(np.float32)
    a[5] = 0.0
    q, s = O.quantize_rows_e4m3(a)
    assert q.shape == a.shape and q.dtype == np.uint8 and s.shape == (64,)
    amax = np.abs(a).max(axis=1)
    np.testing.assert_allclose(s[amax > 0], amax[amax > 0] / 448, rtol=1e-6)
    assert s[5] == 1.0 and not q[5].any()
    # codes: torch's own e4m3fn cast of the row scaled by 448 / amax (float32)
    inv = (np.float32(448.0) / np.where(amax > 0, amax, 1)).astype(np.float32)[:, None]
    ref = torch.from_numpy((a * inv).astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(q, ref)
    # every element within half an e4m3 step of its code's value (normal range:
    # 2^-4 relative; subnormal range: half of 2^-9 absolute, in scaled units)
    deq = O.e4m3_decode(q).astype(np.float64)
    scaled = (a * inv).astype(np.float64)
    err = np.abs(deq - scaled)
    normal = np.abs(scaled) >= 2.0 ** -6
    assert np.all(err[normal] <= np.abs(scaled)[normal] * 2.0 ** -4 * 1.0001)
    assert np.all(err[~normal] <= 2.0 ** -10 * 1.0001)
    # the row max lands on 448 exactly
    rows = np.nonzero(amax > 0)[0]
    np.testing.assert_array_equal(np.abs(deq[rows, np.abs(a[rows]).argmax(axis=1)]), 448.0)


def test_svd_mlp_fp8_act_ref_fixed_point_and_budget():
    r = np.random.default_rng(7)
    T, d, ff, rk = 24, 64, 160, 32
    f = [(r.normal(size=s) / np.sqrt(s[0])).astype(np.float32)
         for s in ((d, rk), (rk, ff), (d, rk), (rk, ff), (ff, rk), (rk, d))]
    x = O.round_bf16(r.normal(size=(T, d)).astype(np.float32))
    ref = O.svd_mlp_ref(x, *f, dtype="bfloat16")
    got = O.svd_mlp_fp8_act_ref(x, *f)
    # the one extra e4m3 rounding of h: above the bf16 level, within the fp8 budget
    err = O.relative_l2(got, ref)
    assert 5e-3 < err < 3e-2, err
    # h already on its rows' e4m3 grid: quantising again changes nothing, so
    # the down half sees exactly h (the dequantised grid is a fixed point)
    h = O.fused_gate_up_ref(x, *f[:4], dtype="bfloat16")
    q, sc = O.quantize_rows_e4m3(h)
    hq = (O.e4m3_decode(q) * sc[:, None]).astype(np.float32)
    q2, sc2 = O.quantize_rows_e4m3(hq)
    np.testing.assert_array_equal(q2, q)
    np.testing.assert_allclose(O.e4m3_decode(q2) * sc2[:, None], hq, rtol=1e-6)


# ---------------------------------------------------------------------------
# silu
# ---------------------------------------------------------------------------

def test_silu_closed_form_special_cases_and_identity():
    x = np.concatenate([rng.normal(size=10000) * 10, [0.0, 1e-30, -1e-30, 80.0, -80.0, 1e4, -1e4]]).astype(np.float32)
    got = O.silu(x).astype(np.float64)
    x64 = x.astype(np.float64)
    with np.errstate(over="ignore"):
        ref = x64 / (1.0 + np.exp(-x64))
    np.testing.assert_allclose(got, ref, rtol=3e-7, atol=1e-37)
    assert O.silu(np.float32(0.0)) == 0.0
    assert O.silu(np.float32(1e4)) == np.float32(1e4)          # silu(x) -> x
    assert -1e-30 < O.silu(np.float32(-1e4)) <= 0.0              # silu(x) -> 0-
    s = rng.normal(size=1000).astype(np.float32) * 5
    np.testing.assert_allclose(O.silu(s).astype(np.float64) - O.silu(-s).astype(np.float64), s, atol=2e-6)
    t = torch.nn.functional.silu(torch.from_numpy(x)).numpy()
    ulps = np.abs(O.silu(x) - t) / np.spacing(np.abs(t).astype(np.float32))
    assert np.max(ulps) <= 4.0  # both are within ~2 ulp of the float64 value


# ---------------------------------------------------------------------------
# low_rank_dim known answers
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("H,I,c,expected", [
    (2048, 8192, 0.8, 1280),     # reference.py:29-31 (1B)
    (3072, 8192, 0.8, 1792),     # 3B
    (4096, 14336, 0.8, 2560),    # 8B
    (4096, 14336, 0.9, 2816),    # models/README.md:67 checkpoint rank
    (4096, 14336, 1.0, 3200),    # e2e_block.py:324, 2816/3200 = 0.88
])
def test_low_rank_dim_known_answers(H, I, c, expected):
    assert O.low_rank_dim(H, I, c) == expected


def test_low_rank_dim_half_even():
    # I*H*c / ((I+H)*128) == 2.5 exactly -> round-half-even gives 2
    H = I = 640
    assert 640 * 640 * 1.0 / (1280 * 128) == 2.5
    assert O.low_rank_dim(H, I, 1.0) == 256
    # 3.5 -> 4
    assert 896 * 896 / (1792 * 128) == 3.5
    assert O.low_rank_dim(896, 896, 1.0) == 512


# ---------------------------------------------------------------------------
# the GEMM chains, brute force in float64
# ---------------------------------------------------------------------------

def _brute_gate_up(x, ug, vg, uu, vu):
    S, H = x.shape
    r, I = vg.shape
    out = np.zeros((S, I))
    for s in range(S):
        xug = [sum(float(x[s, h]) * float(ug[h, k]) for h in range(H)) for k in range(r)]
        xuu = [sum(float(x[s, h]) * float(uu[h, k]) for h in range(H)) for k in range(r)]
        for i in range(I):
            g = sum(xug[k] * float(vg[k, i]) for k in range(r))
            u = sum(xuu[k] * float(vu[k, i]) for k in range(r))
            out[s, i] = g / (1.0 + math.exp(-g)) * u
    return out


def _brute_xuv(x, u, v):
    S, I = x.shape
    r, H = v.shape
    out = np.zeros((S, H))
    for s in range(S):
        xu = [sum(float(x[s, i]) * float(u[i, k]) for i in range(I)) for k in range(r)]
        for h in range(H):
            out[s, h] = sum(xu[k] * float(v[k, h]) for k in range(r))
    return out


def _small(shapes, seed=7):
    g = np.random.default_rng(seed)
    return [(g.normal(size=s) / math.sqrt(s[0])).astype(np.float32) for s in shapes]


def test_gate_up_brute_force_distinguishes_gate_from_up():
    x, ug, vg, uu, vu = _small([(3, 5), (5, 4), (4, 6), (5, 4), (4, 6)])
    got = O.fused_gate_up_ref(x, ug, vg, uu, vu)
    np.testing.assert_allclose(got, _brute_gate_up(x, ug, vg, uu, vu), rtol=1e-5, atol=1e-6)
    swapped = O.fused_gate_up_ref(x, uu, vu, ug, vg)  # silu on the other branch
    assert not np.allclose(swapped, got, rtol=1e-3)


def test_xuv_brute_force_and_associativity():
    x, u, v = _small([(4, 7), (7, 3), (3, 5)])
    got = O.fused_xuv_ref(x, u, v)
    np.testing.assert_allclose(got, _brute_xuv(x, u, v), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(got, x.astype(np.float64) @ (u.astype(np.float64) @ v), rtol=1e-5, atol=1e-6)


def test_identity_u_reduces_to_dense_mlp():
    H, I = 8, 12
    x, wg, wu, wd = _small([(5, H), (H, I), (H, I), (I, H)])
    eye = np.eye(H, dtype=np.float32)
    eye_i = np.eye(I, dtype=np.float32)
    svd = O.svd_mlp_ref(x, eye, wg, eye, wu, eye_i, wd)
    np.testing.assert_allclose(svd, O.dense_mlp_ref(x, wg, wu, wd), rtol=1e-6, atol=1e-7)


def test_zero_u_and_linearity_in_v_up():
    x, ug, vg, uu, vu = _small([(4, 9), (9, 5), (5, 11), (9, 5), (5, 11)])
    assert np.all(O.fused_gate_up_ref(x, ug * 0, vg, uu, vu) == 0)
    assert np.all(O.fused_gate_up_ref(x, ug, vg, uu * 0, vu) == 0)
    a = O.fused_gate_up_ref(x, ug, vg, uu, vu)
    b = O.fused_gate_up_ref(x, ug, vg, uu, 2.5 * vu)
    np.testing.assert_allclose(b, 2.5 * a, rtol=1e-5, atol=1e-7)


def test_svd_mlp_rounds_h_between_halves():
    x, ug, vg, uu, vu, ud, vd = [O.round_bf16(a) for a in _small(
        [(6, 32), (32, 16), (16, 48), (32, 16), (16, 48), (48, 16), (16, 32)])]
    h = O.fused_gate_up_ref(x, ug, vg, uu, vu, "bfloat16")
    assert np.array_equal(h, O.round_bf16(h))
    np.testing.assert_array_equal(O.svd_mlp_ref(x, ug, vg, uu, vu, ud, vd, "bfloat16"),
                                  O.fused_xuv_ref(h, ud, vd, "bfloat16"))
    # and the fp32 golden arm (up-first order) differs from it only by rounding
    gold = O.unfused_reference(x, uu, vu, ug, vg, ud, vd)
    assert O.relative_l2(O.svd_mlp_ref(x, ug, vg, uu, vu, ud, vd, "bfloat16"), gold) < 1e-2


def test_unfused_reference_argument_order_is_up_first():
    x, a, b, c, d, ud, vd = _small([(3, 8), (8, 4), (4, 8), (8, 4), (4, 8), (8, 4), (4, 8)], seed=3)
    # unfused_reference(x, u_up, v_up, u_gate, v_gate, ...) == svd_mlp_ref(x, ug, vg, uu, vu, ...)
    np.testing.assert_allclose(O.unfused_reference(x, a, b, c, d, ud, vd),
                               O.svd_mlp_ref(x, c, d, a, b, ud, vd), rtol=1e-6, atol=1e-7)


# ---------------------------------------------------------------------------
# RMSNorm and the block
# ---------------------------------------------------------------------------

def test_rmsnorm_closed_forms():
    d = 64
    gain = rng.uniform(0.9, 1.1, size=d).astype(np.float32)
    row = np.full((1, d), -3.0, np.float32)          # rms = 3 -> normalised = -1
    np.testing.assert_allclose(O.rmsnorm_ref(row, gain, eps=0.0), -gain[None], rtol=1e-6)
    x = rng.normal(size=(5, d)).astype(np.float32)
    np.testing.assert_allclose(O.rmsnorm_ref(7.0 * x, gain, eps=0.0), O.rmsnorm_ref(x, gain, eps=0.0), rtol=2e-6)
    x64 = x.astype(np.float64)
    brute = gain * x64 / np.sqrt(np.mean(x64 ** 2, axis=1, keepdims=True) + 1e-5)
    np.testing.assert_allclose(O.rmsnorm_ref(x, gain), brute, rtol=2e-6)


def test_mlp_block_is_residual_plus_mlp_of_norm():
    d, ff, r = 16, 24, 8
    x = rng.normal(size=(3, d)).astype(np.float32)
    gain = np.ones(d, np.float32)
    f = _small([(d, r), (r, ff), (d, r), (r, ff), (ff, r), (r, d)])
    y = O.mlp_block_ref(x, gain, f)
    np.testing.assert_allclose(y, x + O.svd_mlp_ref(O.rmsnorm_ref(x, gain), *f), rtol=1e-6, atol=1e-7)


def test_mlp_block_f64_brute_force():
    """The unrounded float64 block against Python-float loops (RMSNorm by
    hand, the brute-force GEMM chains), and against the float32 block."""
    d, ff, r = 6, 7, 3
    x = rng.normal(size=(2, d))
    gain = rng.uniform(0.9, 1.1, size=d)
    f = [a.astype(np.float64) for a in _small([(d, r), (r, ff), (d, r), (r, ff), (ff, r), (r, d)], seed=11)]
    hn = np.zeros_like(x)
    for s_ in range(2):
        rms = math.sqrt(sum(float(v) ** 2 for v in x[s_]) / d + 1e-5)
        hn[s_] = [gain[j] * x[s_, j] / rms for j in range(d)]
    want = x + _brute_xuv(_brute_gate_up(hn, *f[:4]), f[4], f[5])
    got = O.mlp_block_f64(x, gain, f, eps=1e-5)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    y32 = O.mlp_block_ref(x.astype(np.float32), gain.astype(np.float32), [a.astype(np.float32) for a in f])
    np.testing.assert_allclose(y32, got, rtol=2e-5, atol=2e-6)


# ---------------------------------------------------------------------------
# metrics and accounting
# ---------------------------------------------------------------------------

def test_relative_l2_hand_values_and_nan_rejection():
    assert O.relative_l2(np.array([3.0, 4.0]), np.array([0.0, 0.0])) == pytest.approx(5.0 / 1e-12)
    assert O.relative_l2(np.array([1.0, 1.0]), np.array([1.0, 0.0])) == pytest.approx(1.0)
    e = O.errors(np.array([[1.0, 2.0]]), np.array([[1.0, 4.0]]))
    assert e["max_abs_error"] == 2.0 and e["relative_l2"] == pytest.approx(2 / math.sqrt(17))
    with pytest.raises(FloatingPointError):
        O.relative_l2(np.array([np.nan]), np.array([1.0]))
    with pytest.raises(ValueError, match="shape mismatch"):
        O.relative_l2(np.zeros(3), np.zeros(4))


def test_factor_bytes_known_answer():
    # tests_test_profiler.py.before:20 -- 297 MiB; results/real_layer0_cpu.json:21
    assert O.factor_bytes(4096, 14336, 2816) == 311_427_072
    assert O.factor_bytes(4096, 14336, 2816) // 2**20 == 297


def test_layer_flops_matches_baseline_table():
    assert O.layer_flops(1024, 4096, 14336, 2816) / 1e9 == pytest.approx(318.90, abs=0.01)
    assert O.layer_flops(2048, 8192, 28672, 5632) / 1e9 == pytest.approx(2551.2, abs=0.1)
