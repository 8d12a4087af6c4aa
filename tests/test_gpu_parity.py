"""Parity of the HIP kernels (through libsvdmlp.so's C ABI) with the CPU
oracle on seeded inputs.

Tolerances (relative Frobenius error against the oracle's math on the same
inputs): bf16 1e-2 and fp8 3e-2; fp32 1e-4
element-wise (tests_test_speedup_migration.py.before:23-25).  Full-size
shapes are checked on a row subset: the rows of the layer are independent, so
any subset is an exact parity check of those rows.
"""

import numpy as np
import pytest
import torch

import oracle as O
from svdmlp import compat, fp8, inputs, ops

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2
FP8_TOL = 3e-2
GEMV_LAYER_MAX_T = 2   # kGvMaxT in csrc/decode_gemv.hpp
# kDlContractAutoPadded / kDlContractAutoDense in csrc/api.hip: the contracted
# decode layer by default up to 2 tokens with padded factor rows, up to 3 with
# dense factors (_contracted)
CONTRACT_AUTO_T = {True: 2, False: 3}


def _mfma_layer(shape):
    """Whether the MFMA decode layers take a bf16 natural-layout shape (d and
    ranks multiples of 128, ff of 64)."""
    return shape.d % 128 == 0 and shape.r % 128 == 0 and shape.rd % 128 == 0 and shape.ff % 64 == 0


def _p2split_fits(shape, cus=256, max_tiles=384):
    """Whether the MFMA decode layer can run one-branch phase-2 units (ff in
    whole 128-column tiles, a block per unit, a counter per column tile): with
    dense factors it then takes every decode token count."""
    nt2 = shape.ff // 128
    return (shape.ff % 128 == 0 and 2 * nt2 <= cus
            and 2 * (shape.r // 128) + shape.rd // 128 + shape.d // 128 + nt2 <= max_tiles)


def _contracted(shape, T, padded=False):
    """Whether a bf16 natural-layout call runs the contracted decode layer by
    default: its token counts, d and ranks multiples of 128, ff of 64, gate/up
    rank >= 320, a block per h strip and per XU_d tile (256 CUs)."""
    return (T <= CONTRACT_AUTO_T[padded] and _mfma_layer(shape) and shape.r >= 320
            and shape.ff // 64 + shape.rd // 128 <= 256)


def _dl_barriers(T, contracted):
    """Grid barriers of one persistent MFMA decode-layer launch on the 8B and
    test shapes (phase 1 waits for the RMSNorm rows' ready flags in the MLP
    block): the contracted layer keeps the one before phase 2 (phase 4
    waits for its XU_d tiles' ready flags); the four-phase layer the one
    before phase 3 (phase 2 waits for one flag for all of XU at one 16-row
    token tile, for its XU tiles' flags from two tiles up; phase 4 for its
    XU_d tiles' flags), at eight tiles an arrival-only one after phase 1
    (phase 3 waits for its K split's h flag)."""
    return 1


def _gemv_layer(shape, T):
    """Whether a dense bf16 call at decode shapes runs the streaming-GEMV
    layer by default (up to 2 tokens, where neither MFMA layer runs)."""
    return T <= GEMV_LAYER_MAX_T and not _contracted(shape, T) and not (_mfma_layer(shape) and _p2split_fits(shape))


def _to(a, dtype, dev):
    return inputs.to_torch(a, dtype, dev)


def _np(t):
    return t.float().cpu().numpy()


def _rounded(arrs, dtype):
    return [inputs.as_float32(a, dtype) for a in arrs]


def _rel(got, ref):
    return O.relative_l2(got, ref)


def _small(shapes, seed=123):
    rng = np.random.default_rng(seed)
    return [(rng.normal(size=s) / np.sqrt(s[0])).astype(np.float32) for s in shapes]


# ---------------------------------------------------------------------------
# small and odd shapes (tests_test_speedup_migration.py.before:47-92)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("S,H,R,I", [(1, 129, 131, 137), (129, 257, 257, 513), (3, 64, 32, 96)])
def test_fused_gate_and_down_tail_blocks_fp32(gpu, S, H, R, I):
    x, ug, vg, uu, vu, ud, vd = _small([(S, H), (H, R), (R, I), (H, R), (R, I), (I, R), (R, H)])
    t = [_to(a, torch.float32, gpu) for a in (x, ug, vg, uu, vu, ud, vd)]
    got_t = compat.fused_mlp_up_T(t[0], t[1], t[2], t[3], t[4])
    hidden = O.fused_gate_up_ref(x, ug, vg, uu, vu)
    assert tuple(got_t.shape) == (I, S)
    np.testing.assert_allclose(_np(got_t), hidden.T, atol=1e-4, rtol=1e-4)
    got = compat.fused_three_mm_XTUV(got_t, t[5], t[6])
    assert tuple(got.shape) == (S, H)
    np.testing.assert_allclose(_np(got), O.fused_xuv_ref(hidden, ud, vd), atol=1e-4, rtol=1e-4)


def test_multiple_inner_tiles_fp32(gpu):
    x, ug, vg, uu, vu = _small([(257, 513), (513, 513), (513, 1025), (513, 513), (513, 1025)])
    t = [_to(a, torch.float32, gpu) for a in (x, ug, vg, uu, vu)]
    got = compat.fused_mlp_up_T(*t, M_tiles_in_block=2, r_tiles_in_block=2, K_tiles_in_block=2,
                                N_tiles_in_block=2, async_dma=False)
    np.testing.assert_allclose(_np(got), O.fused_gate_up_ref(x, ug, vg, uu, vu).T, atol=1e-4, rtol=1e-4)


def test_wrappers_preserve_pytorch_weight_order_fp32(gpu):
    x, uu, vu, ug, vg, ud, vd = _small([(1, 129), (129, 131), (131, 137), (129, 131), (131, 137),
                                        (137, 131), (131, 129)])
    t = [_to(a, torch.float32, gpu) for a in (x, uu, vu, ug, vg, ud, vd)]
    # nki_mm takes PyTorch Linear weights (out, in): contiguous transposes.
    lin = [a.t().contiguous() for a in t[1:]]
    got = compat.nki_mm(t[0], *lin)
    expected = O.unfused_reference(x, uu, vu, ug, vg, ud, vd)
    np.testing.assert_allclose(_np(got), expected, atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("S,H,R,I", [(5, 136, 64, 200), (130, 256, 136, 520), (64, 128, 64, 256)])
def test_bf16_small_shapes_all_entry_points(gpu, S, H, R, I):
    f = _rounded(_small([(S, H), (H, R), (R, I), (H, R), (R, I), (I, R), (R, H)], seed=S), torch.bfloat16)
    x, ug, vg, uu, vu, ud, vd = f
    t = [_to(a, torch.bfloat16, gpu) for a in f]
    h_ref = O.fused_gate_up_ref(x, ug, vg, uu, vu, "bfloat16")
    assert _rel(_np(ops.fused_gate_up(t[0], t[1], t[2], t[3], t[4])), h_ref) < BF16_TOL
    assert _rel(_np(ops.fused_xuv(_to(h_ref, torch.bfloat16, gpu), t[5], t[6])),
                O.fused_xuv_ref(h_ref, ud, vd, "bfloat16")) < BF16_TOL
    assert _rel(_np(ops.svd_mlp(*t)), O.svd_mlp_ref(*f, dtype="bfloat16")) < BF16_TOL


def test_bf16_odd_shapes_take_the_unaligned_path(gpu):
    f = _rounded(_small([(7, 129), (129, 131), (131, 137), (129, 131), (131, 137), (137, 131), (131, 129)]),
                 torch.bfloat16)
    t = [_to(a, torch.bfloat16, gpu) for a in f]
    assert _rel(_np(ops.svd_mlp(*t)), O.svd_mlp_ref(*f, dtype="bfloat16")) < BF16_TOL


# ---------------------------------------------------------------------------
# the tiny layer (T=128, d=1024, ff=3584, r=256), fp32
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def tiny():
    x, f = inputs.make_layer(inputs.SHAPES["tiny"], T=128, seed=0)
    return x, f


def test_tiny_config_fp32(gpu, tiny):
    x, f = tiny
    t = [_to(a, torch.float32, gpu) for a in (x, *f)]
    got = _np(ops.svd_mlp(*t))
    ref = O.svd_mlp_ref(x, *f)
    np.testing.assert_allclose(got, ref, atol=1e-4, rtol=1e-4)
    assert _rel(got, ref) < 1e-5
    h = _np(ops.fused_gate_up(*t[:5]))
    np.testing.assert_allclose(h, O.fused_gate_up_ref(x, *f[:4]), atol=1e-4, rtol=1e-4)


def test_tiny_config_bf16(gpu, tiny):
    x, f = tiny
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    got = _np(ops.svd_mlp(*t))
    err = _rel(got, O.svd_mlp_ref(xb, *fb, dtype="bfloat16"))
    assert err < BF16_TOL, err
    # and against the fp32 golden arm of test_speedup.py (unrounded h)
    assert _rel(got, O.unfused_reference(xb, fb[2], fb[3], fb[0], fb[1], fb[4], fb[5])) < BF16_TOL


# ---------------------------------------------------------------------------
# BASELINE configs 2 and 3: LLaMA3-8B layer, prefill T=1024 and decode T<=64
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def layer8b(gpu):
    shape = inputs.SHAPES["8b"]
    f = _rounded(inputs.make_factors(shape, seed=0), torch.bfloat16)
    ft = [_to(a, torch.bfloat16, gpu) for a in f]
    return shape, f, ft


def _x(T, d, seed):
    return inputs.as_float32(inputs.make_x(np.random.default_rng(seed), T, d), torch.bfloat16)


def test_8b_prefill_T1024_row_subset(gpu, layer8b):
    shape, f, ft = layer8b
    x = _x(1024, shape.d, 11)
    xt = _to(x, torch.bfloat16, gpu)
    y = ops.svd_mlp(xt, *ft)
    rows = np.r_[0:16, 120:136, 1008:1024, np.random.default_rng(0).choice(1024, 16, replace=False)]
    ref = O.svd_mlp_ref(x[rows], *f, dtype="bfloat16")
    got = _np(y)[rows]
    err = _rel(got, ref)
    print(f"8b T=1024 svd_mlp rel_l2={err:.3e}")
    assert err < BF16_TOL
    assert np.isfinite(_np(y)).all()
    h = ops.fused_gate_up(xt, *ft[:4])
    err_h = _rel(_np(h)[rows], O.fused_gate_up_ref(x[rows], *f[:4], dtype="bfloat16"))
    assert err_h < BF16_TOL, err_h


@pytest.mark.parametrize("T", [1, 2, 4, 8, 32, 64, 65, 128])
def test_8b_decode(gpu, layer8b, T):
    shape, f, ft = layer8b
    x = _x(T, shape.d, 100 + T)
    xt = _to(x, torch.bfloat16, gpu)
    ref = O.svd_mlp_ref(x, *f, dtype="bfloat16")
    err = _rel(_np(ops.svd_mlp(xt, *ft)), ref)
    print(f"8b decode T={T} rel_l2={err:.3e}")
    assert err < BF16_TOL
    h_ref = O.fused_gate_up_ref(x, *f[:4], dtype="bfloat16")
    h = ops.fused_gate_up(xt, *ft[:4])
    assert _rel(_np(h), h_ref) < BF16_TOL
    y = ops.fused_xuv(_to(h_ref, torch.bfloat16, gpu), ft[4], ft[5])
    assert _rel(_np(y), O.fused_xuv_ref(h_ref, f[4], f[5], "bfloat16")) < BF16_TOL


@pytest.mark.parametrize("T", [65, 128, 200, 256, 300, 512, 777])
def test_prefill_token_counts(gpu, T):
    """Token counts change the tile count, hence the split-K plan (and the
    partial-slice reduction) of every large-tile stage."""
    shape = inputs.LayerShape(1024, 2048, 512, 384)
    x, f = inputs.make_layer(shape, T=T, seed=T)
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    got = _np(ops.svd_mlp(*t))
    assert np.isfinite(got).all()
    err = _rel(got, O.svd_mlp_ref(xb, *fb, dtype="bfloat16"))
    assert err < BF16_TOL, err
    h = _np(ops.fused_gate_up(*t[:5]))
    assert _rel(h, O.fused_gate_up_ref(xb, *fb[:4], dtype="bfloat16")) < BF16_TOL
    hb = inputs.as_float32(h, torch.bfloat16)
    y = _np(ops.fused_xuv(_to(hb, torch.bfloat16, gpu), t[5], t[6]))
    assert _rel(y, O.fused_xuv_ref(hb, fb[4], fb[5], "bfloat16")) < BF16_TOL


def _barrier_state(ws):
    """(generation, timeout flag) of the decode kernel's barrier words (the
    64-bit words at bytes 2176 and 2304 of the sync area)."""
    w = ws[:4096].view(torch.int64).cpu().tolist()
    return w[272], w[288]


def _set_spin_bound(ws, polls):
    """The bound of the persistent kernels' barrier waits (the 32-bit word at
    byte 2312 of the sync area; 0 = the kernels' default)."""
    ws[2312:2316].view(torch.int32).fill_(polls)


def _tile_counters(ws):
    """The MFMA decode layer's split-K tile arrival counters (32-bit words
    from byte 2560 of the workspace's sync area to its end)."""
    return ws[2560:4096].view(torch.int32).cpu().tolist()


@pytest.mark.parametrize("shape,Ts", [
    (inputs.LayerShape(1024, 2048, 512), (1, 3, 2, 17, 40, 64, 100, 16, 128)),  # every token-tile count, reused workspace
    (inputs.LayerShape(1024, 32768, 256), (5, 33)),                     # 512 column tiles: two units per block
    (inputs.LayerShape(16640, 1024, 128), (8, 64)),                     # 130 output tiles: phase 4 unsplit
])
def test_decode_layer_workspace_reuse(gpu, shape, Ts):
    """The persistent decode kernels (the contracted layer at 1-3 tokens of
    dense factors, the four-phase MFMA layer above them, the streaming-GEMV
    layer up to 2 tokens where neither MFMA layer runs; one launch
    each, grid barriers and split-K tile
    counters in the workspace's first 4096 bytes) over one reused workspace:
    results match the oracle, every call advances the shared barrier
    generation by its barriers, no barrier times out and every tile counter
    is back at zero."""
    x, f = inputs.make_layer(shape, T=max(Ts), seed=31)
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    ws = ops.svd_mlp_workspace(t[0], r=shape.r, ff=shape.ff)
    gen = 0
    for T in Ts:
        y = _np(ops.svd_mlp(t[0][:T].contiguous(), *t[1:], workspace=ws))
        err = _rel(y, O.svd_mlp_ref(xb[:T], *fb, dtype="bfloat16"))
        assert err < BF16_TOL, (T, err)
        # GEMV layer: 4 barriers, the MFMA layers _dl_barriers
        gen += 4 if _gemv_layer(shape, T) else _dl_barriers(T, _contracted(shape, T))
        assert _barrier_state(ws) == (gen, 0), T
        assert not any(_tile_counters(ws)), T


def test_shared_workspace_across_calls(gpu):
    """Calls without a workspace share one per (device, stream), grown on
    demand: decode, prefill and decode again on it, every result the
    oracle's, its barrier words consistent."""
    from svdmlp import ops

    ops.clear_workspace_cache()
    shape = inputs.LayerShape(1024, 2048, 512)
    x, f = inputs.make_layer(shape, T=300, seed=91)
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    for T in (8, 300, 8, 64):
        y = _np(ops.svd_mlp(t[0][:T].contiguous(), *t[1:]))
        assert _rel(y, O.svd_mlp_ref(xb[:T], *fb, dtype="bfloat16")) < BF16_TOL, T
    (ws,) = ops._WS_CACHE.values()
    assert ws.numel() >= ops._lib.workspace_bytes(300, shape.d, shape.ff, shape.r, ops._lib.SVDMLP_BF16)
    assert _barrier_state(ws)[1] == 0 and not any(_tile_counters(ws))
    ops.clear_workspace_cache()
    assert not ops._WS_CACHE


def test_prepared_layer_cache(gpu):
    """A layer called again reuses its prepared arguments (the same bits:
    split-K partial sums are added in split order); layers whose factors the
    host mirror copies (gate and up with different row pitches) are not
    kept."""
    from svdmlp import ops

    ops._PLANS.clear()
    shape = inputs.LayerShape(1024, 2048, 512)
    x, f = inputs.make_layer(shape, T=8, seed=95)
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    y1 = ops.svd_mlp(*t).clone()
    assert len(ops._PLANS) == 1
    y2 = ops.svd_mlp(*t)
    assert torch.equal(y2.view(torch.int16), y1.view(torch.int16))
    assert _rel(_np(y2), O.svd_mlp_ref(xb, *fb, dtype="bfloat16")) < BF16_TOL
    mixed = list(t[1:])
    mixed[0], mixed[2] = ops.pad_rows(t[1], 8), ops.pad_rows(t[3], 16)
    y3 = _np(ops.svd_mlp(t[0], *mixed))
    assert len(ops._PLANS) == 1
    assert _rel(y3, O.svd_mlp_ref(xb, *fb, dtype="bfloat16")) < BF16_TOL


@pytest.mark.parametrize("T", [1, 2])
def test_gemv_decode_layer_ragged_strips(gpu, T):
    """Streaming-GEMV layer on a shape whose column counts cut its 256- and
    512-column strips (400, 272, 1040, 2064) and whose row counts are only
    multiples of 16: partial strips, ranges that start mid-strip, and block
    ranges that cross from one factor into the other."""
    shape = inputs.LayerShape(1040, 2064, 400, 272)
    x, f = inputs.make_layer(shape, T=T, seed=60 + T)
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    ws = ops.svd_mlp_workspace(t[0], r=shape.r, ff=shape.ff)
    y = _np(ops.svd_mlp(*t, workspace=ws))
    err = _rel(y, O.svd_mlp_ref(xb, *fb, dtype="bfloat16"))
    print(f"gemv layer T={T} rel_l2={err:.3e}")
    assert err < BF16_TOL
    assert _barrier_state(ws) == (4, 0)


def test_decode_and_prefill_paths_agree(gpu, layer8b):
    """T=64 and T=128 run the persistent decode layer (16- and 128-row token
    tiles), T=256 the tiled GEMMs; the first 64 rows of the three must agree
    with each other and with the oracle."""
    shape, f, ft = layer8b
    x = _x(256, shape.d, 7)
    y256 = _np(ops.svd_mlp(_to(x, torch.bfloat16, gpu), *ft))
    y128 = _np(ops.svd_mlp(_to(x[:128], torch.bfloat16, gpu), *ft))
    y64 = _np(ops.svd_mlp(_to(x[:64], torch.bfloat16, gpu), *ft))
    ref = O.svd_mlp_ref(x[:64], *f, dtype="bfloat16")
    for y in (y64, y128[:64], y256[:64]):
        assert _rel(y, ref) < BF16_TOL
    assert _rel(y64, y256[:64]) < 5e-3 and _rel(y128[:64], y256[:64]) < 5e-3


def test_linear_layout_weights_bf16(gpu, layer8b):
    """nki_mm-style (out, in) weights: the .T views reach the kernels
    without copies; prefill and decode paths."""
    shape, f, ft = layer8b
    lin = [a.t().contiguous().t() for a in ft]   # (in, out) views over (out, in) storage
    for T in (8, 256):
        x = _x(T, shape.d, 300 + T)
        rows = np.arange(min(T, 24))
        got = _np(ops.svd_mlp(_to(x, torch.bfloat16, gpu), *lin))[rows]
        assert _rel(got, O.svd_mlp_ref(x[rows], *f, dtype="bfloat16")) < BF16_TOL, T


@pytest.mark.parametrize("T,padded", [(1, True), (8, False), (48, False), (64, True), (100, True), (128, False),
                                     (300, False), (1024, True)])
def test_replay_is_bitwise_identical(gpu, layer8b, T, padded):
    """The analogue of the reference's async-vs-sync bitwise check
    (tests_test_speedup_migration.py.before:217-233): the same call
    repeated gives the same bits.  Split-K partial sums are added in split
    order on every path taken here (the MFMA decode layer up to 128 tokens,
    whichever unit arrives last, its phases started by ready flags; the
    large-tile path's ordered reductions above)."""
    shape, f, ft = layer8b
    xt = _to(_x(T, shape.d, 5 + T), torch.bfloat16, gpu)
    fs = [ops.pad_rows(a, 64) if padded and i % 2 else a for i, a in enumerate(ft)]
    ws = ops.svd_mlp_workspace(xt, r=shape.r, ff=shape.ff)
    ys = [ops.svd_mlp(xt, *fs, workspace=ws).clone() for _ in range(3 if T > 128 else 8)]
    for y in ys[1:]:
        assert torch.equal(y.view(torch.int16), ys[0].view(torch.int16)), T
    assert _rel(_np(ys[0])[: min(T, 16)], O.svd_mlp_ref(_np(xt)[: min(T, 16)], *f, dtype="bfloat16")) < BF16_TOL


@pytest.mark.parametrize("T,padded", [(1, True), (3, False), (8, False), (40, False), (100, True)])
def test_decode_activation_reads_through_the_caches(gpu, T, padded):
    """The MFMA decode layers (contracted at 1 token with padded rows) read the bf16
    activation tiles that other blocks of the same launch wrote (XU, h, XU_d)
    through the caches when the workspace is 128-byte aligned, device-scope
    when it is not.  On a layer small enough (3 MB of factors) that its lines
    stay in the L2s from one launch to the next, calls that alternate three
    inputs on one aligned workspace give, call after call, the bits of the
    device-scope reads of a workspace 16 bytes off alignment: no launch is
    served a line that an earlier launch cached."""
    shape = inputs.LayerShape(512, 1024, 384)
    _, f = inputs.make_layer(shape, T=T, seed=61)
    fb = _rounded(f, torch.bfloat16)
    ft = [_to(a, torch.bfloat16, gpu) for a in fb]
    fs = [ops.pad_rows(a, 64) if padded and i % 2 else a for i, a in enumerate(ft)]
    xs = [_to(_x(T, shape.d, 70 + i), torch.bfloat16, gpu) for i in range(3)]
    nb = ops.svd_mlp_workspace(xs[0], r=shape.r, ff=shape.ff).numel()
    aligned = torch.zeros(nb, dtype=torch.uint8, device=gpu)
    off = torch.zeros(nb + 16, dtype=torch.uint8, device=gpu)[16:]
    assert aligned.data_ptr() % 128 == 0 and off.data_ptr() % 128 == 16
    refs = [ops.svd_mlp(x, *fs, workspace=off).clone() for x in xs]
    for x, y in zip(xs, refs):
        assert _rel(_np(y), O.svd_mlp_ref(_np(x), *fb, dtype="bfloat16")) < BF16_TOL
    for i in range(30):
        y = ops.svd_mlp(xs[i % 3], *fs, workspace=aligned)
        assert torch.equal(y.view(torch.int16), refs[i % 3].view(torch.int16)), (T, i)
    assert _barrier_state(aligned)[1] == 0 and _barrier_state(off)[1] == 0


@pytest.mark.parametrize("shape,T,contracted", [
    (inputs.LayerShape(1024, 2048, 512), 8, False),        # MFMA decode layer
    (inputs.LayerShape(1024, 2048, 512), 48, False),       # four token tiles: XU and XU_d tiles' ready flags
    (inputs.LayerShape(1024, 2048, 512), 100, False),      # eight tiles: phase 3 on its K splits' h flags
    (inputs.LayerShape(1040, 2064, 400, 272), 1, False),   # streaming-GEMV layer
    (inputs.LayerShape(1040, 2064, 400, 272), 2, False),   # GEMV, ragged strips
    (inputs.LayerShape(1024, 2048, 512), 4, True),         # contracted layer (asked for): tile-combine waits too
    (inputs.LayerShape(1024, 2048, 512), 4, False)])       # four-phase layer, one-branch phase 2 at one token tile (dense)
def test_barrier_timeout_poisons_output_and_recovers(gpu, shape, T, contracted):
    """A persistent decode launch whose grid-barrier waits give up (forced
    from the host with a bound of one poll, so every block still runs to its
    end) writes NaN into y, reports the timeout through the workspace
    status, and the workspace works again once reset."""
    x, f = inputs.make_layer(shape, T=T, seed=80 + T)
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    ref = O.svd_mlp_ref(xb, *fb, dtype="bfloat16")
    ws = ops.svd_mlp_workspace(t[0], r=max(shape.r, shape.rd), ff=shape.ff)
    assert _rel(_np(ops.svd_mlp(*t, workspace=ws, contracted=contracted)), ref) < BF16_TOL
    assert ops.workspace_status(ws) is False
    _set_spin_bound(ws, 1)
    y = _np(ops.svd_mlp(*t, workspace=ws, contracted=contracted))
    assert np.isnan(y).all(), f"{np.isnan(y).mean():.3f} of y is NaN"
    assert ops.workspace_status(ws) is True
    assert ops.workspace_status(ws, reset=True) is True   # reports, then zeroes the sync area
    assert ops.workspace_status(ws) is False and _barrier_state(ws) == (0, 0)
    for _ in range(2):
        assert _rel(_np(ops.svd_mlp(*t, workspace=ws, contracted=contracted)), ref) < BF16_TOL
    assert ops.workspace_status(ws) is False


# ---------------------------------------------------------------------------
# the contracted layer (SVDMLP_CONTRACT; models/modeling_llama.py:865-886)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("T", [1, 2, 3, 4])
def test_contracted_decode_layer_8b(gpu, layer8b, T):
    """The contracted decode layer (each block's h strip kept in LDS and
    multiplied by its Ud rows; the (T, r_d) partials of XU_d summed in unit
    order by dedicated blocks) against the oracle, bitwise on replay, with
    dense and row-padded factors: one launch with one grid barrier per call,
    every tile counter back at zero."""
    shape, f, ft = layer8b
    xt = _to(_x(T, shape.d, 600 + T), torch.bfloat16, gpu)
    ref = O.svd_mlp_ref(_np(xt), *f, dtype="bfloat16")
    for fs in (ft, [ops.pad_rows(a, 64) if i % 2 else a for i, a in enumerate(ft)]):
        ws = ops.svd_mlp_workspace(xt, r=shape.r, ff=shape.ff)
        ys = [ops.svd_mlp(xt, *fs, workspace=ws, contracted=True).clone() for _ in range(3)]
        assert _barrier_state(ws) == (3 * _dl_barriers(T, True), 0) and not any(_tile_counters(ws))
        for y in ys[1:]:
            assert torch.equal(y.view(torch.int16), ys[0].view(torch.int16))
        err = _rel(_np(ys[0]), ref)
        print(f"contracted 8B T={T} rel_l2={err:.3e}")
        assert err < BF16_TOL
        assert _rel(_np(ys[0]), _np(ops.svd_mlp(xt, *fs, workspace=ws))) < 5e-3


@pytest.mark.parametrize("shape,T", [
    (inputs.LayerShape(1024, 2048, 512, 384), 1),   # 3 XU_d tiles: fewer than the ring depth
    (inputs.LayerShape(1024, 2048, 512, 384), 4),
    (inputs.LayerShape(3072, 8192, 1792), 2),       # the reference runner's default (3B) shape
    (inputs.LayerShape(1024, 2048, 512, 384), 8),   # beyond 4 tokens: the three-barrier layer
    (inputs.LayerShape(1024, 2048, 512, 384), 300)])
def test_contracted_svd_mlp_entry(gpu, shape, T):
    """pallas_ops.contracted_svd_mlp: the contracted layer at 1-4 tokens, the
    same y from the other paths elsewhere."""
    from svdmlp import pallas_ops

    x, f = inputs.make_layer(shape, T=T, seed=610 + T)
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    ws = ops.svd_mlp_workspace(t[0], r=max(shape.r, shape.rd), ff=shape.ff)
    y = _np(ops.svd_mlp(*t, workspace=ws, contracted=True))
    if T <= 128:
        assert _barrier_state(ws)[0] == _dl_barriers(T, T <= 4) and not any(_tile_counters(ws))
    ref = O.svd_mlp_ref(xb, *fb, dtype="bfloat16")
    assert _rel(y, ref) < BF16_TOL
    assert _rel(_np(pallas_ops.contracted_svd_mlp(*t)), ref) < BF16_TOL


# ---------------------------------------------------------------------------
# the reference's transposed launchers in bf16 (test_speedup.py:500-544)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("S,H,R,I", [(1, 136, 64, 200), (13, 264, 136, 520), (129, 256, 72, 392),
                                     (200, 1024, 256, 2048)])
def test_transposed_launchers_bf16(gpu, S, H, R, I):
    """fused_mlp_up_T returns (I, S); fused_three_mm_XTUV takes X as (I, S):
    bf16 against the oracle at 1e-2, on token counts that are and are not
    multiples of 8 (the latter leave the 16-byte vector path)."""
    f = _rounded(_small([(S, H), (H, R), (R, I), (H, R), (R, I), (I, R), (R, H)], seed=S + 7), torch.bfloat16)
    x, ug, vg, uu, vu, ud, vd = f
    t = [_to(a, torch.bfloat16, gpu) for a in f]
    hT = compat.fused_mlp_up_T(t[0], t[1], t[2], t[3], t[4])
    assert tuple(hT.shape) == (I, S) and hT.dtype == torch.bfloat16
    h_ref = O.fused_gate_up_ref(x, ug, vg, uu, vu, "bfloat16")
    assert _rel(_np(hT), h_ref.T) < BF16_TOL
    y = compat.fused_three_mm_XTUV(_to(np.ascontiguousarray(h_ref.T), torch.bfloat16, gpu), t[5], t[6])
    assert tuple(y.shape) == (S, H)
    assert _rel(_np(y), O.fused_xuv_ref(h_ref, ud, vd, "bfloat16")) < BF16_TOL
    if S % 8 == 0:
        # the 16-byte transpose (partial 64-row / 64-column tiles at S=200):
        # bitwise the natural-layout entry points' results
        h = ops.fused_gate_up(t[0], *t[1:5])
        assert torch.equal(hT.view(torch.int16), h.t().contiguous().view(torch.int16))
        hn = _to(h_ref, torch.bfloat16, gpu)
        yn = ops.fused_xuv(hn, t[5], t[6])
        assert torch.equal(y.view(torch.int16), yn.view(torch.int16))
    both = compat.svd_mlp_with_fused_kernel(t[0], t[3], t[4], t[1], t[2], t[5], t[6])
    assert _rel(_np(both), O.svd_mlp_ref(*f, dtype="bfloat16")) < BF16_TOL


def test_transposed_launchers_bf16_8b_shape(gpu, layer8b):
    """The same launchers on the LLaMA3-8B factors at S=128 (the reference's
    headline TPU shape, test_speedup.py:755)."""
    shape, f, ft = layer8b
    S = 128
    x = _x(S, shape.d, 900)
    xt = _to(x, torch.bfloat16, gpu)
    hT = compat.fused_mlp_up_T(xt, ft[0], ft[1], ft[2], ft[3])
    h_ref = O.fused_gate_up_ref(x, *f[:4], dtype="bfloat16")
    assert _rel(_np(hT), h_ref.T) < BF16_TOL
    y = compat.fused_three_mm_XTUV(hT, ft[4], ft[5])
    hb = inputs.as_float32(_np(hT).T, torch.bfloat16)
    assert _rel(_np(y), O.fused_xuv_ref(hb, f[4], f[5], "bfloat16")) < BF16_TOL
    assert _rel(_np(y), O.svd_mlp_ref(x, *f, dtype="bfloat16")) < BF16_TOL
    # the transposed operands ride on the natural-layout kernels (one transpose
    # pass each): bitwise the natural-layout entry points' results
    h = ops.fused_gate_up(xt, *ft[:4])
    assert torch.equal(hT.view(torch.int16), h.t().contiguous().view(torch.int16))
    yn = ops.fused_xuv(hT.t().contiguous(), ft[4], ft[5])
    assert torch.equal(y.view(torch.int16), yn.view(torch.int16))


# ---------------------------------------------------------------------------
# BASELINE config 5 (scaled down): fp8 e4m3 factors, bf16 activations
# ---------------------------------------------------------------------------

def _fp8_layer(shape, T, seed, gpu):
    x, f = inputs.make_layer(shape, T=T, seed=seed)
    xb = inputs.as_float32(x, torch.bfloat16)
    q = [fp8.quantize_per_channel(torch.from_numpy(a)) for a in f]
    deq = [O.e4m3_decode(qq.data.view(torch.uint8).numpy()) * qq.scale.numpy() for qq in q]
    qg = [ops.QuantizedFactor(qq.data.to(gpu), qq.scale.to(gpu)) for qq in q]
    return xb, deq, qg


# T=8: decode path; T=256: large-tile path with split-K; T=300: ragged M.
# The second shape has N edges that cut the 224/256-wide tiles and d not a
# multiple of the tile width (large-tile path, partial B tiles).
@pytest.mark.parametrize("T,shape", [
    (8, inputs.LayerShape(1024, 2048, 512)),
    (256, inputs.LayerShape(1024, 2048, 512)),
    (300, inputs.LayerShape(1024, 2048, 512)),
    (640, inputs.LayerShape(1056, 1120, 416, 288)),
])
def test_fp8_factors(gpu, T, shape):
    xb, deq, qg = _fp8_layer(shape, T, 9 + T, gpu)
    got = _np(ops.svd_mlp(_to(xb, torch.bfloat16, gpu), *qg))
    err = _rel(got, O.svd_mlp_ref(xb, *deq, dtype="bfloat16"))
    print(f"fp8 T={T} {shape} rel_l2={err:.3e}")
    assert err < FP8_TOL


# fp8 activations for h . Ud (SVDMLP_FP8_ACT): T=256 one row tile, T=300
# ragged rows, r_d = 288 a partial 128-column tile (the large-tile path takes
# ranks in multiples of 32), T=1024 / ff = 4096 more k-steps per split; T=1700
# / r_d = 5120 more 256 x 128 tiles than CUs (7 x 40): an unsplit launch of 252
# tiles (36 whole n-tile columns) and a 28-tile tail in 4 K splits; T=16
# (decode) runs as without the flag
@pytest.mark.parametrize("T,shape", [
    (256, inputs.LayerShape(1024, 2048, 512)),
    (300, inputs.LayerShape(1024, 2048, 512, 288)),
    (1024, inputs.LayerShape(2048, 4096, 640, 384)),
    (1700, inputs.LayerShape(5120, 4096, 512, 5120)),
    (16, inputs.LayerShape(1024, 2048, 512)),
])
def test_fp8_activations_down_stage(gpu, T, shape):
    xb, deq, qg = _fp8_layer(shape, T, 40 + T, gpu)
    xt = _to(xb, torch.bfloat16, gpu)
    got = _np(ops.svd_mlp(xt, *qg, fp8_activations=True))
    plain = O.svd_mlp_ref(xb, *deq, dtype="bfloat16")
    # the same quantisation applied to the GPU's own h: h's bf16-level
    # differences from the oracle's h would move ~10% of the e4m3 codes by a
    # step (~1.5e-2 relative), which is not what this compares
    h = _np(ops.fused_gate_up(xt, *qg[:4]))
    q, sc = O.quantize_rows_e4m3(h)
    hq = (O.e4m3_decode(q) * sc[:, None]).astype(np.float32)
    err_q = _rel(got, O.fused_xuv_ref(hq, *deq[4:], dtype="bfloat16"))
    err = _rel(got, plain)
    print(f"fp8 activations T={T} {shape}: vs the same quantisation {err_q:.3e}, vs bf16 activations {err:.3e}")
    assert err < FP8_TOL
    if T > 64:   # the large-tile path quantises h; replays are bitwise identical
        assert err_q < 1e-2 and err > 5e-3
        assert np.array_equal(got, _np(ops.svd_mlp(xt, *qg, fp8_activations=True)))
    else:        # decode shapes run as without the flag (fp32-atomic split-K sums there)
        assert _rel(got, _np(ops.svd_mlp(xt, *qg))) < 1e-3


def test_fp8_activations_need_fp8_factors(gpu):
    shape = inputs.LayerShape(1024, 2048, 512)
    x, f = inputs.make_layer(shape, T=256, seed=3)
    t = [_to(a, torch.bfloat16, gpu) for a in (x, *f)]
    with pytest.raises(Exception, match="SVDMLP_FP8_ACT needs fp8 factors"):
        ops.svd_mlp(*t, fp8_activations=True)


@pytest.mark.parametrize("T", [16, 512])
def test_fp8_gate_up_and_xuv_entries(gpu, T):
    """The two halves as separate entry points with fp8 factors."""
    shape = inputs.LayerShape(1024, 2048, 512)
    xb, deq, qg = _fp8_layer(shape, T, 70 + T, gpu)
    xt = _to(xb, torch.bfloat16, gpu)
    h = ops.fused_gate_up(xt, *qg[:4])
    ref_h = O.fused_gate_up_ref(xb, *deq[:4], dtype="bfloat16")
    assert _rel(_np(h), ref_h) < FP8_TOL
    hb = inputs.as_float32(_np(h), torch.bfloat16)
    y = ops.fused_xuv(_to(hb, torch.bfloat16, gpu), *qg[4:])
    assert _rel(_np(y), O.fused_xuv_ref(hb, *deq[4:], dtype="bfloat16")) < FP8_TOL


# ---------------------------------------------------------------------------
# BASELINE config 4 (scaled): RMSNorm + MLP + residual blocks, non-uniform ranks
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("T", [48, 300])
def test_mlp_block(gpu, T):
    """x + svd_mlp(RMSNorm(x) * gain) against the oracle's block
    (decode-layer path at T=48, large-tile path at T=300)."""
    shape = inputs.LayerShape(1024, 2048, 512, 384)
    x, f = inputs.make_layer(shape, T=T, seed=41 + T)
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    gain = np.random.default_rng(T).uniform(0.9, 1.1, size=shape.d).astype(np.float32)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    y = _np(ops.svd_mlp_block(t[0], torch.from_numpy(gain).to(gpu), *t[1:], eps=1e-5))
    ref = O.mlp_block_ref(xb, gain, fb, eps=1e-5, dtype="bfloat16")
    # the residual dominates y: compare the MLP part as well
    assert _rel(y, ref) < BF16_TOL
    assert _rel(y - xb, ref - xb) < BF16_TOL


@pytest.mark.parametrize("dtype,d", [(torch.float32, 256), (torch.bfloat16, 260), (torch.float32, 258)])
def test_mlp_block_fp32_and_odd_widths(gpu, dtype, d):
    """The block's RMSNorm and residual kernels in fp32 and on widths that
    are no multiple of the 16-byte piece (their element-wise form)."""
    shape = inputs.LayerShape(d, 392, 72)
    x, f = inputs.make_layer(shape, T=37, seed=d)
    gain = np.random.default_rng(d).uniform(0.9, 1.1, size=d).astype(np.float32)
    name = "bfloat16" if dtype == torch.bfloat16 else "float32"
    xr, *fr = _rounded((x, *f), dtype) if dtype == torch.bfloat16 else (x, *f)
    t = [_to(a, dtype, gpu) for a in (xr, *fr)]
    y = _np(ops.svd_mlp_block(t[0], torch.from_numpy(gain).to(gpu), *t[1:], eps=1e-5))
    ref = O.mlp_block_ref(xr, gain, fr, eps=1e-5, dtype=name)
    tol = BF16_TOL if dtype == torch.bfloat16 else 1e-4
    assert _rel(y, ref) < tol and _rel(y - xr, ref - xr) < tol


def test_mlp_stack_nonuniform_ranks(gpu):
    """Three blocks with independently drawn gate/up/down ranks against the
    oracle, layer after layer (T=96: decode shapes, where the host mirror
    zero-pads the smaller of the gate and up branches)."""
    from svdmlp import stack

    d, ff, T = 1024, 2048, 96
    layers = stack.make_stack(3, d, ff, seed=5, device=gpu, choices=(256, 384, 512))
    assert len({l.ranks for l in layers}) > 1
    x = torch.from_numpy(_x(T, d, 17)).to(gpu).to(torch.bfloat16)
    y = _np(stack.run_stack(x, layers, eps=1e-5))
    ref = x.float().cpu().numpy()
    for l in layers:
        f = [a.float().cpu().numpy() for a in l.factors]
        ref = O.mlp_block_ref(ref, l.gain.cpu().numpy(), f, eps=1e-5, dtype="bfloat16")
    x0 = x.float().cpu().numpy()
    assert _rel(y, ref) < BF16_TOL
    assert _rel(y - x0, ref - x0) < BF16_TOL


def _block_case(shape, T, seed):
    x, f = inputs.make_layer(shape, T=T, seed=seed)
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    gain = np.random.default_rng(seed).uniform(0.9, 1.1, size=shape.d).astype(np.float32)
    return xb, fb, gain


@pytest.mark.parametrize("T,padded", [(1, True), (1, False), (2, True), (3, False), (8, True), (32, True),
                                      (64, True), (100, False)])
def test_mlp_block_fused_into_decode_layer(gpu, layer8b, T, padded):
    """The 8B block at decode shapes: one decode-layer launch, whose phase 0
    writes RMSNorm(x) (a block per token row) and whose phase 4 adds the
    residual; against the oracle's block, bitwise on replay."""
    shape, fb, ft = layer8b
    xb = _x(T, shape.d, 900 + T)
    gain = np.random.default_rng(T).uniform(0.9, 1.1, size=shape.d).astype(np.float32)
    g = torch.from_numpy(gain).to(gpu)
    xt = _to(xb, torch.bfloat16, gpu)
    fs = [ops.pad_rows(a, 64) if padded and i % 2 else a for i, a in enumerate(ft)]
    ws = ops.svd_mlp_workspace(xt, r=shape.r, ff=shape.ff)
    runs = [_np(ops.svd_mlp_block(xt, g, *fs, eps=1e-5, workspace=ws)) for _ in range(2)]
    ref = O.mlp_block_ref(xb, gain, fb, eps=1e-5, dtype="bfloat16")
    assert _rel(runs[0], ref) < BF16_TOL
    assert _rel(runs[0] - xb, ref - xb) < BF16_TOL, _rel(runs[0] - xb, ref - xb)
    assert np.array_equal(runs[0], runs[1])
    # two launches of _dl_barriers each (phase 0's rows signal phase 1 by ready flags); counters back at zero
    per = _dl_barriers(T, _contracted(shape, T, padded=padded))
    assert _barrier_state(ws) == (2 * per, 0) and not any(_tile_counters(ws))


@pytest.mark.parametrize("T", [1, 8])
def test_mlp_block_decode_unaligned_gain(gpu, T):
    """Gains that are not 16-byte aligned (a view 4 bytes into a buffer): the
    decode layer runs the RMSNorm as its own pass, then adds the residual in
    its last phase; the result matches the fused phase 0's to the bf16
    level and the oracle's block."""
    shape = inputs.LayerShape(1024, 2048, 512, 384)
    xb, fb, gain = _block_case(shape, T, 970 + T)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    g = torch.from_numpy(gain).to(gpu)
    buf = torch.empty(shape.d + 4, dtype=torch.float32, device=gpu)
    buf[1:shape.d + 1] = g
    g_off = buf[1:shape.d + 1]
    assert g_off.data_ptr() % 16 != 0
    y_off = _np(ops.svd_mlp_block(t[0], g_off, *t[1:], eps=1e-5))
    y = _np(ops.svd_mlp_block(t[0], g, *t[1:], eps=1e-5))
    ref = O.mlp_block_ref(xb, gain, fb, eps=1e-5, dtype="bfloat16")
    assert _rel(y_off, ref) < BF16_TOL and _rel(y_off - xb, ref - xb) < BF16_TOL
    assert _rel(y_off - xb, y - xb) < 5e-3


@pytest.mark.parametrize("shape", [inputs.LayerShape(128, 256, 384, 128), inputs.LayerShape(5248, 1024, 512, 256)])
@pytest.mark.parametrize("T", [1, 7, 16])
def test_mlp_block_fused_norm_row_widths(gpu, shape, T):
    """Phase 0's row pieces (8 elements per thread per 4096): a row shorter
    than one piece round (d = 128) and one of two rounds, the second partial
    (d = 5248)."""
    xb, fb, gain = _block_case(shape, T, 950 + T)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    y = _np(ops.svd_mlp_block(t[0], torch.from_numpy(gain).to(gpu), *t[1:], eps=1e-5))
    ref = O.mlp_block_ref(xb, gain, fb, eps=1e-5, dtype="bfloat16")
    assert _rel(y, ref) < BF16_TOL and _rel(y - xb, ref - xb) < BF16_TOL


@pytest.mark.parametrize("T", [1, 2])
def test_mlp_block_gemv_layer_residual(gpu, T):
    """The streaming-GEMV layer (d = 1040: no multiple of 128) takes the
    block's residual add in its output write after the RMSNorm pass."""
    shape = inputs.LayerShape(1040, 2064, 400, 272)
    xb, fb, gain = _block_case(shape, T, 960 + T)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    ws = ops.svd_mlp_workspace(t[0], r=shape.r, ff=shape.ff)
    y = _np(ops.svd_mlp_block(t[0], torch.from_numpy(gain).to(gpu), *t[1:], eps=1e-5, workspace=ws))
    ref = O.mlp_block_ref(xb, gain, fb, eps=1e-5, dtype="bfloat16")
    assert _rel(y, ref) < BF16_TOL and _rel(y - xb, ref - xb) < BF16_TOL
    assert _barrier_state(ws) == (4, 0)   # one GEMV-layer launch


# ---------------------------------------------------------------------------
# distinct gate and up ranks (svdmlp_svd_mlp_ranks)
# ---------------------------------------------------------------------------

def _two_rank_layer(d, ff, r_g, r_u, r_d, T, seed):
    """bf16-valued x and factors with a gate rank and an up rank of their own."""
    rng = np.random.default_rng(seed)
    f = [inputs.random_matrix(rng, a, b) for a, b in ((d, r_g), (r_g, ff), (d, r_u), (r_u, ff), (ff, r_d), (r_d, d))]
    return _rounded((inputs.make_x(rng, T, d), *f), torch.bfloat16)


# T=8 and 96: decode shapes, the persistent decode layer with each branch at
# its rank (phase-1 tiles of both branches, one-branch phase-2 units over
# their own K); T=200: split gate/up XU.V passes (one row tile, K split in two per
# branch); T=300: fragment-order g pass + SwiGLU pass at each branch's rank;
# T=1024: split-K X.U with both branches' column tiles in one launch; ranks
# that are no multiple of the 256-wide tile leave ragged last tiles per branch.
@pytest.mark.parametrize("T,ranks", [(8, (512, 256, 384)), (96, (384, 640, 256)), (200, (512, 256, 384)),
                                     (300, (256, 512, 384)), (1024, (384, 640, 512))])
def test_distinct_gate_up_ranks(gpu, T, ranks):
    r_g, r_u, r_d = ranks
    d, ff = 1024, 2048
    xb, *fb = _two_rank_layer(d, ff, r_g, r_u, r_d, T, 900 + T)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    ref = O.svd_mlp_ref(xb, *fb, dtype="bfloat16")
    got = _np(ops.svd_mlp(*t))
    err = _rel(got, ref)
    print(f"two ranks T={T} r_g={r_g} r_u={r_u} r_d={r_d} rel_l2={err:.3e}")
    assert err < BF16_TOL
    # the same layer with the smaller branch zero-padded to one rank
    padded = _np(ops.svd_mlp(t[0], *ops._pad_branches(*t[1:5]), *t[5:]))
    assert _rel(got, padded) < 5e-3


# More gate/up X.U tiles than one round of blocks (12 row tiles of 256 at
# 3000 tokens, 22-23 column tiles of 256 over both branches): one launch of
# whole column tiles without a K split, then the remaining tiles in K splits
# whose compact fp32 slices are summed per branch; equal ranks take the same
# two-entry form.  (5632, 256): the split tail holds the last gate column tile
# and the up branch's.  Ragged last row tile.
@pytest.mark.parametrize("ranks", [(2816, 2816, 512), (2816, 3072, 512), (3072, 2560, 384), (5632, 256, 384)])
def test_gate_up_split_tail(gpu, ranks):
    from svdmlp import _lib

    r_g, r_u, r_d = ranks
    T, d, ff = 3000, 1024, 2048
    xb, *fb = _two_rank_layer(d, ff, r_g, r_u, r_d, T, 1300 + r_g + r_u)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    ref = O.svd_mlp_ref(xb, *fb, dtype="bfloat16")
    with _lib.StageProfile() as prof:
        got = _np(ops.svd_mlp(*t))
    err = _rel(got, ref)
    print(f"split tail T={T} ranks={ranks} rel_l2={err:.3e} launches={ {k: v[1] for k, v in prof.result.items()} }")
    assert err < BF16_TOL
    assert prof.result["gate_up_xu"][1] == 2   # the unsplit head and the split tail
    assert np.array_equal(got, _np(ops.svd_mlp(*t)))  # replays are bitwise identical


# The gate/up XU.V passes run as one launch: above 512 tokens every block its
# g tile, then its u tile, reading its own gate values back; at one or two
# row tiles (the passes split K) every block its g split, then its u split,
# both storing fp32 slices for the one reduction.  The bits of the
# two-launch form, which SVDMLP_TUNE=gudual=0 (read once per process) keeps,
# computed in a child process on the same seeded inputs: 256 x 224 tiles (ff
# a multiple of 224), 256 x 256 with distinct gate and up ranks, 256 x 128 in
# four K splits (T=200), 256 x 256 in two (T=500), 256 x 128 unsplit (T=384),
# a ragged last column tile (ff=1088) and fp8 factors.
_DUAL_CHILD = """
import sys, numpy as np, torch
sys.path[:0] = sys.argv[1].split("|")
from svdmlp import fp8, inputs, ops
d, ff, rg, ru, rd, T, seed, q = (int(a) for a in sys.argv[2:10])
rng = np.random.default_rng(seed)
f = [inputs.random_matrix(rng, a, b) for a, b in ((d, rg), (rg, ff), (d, ru), (ru, ff), (ff, rd), (rd, d))]
t = [inputs.to_torch(a, torch.bfloat16, torch.device("cuda:0")) for a in (inputs.make_x(rng, T, d), *f)]
if q:
    t = t[:1] + [fp8.quantize_per_channel(a) for a in t[1:]]
np.save(sys.argv[10], ops.svd_mlp(*t).view(torch.int16).cpu().numpy())
"""


@pytest.mark.parametrize("T,d,ff,ranks,q", [(600, 1024, 3584, (512, 512, 384), 0), (700, 1024, 4096, (384, 640, 256), 0),
                                            (1000, 2048, 4096, (768, 768, 512), 0), (200, 1024, 4096, (512, 384, 256), 0),
                                            (500, 1024, 4096, (512, 512, 384), 0), (384, 1024, 4096, (384, 512, 256), 0),
                                            (600, 1024, 1088, (256, 320, 192), 0), (700, 1024, 3584, (512, 384, 256), 1)])
def test_gate_up_dual_launch_bitwise(gpu, tmp_path, T, d, ff, ranks, q):
    import os
    import subprocess
    import sys

    r_g, r_u, r_d = ranks
    seed = 1700 + T
    rng = np.random.default_rng(seed)
    f = [inputs.random_matrix(rng, a, b) for a, b in ((d, r_g), (r_g, ff), (d, r_u), (r_u, ff), (ff, r_d), (r_d, d))]
    t = [inputs.to_torch(a, torch.bfloat16, gpu) for a in (inputs.make_x(rng, T, d), *f)]
    if q:  # fp8 e4m3 factors with per-column scales (the 70B configuration's format)
        t = t[:1] + [fp8.quantize_per_channel(a) for a in t[1:]]
    paths = "|".join(p for p in sys.path if p)

    def child(tune, name):
        out = tmp_path / name
        subprocess.run([sys.executable, "-c", _DUAL_CHILD, paths, *map(str, (d, ff, r_g, r_u, r_d, T, seed, q)),
                        str(out)], env=dict(os.environ, SVDMLP_TUNE=tune), check=True, timeout=120)
        return np.load(out)

    # (at 129-512 tokens, while the 128-row K-group tiles fit one round of the
    # CUs, the default runs them, whose sums are ordered differently: there the
    # one- and two-launch forms on 256-row tiles)
    kg = 128 < T <= 512 and not q and -(-T // 128) * -(-ff // 128) <= 256
    got = child("gukgu=0", "one_launch.npy") if kg else ops.svd_mlp(*t).view(torch.int16).cpu().numpy()
    assert np.array_equal(got, child("gudual=0,gukgu=0" if kg else "gudual=0", "two_launch.npy")), (T, d, ff, ranks)


_GU_CHILD = """
import sys, numpy as np, torch
sys.path[:0] = sys.argv[1].split("|")
from svdmlp import inputs, ops
d, ff, r, T, seed = (int(a) for a in sys.argv[2:7])
rng = np.random.default_rng(seed)
f = [inputs.random_matrix(rng, a, b) for a, b in ((d, r), (r, ff), (d, r), (r, ff))]
t = [inputs.to_torch(a, torch.bfloat16, torch.device("cuda:0")) for a in (inputs.make_x(rng, T, d), *f)]
np.save(sys.argv[7], ops.fused_gate_up(*t).view(torch.int16).cpu().numpy())
"""


@pytest.mark.parametrize("T,d,ff,r", [(72, 1024, 4096, 512), (100, 1024, 4096, 512), (128, 4096, 14336, 2816),
                                      (160, 1024, 4096, 512), (200, 4096, 14336, 2816), (256, 1024, 4096, 384),
                                      (384, 1024, 8192, 512), (512, 3072, 8192, 1792)])
def test_gate_up_kgroup_tiles(gpu, tmp_path, T, d, ff, r):
    """fused_gate_up at 65-512 tokens on the large-tile path: the one-launch
    passes on 128 x 128 K-group tiles (each 64-k stage summed in two 32-k
    halves), split at up to 128 tokens and unsplit (the SwiGLU epilogue) at
    129-512 while the tiles fit one round of the CUs: against the oracle, bitwise on replay, and within the tolerance
    of the 256-row tiles (SVDMLP_TUNE=gukg=0,gukgu=0, another process), whose
    differently ordered sums show the K-group instance ran."""
    import os
    import subprocess
    import sys

    seed = 1900 + T
    rng = np.random.default_rng(seed)
    f = [inputs.random_matrix(rng, a, b) for a, b in ((d, r), (r, ff), (d, r), (r, ff))]
    x = inputs.make_x(rng, T, d)
    t = [inputs.to_torch(a, torch.bfloat16, gpu) for a in (x, *f)]
    h = ops.fused_gate_up(*t)
    again = ops.fused_gate_up(*t)
    assert torch.equal(h.view(torch.int16), again.view(torch.int16))
    xb, *fb = (inputs.as_float32(a, torch.bfloat16) for a in (x, *f))
    rows = slice(0, min(T, 32))
    assert _rel(_np(h)[rows], O.fused_gate_up_ref(xb[rows], *fb, "bfloat16")) < BF16_TOL
    out = tmp_path / "kg1.npy"
    env = dict(os.environ, SVDMLP_TUNE="gukg=0,gukgu=0")
    paths = "|".join(p for p in sys.path if p)
    subprocess.run([sys.executable, "-c", _GU_CHILD, paths, *map(str, (d, ff, r, T, seed)), str(out)],
                   env=env, check=True, timeout=120)
    h1 = torch.from_numpy(np.load(out)).view(torch.bfloat16).float().numpy()
    assert _rel(_np(h), h1) < 5e-3
    assert not np.array_equal(_np(h), h1)


def test_distinct_gate_up_ranks_fp8(gpu):
    T, d, ff, r_g, r_u, r_d = 300, 1024, 2048, 512, 256, 384
    xb, *fb = _two_rank_layer(d, ff, r_g, r_u, r_d, T, 950)
    q = [fp8.quantize_per_channel(torch.from_numpy(a)) for a in fb]
    deq = [O.e4m3_decode(qq.data.view(torch.uint8).numpy()) * qq.scale.numpy() for qq in q]
    qg = [ops.QuantizedFactor(qq.data.to(gpu), qq.scale.to(gpu)) for qq in q]
    xt = _to(xb, torch.bfloat16, gpu)
    got = _np(ops.svd_mlp(xt, *qg))
    assert _rel(got, O.svd_mlp_ref(xb, *deq, dtype="bfloat16")) < FP8_TOL
    # fp8 activations for h . Ud on the two-rank large-tile path: h is
    # quantised (further from the bf16-activation math than the plain layer)
    # and the layer stays within the fp8 budget (fused_gate_up takes one rank,
    # so the GPU's own h is not at hand to quantise as the other tests do)
    got8 = _np(ops.svd_mlp(xt, *qg, fp8_activations=True))
    err8 = _rel(got8, O.svd_mlp_ref(xb, *deq, dtype="bfloat16"))
    assert 1e-2 < err8 < FP8_TOL, err8
    # fp8 at a decode shape: zero-padded fp8 branches (zero data, unit scales)
    xs = xb[:8]
    got = _np(ops.svd_mlp(_to(xs, torch.bfloat16, gpu), *qg))
    assert _rel(got, O.svd_mlp_ref(xs, *deq, dtype="bfloat16")) < FP8_TOL


def test_distinct_gate_up_ranks_block_and_row_pitches(gpu):
    """The block with two ranks, and gate / up factors with padded rows of
    different pitches (each branch read with its own on the large-tile path)."""
    T, d, ff, r_g, r_u, r_d = 300, 1024, 2048, 384, 256, 512
    xb, *fb = _two_rank_layer(d, ff, r_g, r_u, r_d, T, 960)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    gain = np.random.default_rng(4).uniform(0.9, 1.1, size=d).astype(np.float32)
    g = torch.from_numpy(gain).to(gpu)
    ref = O.mlp_block_ref(xb, gain, fb, eps=1e-5, dtype="bfloat16")
    y = _np(ops.svd_mlp_block(t[0], g, *t[1:], eps=1e-5))
    assert _rel(y, ref) < BF16_TOL and _rel(y - xb, ref - xb) < BF16_TOL
    padded = [ops.pad_rows(a, p) for a, p in zip(t[1:], (8, 64, 72, 128, 24, 40))]
    assert all(ops.padded_rows(a) for a in padded)
    y = _np(ops.svd_mlp_block(t[0], g, *padded, eps=1e-5))
    assert _rel(y, ref) < BF16_TOL and _rel(y - xb, ref - xb) < BF16_TOL


def test_distinct_gate_up_ranks_abi(gpu):
    """svdmlp_svd_mlp_ranks runs two ranks on the decode layer and the
    large-tile path and returns SVDMLP_EUNSUP, with a message, where only one
    rank is taken (decode shapes with an up rank the decode layer's 128-column
    tiles do not divide)."""
    import ctypes

    from svdmlp import _lib

    lib = _lib.load()
    d, ff, r_d = 1024, 2048, 384
    ws = None
    for T, (r_g, r_u), want in ((8, (512, 320), _lib.SVDMLP_EUNSUP), (8, (512, 256), _lib.SVDMLP_OK),
                                (300, (512, 256), _lib.SVDMLP_OK)):
        xb, *fb = _two_rank_layer(d, ff, r_g, r_u, r_d, T, 970)
        t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
        y = torch.zeros((T, d), dtype=torch.bfloat16, device=gpu)
        ws = ops.svd_mlp_workspace(t[0], r=max(r_g, r_u, r_d), ff=ff)
        bf = _lib.SVDMLP_BF16
        rc = lib.svdmlp_svd_mlp_ranks(t[0].data_ptr(), *(a.data_ptr() for a in t[1:]), None, None, y.data_ptr(),
                                      T, d, ff, r_g, r_u, r_d, bf, bf, 0, ws.data_ptr(), ws.numel(),
                                      torch.cuda.current_stream(gpu).cuda_stream)
        assert rc == want
        if want == _lib.SVDMLP_EUNSUP:
            assert "persistent decode layer" in lib.svdmlp_last_error().decode()
        else:
            assert _rel(_np(y), O.svd_mlp_ref(xb, *fb, dtype="bfloat16")) < BF16_TOL
        if T <= 128 and want == _lib.SVDMLP_OK:
            # one decode-layer launch
            assert _barrier_state(ws) == (_dl_barriers(T, False), 0) and not any(_tile_counters(ws))


@pytest.mark.parametrize("T", [1, 8, 64])
def test_distinct_gate_up_ranks_decode_8b(gpu, T):
    """LLaMA3-8B decode with a gate rank, an up rank and a down rank drawn
    from BASELINE config 4's menu {2048, ..., 3072}: the layer and the MLP
    block each run as one decode-layer launch with every branch at its own
    rank (no zero padding, no allocation with a workspace and out), match
    the oracle and replay bitwise."""
    d, ff, r_g, r_u, r_d = 4096, 14336, 2304, 3072, 2560
    xb, *fb = _two_rank_layer(d, ff, r_g, r_u, r_d, T, 980 + T)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    gain = np.random.default_rng(5).uniform(0.9, 1.1, size=d).astype(np.float32)
    g = torch.from_numpy(gain).to(gpu)
    ws = ops.svd_mlp_workspace(t[0], r=max(r_g, r_u, r_d), ff=ff)
    out = torch.empty((T, d), dtype=torch.bfloat16, device=gpu)
    y0 = ops.svd_mlp(*t, workspace=ws, out=out).clone()
    torch.cuda.synchronize(gpu)
    before = torch.cuda.memory_allocated(gpu)
    ops.svd_mlp(*t, workspace=ws, out=out)
    torch.cuda.synchronize(gpu)
    assert torch.cuda.memory_allocated(gpu) == before   # no padded copies, no allocation
    ys = [y0, out.clone(), ops.svd_mlp(*t, workspace=ws, out=out).clone()]
    assert torch.equal(ys[0].view(torch.int16), ys[1].view(torch.int16))
    assert torch.equal(ys[0].view(torch.int16), ys[2].view(torch.int16))
    assert _barrier_state(ws) == (3 * _dl_barriers(T, False), 0) and not any(_tile_counters(ws))   # three launches
    err = _rel(_np(ys[0]), O.svd_mlp_ref(xb, *fb, dtype="bfloat16"))
    print(f"two ranks 8B decode T={T} rel_l2={err:.3e}")
    assert err < BF16_TOL
    yb = _np(ops.svd_mlp_block(t[0], g, *t[1:], eps=1e-5, workspace=ws, out=out))
    ref = O.mlp_block_ref(xb, gain, fb, eps=1e-5, dtype="bfloat16")
    assert _rel(yb, ref) < BF16_TOL and _rel(yb - xb, ref - xb) < BF16_TOL
    # + one launch of the block (its RMSNorm phase 0 signals phase 1 by ready flags)
    assert _barrier_state(ws) == (4 * _dl_barriers(T, False), 0)


# ---------------------------------------------------------------------------
# safetensors SVD checkpoint (models/hf_svd.py) -> the HIP layer
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("layout,T", [("natural", 1), ("padded", 1), ("natural", 300), ("padded", 300), ("linear", 64)])
def test_checkpoint_layers_run_on_the_hip_path(gpu, tmp_path, layout, T):
    """Factors written as a two-shard checkpoint (stored as Linear weights with
    the v/u names swapped), loaded back onto the GPU, give the oracle's layer."""
    from svdmlp import checkpoint

    shape = inputs.LayerShape(1024, 2048, 512)
    layers = []
    for seed in (3, 4):
        _, f = inputs.make_layer(shape, T=1, seed=seed)
        layers.append([torch.from_numpy(inputs.as_float32(a, torch.bfloat16)).to(torch.bfloat16) for a in f])
    checkpoint.save_mlp_checkpoint(tmp_path, layers, hidden_size=shape.d, intermediate_size=shape.ff)
    loaded = checkpoint.load_mlp_factors(tmp_path, [1, 0], device=gpu, layout=layout)
    x = _x(T, shape.d, 500 + T)
    xt = _to(x, torch.bfloat16, gpu)
    for got, want in zip(loaded, (layers[1], layers[0])):
        y = _np(ops.svd_mlp(xt, *got))
        err = _rel(y, O.svd_mlp_ref(x, *[w.float().numpy() for w in want], dtype="bfloat16"))
        assert err < BF16_TOL, (layout, T, err)


def test_checkpoint_runner_per_layer_report(gpu, tmp_path):
    """python -m svdmlp.checkpoint_speedup on a synthetic checkpoint: every
    (layer, T) verified against the fp32 arm, timed, summarised."""
    from svdmlp import checkpoint, checkpoint_speedup

    shape = inputs.LayerShape(1024, 2048, 512)
    layers = []
    for seed in (5, 6):
        _, f = inputs.make_layer(shape, T=1, seed=seed)
        layers.append([torch.from_numpy(a).to(torch.bfloat16) for a in f])
    ckpt = tmp_path / "ckpt"
    checkpoint.save_mlp_checkpoint(ckpt, layers, hidden_size=shape.d, intermediate_size=shape.ff)
    out = tmp_path / "report.json"
    report = checkpoint_speedup.run(checkpoint_speedup._parser().parse_args(
        ["--model-path", str(ckpt), "--seq-lens", "1", "128", "--warmup", "1", "--repeats", "3",
         "--output", str(out)]))
    assert report["complete"] and len(report["records"]) == 4
    for rec in report["records"]:
        assert rec["passed"] and rec["fused_vs_fp32"]["relative_l2"] < BF16_TOL
        assert rec["fused_ms"] > 0 and rec["unfused_low_rank_ms"] > 0
    assert all(s["complete"] and s["passed"] for s in report["summaries"])
    assert out.with_suffix(".csv").exists()


# ---------------------------------------------------------------------------
# factors with padded rows (svdmlp_svd_mlp_ld)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("T", [1, 2, 8, 64, 128, 300])
def test_padded_factor_rows(gpu, T):
    """Row-padded natural-layout views (column slices of wider buffers) are
    read in place by the MFMA decode layer (T <= 128; it takes T <= 2 too when
    rows are padded) and the large-tile path, with each factor's own pitch."""
    shape = inputs.LayerShape(1024, 2048, 512, 384)
    x, f = inputs.make_layer(shape, T=T, seed=700 + T)
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    pads = (8, 64, 8, 64, 24, 128)  # ug, vg, uu, vu, ud, vd
    padded = [ops.pad_rows(a, p) for a, p in zip(t[1:], pads)]
    assert all(ops.padded_rows(a) for a in padded)
    ref = O.svd_mlp_ref(xb, *fb, dtype="bfloat16")
    ws = ops.svd_mlp_workspace(t[0], r=max(shape.r, shape.rd), ff=shape.ff)
    err = _rel(_np(ops.svd_mlp(t[0], *padded, workspace=ws)), ref)
    assert err < BF16_TOL, err
    if T <= 128:   # one MFMA decode-layer launch (_dl_barriers), counters back at zero
        assert (_barrier_state(ws) == (_dl_barriers(T, _contracted(shape, T, padded=True)), 0)
                and not any(_tile_counters(ws)))
    dense = _np(ops.svd_mlp(*t))
    # the same math; split-K partials are summed in other orders on the
    # paths the two layouts take, so roundings may differ
    assert _rel(_np(ops.svd_mlp(t[0], *padded)), dense) < 5e-3


@pytest.mark.parametrize("T", [1, 2])
def test_padded_factor_rows_gemv_layer(gpu, T):
    """Padded rows on a shape only the streaming-GEMV layer takes at decode
    (d = 1040 is no multiple of 128): ragged strips read with each factor's
    pitch."""
    shape = inputs.LayerShape(1040, 2064, 400, 272)
    x, f = inputs.make_layer(shape, T=T, seed=720 + T)
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    padded = [ops.pad_rows(a, p) for a, p in zip(t[1:], (8, 64, 8, 64, 24, 128))]
    ws = ops.svd_mlp_workspace(t[0], r=shape.r, ff=shape.ff)
    got = _np(ops.svd_mlp(t[0], *padded, workspace=ws))
    assert _rel(got, O.svd_mlp_ref(xb, *fb, dtype="bfloat16")) < BF16_TOL
    assert _barrier_state(ws) == (4, 0)   # one GEMV-layer launch: 4 barriers


def test_padded_factor_rows_block_and_mixed_pitch(gpu):
    shape = inputs.LayerShape(1024, 2048, 512)
    x, f = inputs.make_layer(shape, T=48, seed=77)
    xb, *fb = _rounded((x, *f), torch.bfloat16)
    t = [_to(a, torch.bfloat16, gpu) for a in (xb, *fb)]
    gain = np.random.default_rng(3).uniform(0.9, 1.1, size=shape.d).astype(np.float32)
    g = torch.from_numpy(gain).to(gpu)
    padded = [ops.pad_rows(a, 64) for a in t[1:]]
    got = _np(ops.svd_mlp_block(t[0], g, *padded))
    assert _rel(got, O.mlp_block_ref(xb, gain, fb, eps=1e-5, dtype="bfloat16")) < BF16_TOL
    # gate and up with different pitches: the host mirror reads them densely
    mixed = list(padded)
    mixed[2] = ops.pad_rows(t[3], 32)
    assert _rel(_np(ops.svd_mlp(t[0], *mixed)), O.svd_mlp_ref(xb, *fb, dtype="bfloat16")) < BF16_TOL


def test_padded_factor_rows_invalid(gpu):
    """The C ABI rejects pitches below the row length, unaligned pitches,
    different gate / up pitches and padded rows with fp32 factors."""
    import ctypes

    from svdmlp import _lib

    lib = _lib.load()
    T, d, ff, r = 8, 1024, 2048, 512
    dev = gpu
    x = torch.zeros((T, d), dtype=torch.bfloat16, device=dev)
    fs = [torch.zeros(s, dtype=torch.bfloat16, device=dev)
          for s in ((d, r + 64), (r, ff + 64), (d, r + 64), (r, ff + 64), (ff, r), (r, d))]
    y = torch.empty((T, d), dtype=torch.bfloat16, device=dev)
    ws = ops.svd_mlp_workspace(x, r=r, ff=ff)

    def call(ld, act=_lib.SVDMLP_BF16):
        arr = (ctypes.c_int64 * 6)(*ld)
        return lib.svdmlp_svd_mlp_ld(x.data_ptr(), *(f.data_ptr() for f in fs), None, ctypes.addressof(arr),
                                     y.data_ptr(), T, d, ff, r, r, act, act, 0, ws.data_ptr(), ws.numel(),
                                     torch.cuda.current_stream(dev).cuda_stream)

    for ld, msg in (((r - 8, 0, 0, 0, 0, 0), "below its row length"),
                    ((r + 4, ff + 64, r + 4, ff + 64, 0, 0), "multiples of 8"),
                    ((r + 64, ff + 64, r + 64, ff + 32, 0, 0), "share their leading dimensions")):
        assert call(ld) == _lib.SVDMLP_EINVAL
        assert msg in lib.svdmlp_last_error().decode()
    assert call((r + 64, ff + 64, r + 64, ff + 64, 0, 0), act=_lib.SVDMLP_F32) == _lib.SVDMLP_EINVAL
    assert "bf16 natural-layout" in lib.svdmlp_last_error().decode()
    assert call((r + 64, ff + 64, r + 64, ff + 64, 0, 0)) == 0
    torch.cuda.synchronize()
