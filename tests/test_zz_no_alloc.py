"""svdmlp_svd_mlp_noalloc: the layer without a caller workspace, in the
library's fixed per-device scratch (no allocation on the call).  Checked
through the C ABI against svdmlp_svd_mlp_ld with a caller workspace on the
same inputs, on consecutive calls (the second smaller), on the decode and
the prefill kernels, and for the size limit."""

import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from svdmlp import _lib, inputs, ops

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20


def _ptrs(ts):
    return [t.data_ptr() for t in ts]


def _ld(factors):
    """Row pitches (elements) of the six factors, as svdmlp_svd_mlp_ld takes them."""
    return (ctypes.c_int64 * 6)(*[f.stride(0) for f in factors])


def _call_both(lib, x, fs, dims, dev):
    T, d, ff, r_gu, r_d = dims
    stream = torch.cuda.current_stream(dev).cuda_stream
    y_ws = torch.full((T, d), 7.0, dtype=torch.bfloat16, device=dev)
    y_na = torch.full((T, d), -7.0, dtype=torch.bfloat16, device=dev)
    ws = ops.svd_mlp_workspace(x, r=max(r_gu, r_d), ff=ff)
    bf = _lib.SVDMLP_BF16
    ld = _ld(fs)   # kept alive across both calls
    rc = lib.svdmlp_svd_mlp_ld(x.data_ptr(), *_ptrs(fs), None, ctypes.addressof(ld), y_ws.data_ptr(),
                               T, d, ff, r_gu, r_d, bf, bf, 0, ws.data_ptr(), ws.numel(), stream)
    assert rc == 0, lib.svdmlp_last_error()
    rc = lib.svdmlp_svd_mlp_noalloc(x.data_ptr(), *_ptrs(fs), None, ctypes.addressof(ld), y_na.data_ptr(),
                                    T, d, ff, r_gu, r_d, bf, bf, 0, stream)
    assert rc == 0, lib.svdmlp_last_error()
    torch.cuda.synchronize(dev)
    return y_ws, y_na


@pytest.mark.parametrize("shape,Ts,pad", [
    (inputs.LayerShape(4096, 14336, 2816), (64, 8, 2, 1), 64),  # LLaMA3-8B decode: MFMA decode layer (contracted at 1, 2)
    (inputs.LayerShape(1024, 2048, 512, 384), (300, 160), 0),   # large-tile prefill path (fits the scratch)
    (inputs.LayerShape(1040, 2064, 400, 272), (2, 1), 0),       # streaming-GEMV layer (1-2 tokens, d % 128 != 0)
])
def test_noalloc_matches_workspace_entry_point(gpu, shape, Ts, pad):
    lib = _lib.load()
    x, f = inputs.make_layer(shape, T=max(Ts), seed=61)
    xb, *fb = [inputs.as_float32(a, torch.bfloat16) for a in (x, *f)]
    xt = inputs.to_torch(xb, torch.bfloat16, gpu)
    fs = [inputs.to_torch(a, torch.bfloat16, gpu) for a in fb]
    if pad:
        fs = [ops.pad_rows(a, pad) if i % 2 else a for i, a in enumerate(fs)]
    for T in Ts:   # consecutive calls share the scratch; each smaller than the last
        xs = xt[:T].contiguous()
        dims = (T, shape.d, shape.ff, shape.r, shape.rd)
        need = lib.svdmlp_workspace_bytes(T, shape.d, shape.ff, max(shape.r, shape.rd), _lib.SVDMLP_BF16)
        assert need <= SCRATCH_BYTES
        y_ws, y_na = _call_both(lib, xs, fs, dims, gpu)
        assert torch.isfinite(y_na.float()).all()
        if T > 2 or pad:   # deterministic kernels: the same bits
            assert torch.equal(y_na.view(torch.int16), y_ws.view(torch.int16)), T
        rows = slice(0, min(T, 16))
        err = O.relative_l2(y_na[rows].float().cpu().numpy(), O.svd_mlp_ref(xb[rows], *fb, dtype="bfloat16"))
        assert err < 1e-2, (T, err)
        assert O.relative_l2(y_na.float().cpu().numpy(), y_ws.float().cpu().numpy()) < 5e-3


def test_noalloc_rejects_shapes_beyond_the_scratch(gpu):
    lib = _lib.load()
    T, d, ff, r = 1024, 4096, 14336, 2816
    assert lib.svdmlp_workspace_bytes(T, d, ff, r, _lib.SVDMLP_BF16) > SCRATCH_BYTES
    x = torch.zeros((T, d), dtype=torch.bfloat16, device=gpu)
    fs = [torch.zeros(s, dtype=torch.bfloat16, device=gpu) for s in ((d, r), (r, ff), (d, r), (r, ff), (ff, r), (r, d))]
    y = torch.empty_like(x)
    rc = lib.svdmlp_svd_mlp_noalloc(x.data_ptr(), *_ptrs(fs), None, None, y.data_ptr(), T, d, ff, r, r,
                                    _lib.SVDMLP_BF16, _lib.SVDMLP_BF16, 0, torch.cuda.current_stream(gpu).cuda_stream)
    assert rc == _lib.SVDMLP_EINVAL
    msg = lib.svdmlp_last_error().decode()
    assert "fixed scratch" in msg and str(SCRATCH_BYTES) in msg


def _noalloc(lib, x, fs, y, dims, dev):
    T, d, ff, r_gu, r_d = dims
    bf = _lib.SVDMLP_BF16
    ld = _ld(fs)   # row pitches: the V factors may be row-padded
    return lib.svdmlp_svd_mlp_noalloc(x.data_ptr(), *_ptrs(fs), None, ctypes.addressof(ld), y.data_ptr(), T, d, ff,
                                      r_gu, r_d, bf, bf, 0, torch.cuda.current_stream(dev).cuda_stream)


def _status(lib, dev, reset=0, wait_bound=-1):
    rc = lib.svdmlp_noalloc_status(reset, wait_bound, torch.cuda.current_stream(dev).cuda_stream)
    assert rc in (0, 1), lib.svdmlp_last_error()
    return rc


def test_noalloc_timeout_poisons_output_and_status_resets(gpu):
    """A noalloc call whose grid-barrier waits give up (forced from the host
    with a wait bound of one poll, so every block still runs to its end)
    writes NaN into y; the scratch's flag stays set, so the next call writes
    NaN as well, until svdmlp_noalloc_status resets the scratch; then calls
    compute again (MFMA decode layer, 8 tokens)."""
    lib = _lib.load()
    shape, T = inputs.LayerShape(1024, 2048, 512), 8
    x, f = inputs.make_layer(shape, T=T, seed=93)
    xb, *fb = [inputs.as_float32(a, torch.bfloat16) for a in (x, *f)]
    xt = inputs.to_torch(xb, torch.bfloat16, gpu)
    fs = [inputs.to_torch(a, torch.bfloat16, gpu) for a in fb]
    dims = (T, shape.d, shape.ff, shape.r, shape.rd)
    ref = O.svd_mlp_ref(xb, *fb, dtype="bfloat16")
    y = torch.empty((T, shape.d), dtype=torch.bfloat16, device=gpu)

    def run():
        assert _noalloc(lib, xt, fs, y, dims, gpu) == 0, lib.svdmlp_last_error()
        torch.cuda.synchronize(gpu)
        return y.float().cpu().numpy()

    assert O.relative_l2(run(), ref) < 1e-2
    assert _status(lib, gpu) == 0
    _status(lib, gpu, wait_bound=1)
    assert np.isnan(run()).all()
    assert _status(lib, gpu) == 1
    _status(lib, gpu, wait_bound=0)      # the default bound again: the flag still poisons the result
    assert np.isnan(run()).all()
    assert _status(lib, gpu, reset=1) == 1   # reports, then zeroes the sync area
    assert _status(lib, gpu) == 0
    for _ in range(2):
        assert O.relative_l2(run(), ref) < 1e-2
    assert _status(lib, gpu) == 0


def test_noalloc_graph_capture_replays(gpu):
    """The noalloc entry point captured into a graph (torch.cuda.CUDAGraph):
    every replay, with eager work and synchronisation between replays,
    writes the eager call's bits, and eager calls change neither torch's
    allocated bytes nor the device's free memory (hipMemGetInfo)."""
    lib = _lib.load()
    shape = inputs.LayerShape(1024, 2048, 512)
    for T in (8, 1):   # the three-barrier MFMA decode layer, then the contracted one
        x, f = inputs.make_layer(shape, T=T, seed=95 + T)
        xb, *fb = [inputs.as_float32(a, torch.bfloat16) for a in (x, *f)]
        xt = inputs.to_torch(xb, torch.bfloat16, gpu)
        fs = [ops.pad_rows(a, 64) if i % 2 else a
              for i, a in enumerate(inputs.to_torch(a, torch.bfloat16, gpu) for a in fb)]
        dims = (T, shape.d, shape.ff, shape.r, shape.rd)
        y_eager = torch.empty((T, shape.d), dtype=torch.bfloat16, device=gpu)
        assert _noalloc(lib, xt, fs, y_eager, dims, gpu) == 0, lib.svdmlp_last_error()
        torch.cuda.synchronize(gpu)
        alloc0, free0 = torch.cuda.memory_allocated(gpu), torch.cuda.mem_get_info(gpu)[0]
        for _ in range(3):
            assert _noalloc(lib, xt, fs, y_eager, dims, gpu) == 0
        torch.cuda.synchronize(gpu)
        assert torch.cuda.memory_allocated(gpu) == alloc0 and torch.cuda.mem_get_info(gpu)[0] == free0
        y = torch.full((T, shape.d), 3.0, dtype=torch.bfloat16, device=gpu)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            rc = _noalloc(lib, xt, fs, y, dims, gpu)
        assert rc == 0, lib.svdmlp_last_error()
        for i in range(3):
            y.fill_(5.0)
            torch.cuda.synchronize(gpu)
            g.replay()
            torch.cuda.synchronize(gpu)
            assert torch.equal(y.view(torch.int16), y_eager.view(torch.int16)), (T, i)
            assert _noalloc(lib, xt, fs, y_eager, dims, gpu) == 0   # eager work between replays
            torch.cuda.synchronize(gpu)
        err = O.relative_l2(y.float().cpu().numpy(), O.svd_mlp_ref(xb, *fb, dtype="bfloat16"))
        assert err < 1e-2, (T, err)
        del g
    assert _status(lib, gpu) == 0
