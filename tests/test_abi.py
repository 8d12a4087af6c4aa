"""The C ABI surface without a GPU: libsvdmlp.so loads, exports every symbol
include/svdmlp.h declares, and its host-only entry points (version, last
error, workspace size, argument validation -- all of which return before any
HIP call) behave as documented."""

import ctypes
import re
from pathlib import Path

import pytest

from svdmlp import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "svdmlp.h"


def _declared():
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(svdmlp_\w+)\s*\(", text, re.M))


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def test_header_and_binding_agree():
    assert _declared() == set(_lib.EXPORTED)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name


def test_header_constants_match_binding():
    text = HEADER.read_text()
    for name in ("SVDMLP_F32", "SVDMLP_BF16", "SVDMLP_FP8_E4M3", "SVDMLP_U_LINEAR", "SVDMLP_V_LINEAR",
                 "SVDMLP_OUT_T", "SVDMLP_X_T", "SVDMLP_CONTRACT"):
        m = re.search(rf"#define {name} (0x[0-9a-f]+|\d+)", text)
        assert m, name
        assert int(m.group(1), 0) == getattr(_lib, name), name
    for name, val in (("SVDMLP_EINVAL", -1), ("SVDMLP_EHIP", -2), ("SVDMLP_EUNSUP", -3), ("SVDMLP_OK", 0)):
        assert re.search(rf"#define {name} \(?{val}\)?", text), name


def test_version_and_workspace(lib):
    assert lib.svdmlp_version() == 100
    assert lib.svdmlp_workspace_bytes(0, 1, 1, 1, 1) == 0
    small = lib.svdmlp_workspace_bytes(1, 4096, 14336, 2816, 1)
    big = lib.svdmlp_workspace_bytes(1024, 4096, 14336, 2816, 1)
    assert 0 < small < big
    # prefill: bf16 XU (2*T*r*2) + fp32 XU (3*T*r*4) + h (T*ff*4)
    assert big >= 2 * 1024 * 2816 * 2 + 3 * 1024 * 2816 * 4 + 1024 * 14336 * 4
    # 1-4 tokens: the contracted layer's partial XU_d tiles, (r/128) x (ff/64) x T x 128 fp32
    for T in (1, 4):
        assert lib.svdmlp_workspace_bytes(T, 4096, 14336, 2816, 1) >= 22 * 224 * T * 512


def _call_gate_up(lib, T=4, d=16, ff=32, r=8, act=1, wt=1, flags=0, ptr=256, ws=1 << 20):
    p = ctypes.c_void_p(ptr)
    return lib.svdmlp_gate_up(p, p, p, p, p, None, None, None, None, p, T, d, ff, r, act, wt, flags,
                              p, ws, None)


def test_invalid_arguments_rejected_before_any_hip_call(lib):
    assert _call_gate_up(lib, T=0) == _lib.SVDMLP_EINVAL
    assert b"positive" in lib.svdmlp_last_error()
    assert _call_gate_up(lib, act=1, wt=0) == _lib.SVDMLP_EINVAL
    assert b"dtype" in lib.svdmlp_last_error()
    assert _call_gate_up(lib, wt=2) == _lib.SVDMLP_EINVAL          # fp8 without scales
    assert b"scales" in lib.svdmlp_last_error()
    assert _call_gate_up(lib, flags=0x8) == _lib.SVDMLP_EINVAL     # X_T is an xuv flag
    assert _call_gate_up(lib, ws=16) == _lib.SVDMLP_EINVAL
    assert b"workspace too small" in lib.svdmlp_last_error()
    assert _call_gate_up(lib, ptr=0) == _lib.SVDMLP_EINVAL
    assert b"null" in lib.svdmlp_last_error()
    p = ctypes.c_void_p(256)
    assert lib.svdmlp_xuv(p, p, p, None, None, p, 4, 16, 16, 0, 1, 1, 0, p, 1 << 20, None) == _lib.SVDMLP_EINVAL
    assert lib.svdmlp_svd_mlp(p, p, p, p, p, p, p, None, p, 4, 16, 32, 8, 8, 1, 2, 0, p, 1 << 20,
                              None) == _lib.SVDMLP_EINVAL
    # the two-rank entries validate as the one-rank ones (ranks must be positive, flags known)
    assert lib.svdmlp_svd_mlp_ranks(p, p, p, p, p, p, p, None, None, p, 4, 16, 32, 8, 0, 8, 1, 1, 0, p, 1 << 20,
                                    None) == _lib.SVDMLP_EINVAL
    assert b"positive" in lib.svdmlp_last_error()
    assert lib.svdmlp_svd_mlp_ranks(p, p, p, p, p, p, p, None, None, p, 4, 16, 32, 8, 16, 8, 1, 1, 0x40, p, 1 << 20,
                                    None) == _lib.SVDMLP_EINVAL
    assert b"unsupported flags" in lib.svdmlp_last_error()
    # SVDMLP_FP8_ACT (0x20) quantises activations for fp8 factors only
    assert lib.svdmlp_svd_mlp_ranks(p, p, p, p, p, p, p, None, None, p, 4, 16, 32, 8, 16, 8, 1, 1,
                                    _lib.SVDMLP_FP8_ACT, p, 1 << 20, None) == _lib.SVDMLP_EINVAL
    assert b"SVDMLP_FP8_ACT needs fp8 factors" in lib.svdmlp_last_error()
    assert lib.svdmlp_svd_mlp_block_ranks(p, p, ctypes.c_float(0.0), p, p, p, p, p, p, None, None, ctypes.c_void_p(512),
                                          4, 16, 32, 8, 16, 8, 1, 1, 0, p, 1 << 20, None) == _lib.SVDMLP_EINVAL
    assert b"eps" in lib.svdmlp_last_error()


def test_check_maps_status_to_exceptions(lib):
    _call_gate_up(lib, T=0)
    with pytest.raises(ValueError, match="positive"):
        _lib.check(_lib.SVDMLP_EINVAL)
    with pytest.raises(_lib.SvdMlpError):
        _lib.check(_lib.SVDMLP_EHIP)


def test_read_probe_library_validates_before_launch():
    """bench.py's streaming-read probe (libhbmread.so, csrc/probe/): built
    beside libsvdmlp.so, exports hbm_read_words, and rejects invalid
    arguments (-1) before any HIP call."""
    path = Path(_lib.__file__).resolve().parent / "libhbmread.so"
    assert path.exists(), f"{path} is not built"
    probe = ctypes.CDLL(str(path))
    fn = probe.hbm_read_words
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]
    fake, out = 0x1000, 0x2000  # never dereferenced: every case fails validation
    assert fn(None, 1 << 20, out, 1 << 23, 8192, None) == -1        # no buffer
    assert fn(fake, (1 << 20) + 8, out, 1 << 23, 8192, None) == -1  # not whole 16-byte words
    assert fn(fake + 8, 1 << 20, out, 1 << 23, 8192, None) == -1    # misaligned
    assert fn(fake, 1 << 20, out, 8192 * 256 * 4 - 4, 8192, None) == -1  # out too small for the grid
    assert fn(fake, 1 << 20, out, 1 << 23, 0, None) == -1           # no blocks
