"""ctypes binding of libsvdmlp.so (declared in include/svdmlp.h).

The library is loaded lazily, after ``torch`` so that its ``libamdhip64.so.7``
dependency resolves (by soname) to the HIP runtime torch already mapped; the
loader then checks that exactly one HIP runtime is mapped in the process, so
torch streams and device pointers are valid inside the library.  There is no
fallback: a missing or unloadable library raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsvdmlp.so"

# Constants mirrored from include/svdmlp.h
SVDMLP_F32 = 0
SVDMLP_BF16 = 1
SVDMLP_FP8_E4M3 = 2
SVDMLP_U_LINEAR = 0x1
SVDMLP_V_LINEAR = 0x2
SVDMLP_OUT_T = 0x4
SVDMLP_X_T = 0x8
SVDMLP_CONTRACT = 0x10
SVDMLP_FP8_ACT = 0x20
SVDMLP_OK = 0
SVDMLP_EINVAL = -1
SVDMLP_EHIP = -2
SVDMLP_EUNSUP = -3

# Every symbol include/svdmlp.h declares.
EXPORTED = (
    "svdmlp_version",
    "svdmlp_last_error",
    "svdmlp_workspace_bytes",
    "svdmlp_workspace_status",
    "svdmlp_gate_up",
    "svdmlp_xuv",
    "svdmlp_svd_mlp",
    "svdmlp_svd_mlp_block",
    "svdmlp_svd_mlp_ld",
    "svdmlp_svd_mlp_block_ld",
    "svdmlp_svd_mlp_ranks",
    "svdmlp_svd_mlp_block_ranks",
    "svdmlp_svd_mlp_noalloc",
    "svdmlp_noalloc_status",
    "svdmlp_profile_enable",
    "svdmlp_profile_read",
    "svdmlp_stage_name",
)

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_u32 = ctypes.c_uint32
_sz = ctypes.c_size_t


class SvdMlpError(RuntimeError):
    """A call into libsvdmlp.so returned a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def _declare(lib: ctypes.CDLL) -> None:
    lib.svdmlp_version.restype = ctypes.c_int
    lib.svdmlp_version.argtypes = []
    lib.svdmlp_last_error.restype = ctypes.c_char_p
    lib.svdmlp_last_error.argtypes = []
    lib.svdmlp_workspace_bytes.restype = _sz
    lib.svdmlp_workspace_bytes.argtypes = [_i64, _i64, _i64, _i64, _i32]
    lib.svdmlp_workspace_status.restype = ctypes.c_int
    lib.svdmlp_workspace_status.argtypes = [_vp, _sz, _i32, _vp]
    lib.svdmlp_gate_up.restype = ctypes.c_int
    lib.svdmlp_gate_up.argtypes = [_vp] * 5 + [_vp] * 4 + [_vp] + [_i64] * 4 + [_i32, _i32, _u32, _vp, _sz, _vp]
    lib.svdmlp_xuv.restype = ctypes.c_int
    lib.svdmlp_xuv.argtypes = [_vp] * 3 + [_vp] * 2 + [_vp] + [_i64] * 4 + [_i32, _i32, _u32, _vp, _sz, _vp]
    lib.svdmlp_svd_mlp.restype = ctypes.c_int
    lib.svdmlp_svd_mlp.argtypes = [_vp] * 7 + [_vp, _vp] + [_i64] * 5 + [_i32, _i32, _u32, _vp, _sz, _vp]
    lib.svdmlp_svd_mlp_block.restype = ctypes.c_int
    lib.svdmlp_svd_mlp_block.argtypes = ([_vp, _vp, ctypes.c_float] + [_vp] * 6 + [_vp, _vp] + [_i64] * 5
                                         + [_i32, _i32, _u32, _vp, _sz, _vp])
    lib.svdmlp_svd_mlp_ld.restype = ctypes.c_int
    lib.svdmlp_svd_mlp_ld.argtypes = [_vp] * 7 + [_vp, _vp, _vp] + [_i64] * 5 + [_i32, _i32, _u32, _vp, _sz, _vp]
    lib.svdmlp_svd_mlp_block_ld.restype = ctypes.c_int
    lib.svdmlp_svd_mlp_block_ld.argtypes = ([_vp, _vp, ctypes.c_float] + [_vp] * 6 + [_vp, _vp, _vp] + [_i64] * 5
                                            + [_i32, _i32, _u32, _vp, _sz, _vp])
    lib.svdmlp_svd_mlp_ranks.restype = ctypes.c_int
    lib.svdmlp_svd_mlp_ranks.argtypes = [_vp] * 7 + [_vp, _vp, _vp] + [_i64] * 6 + [_i32, _i32, _u32, _vp, _sz, _vp]
    lib.svdmlp_svd_mlp_block_ranks.restype = ctypes.c_int
    lib.svdmlp_svd_mlp_block_ranks.argtypes = ([_vp, _vp, ctypes.c_float] + [_vp] * 6 + [_vp, _vp, _vp]
                                               + [_i64] * 6 + [_i32, _i32, _u32, _vp, _sz, _vp])
    lib.svdmlp_svd_mlp_noalloc.restype = ctypes.c_int
    lib.svdmlp_svd_mlp_noalloc.argtypes = [_vp] * 7 + [_vp, _vp, _vp] + [_i64] * 5 + [_i32, _i32, _u32, _vp]
    lib.svdmlp_noalloc_status.restype = ctypes.c_int
    lib.svdmlp_noalloc_status.argtypes = [_i32, _i64, _vp]
    lib.svdmlp_profile_enable.restype = ctypes.c_int
    lib.svdmlp_profile_enable.argtypes = [ctypes.c_int]
    lib.svdmlp_profile_read.restype = ctypes.c_int
    lib.svdmlp_profile_read.argtypes = [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64),
                                        ctypes.c_int]
    lib.svdmlp_stage_name.restype = ctypes.c_char_p
    lib.svdmlp_stage_name.argtypes = [ctypes.c_int]


def _mapped_hip_runtimes() -> set[str]:
    found = set()
    try:
        with open("/proc/self/maps", encoding="utf-8") as fh:
            for line in fh:
                path = line.rsplit(None, 1)[-1] if "/" in line else ""
                if "libamdhip64.so" in path:
                    found.add(os.path.realpath(path))
    except OSError:
        pass
    return found


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and return the library; raises RuntimeError if unavailable."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  (binds the HIP runtime first)

        lib_path = Path(path) if path is not None else LIB_PATH
        if not lib_path.is_file():
            raise RuntimeError(
                f"libsvdmlp.so not found at {lib_path}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950)"
            )
        try:
            lib = ctypes.CDLL(str(lib_path), mode=ctypes.RTLD_LOCAL)
        except OSError as exc:
            raise RuntimeError(f"failed to load {lib_path}: {exc}") from exc
        _declare(lib)
        runtimes = _mapped_hip_runtimes()
        if len(runtimes) > 1:
            raise RuntimeError(
                "two HIP runtimes are mapped in this process "
                f"({sorted(runtimes)}); libsvdmlp.so must share torch's runtime"
            )
        _lib = lib
        return lib


def is_loaded() -> bool:
    return _lib is not None


def check(status: int) -> None:
    if status != SVDMLP_OK:
        msg = load().svdmlp_last_error().decode("utf-8", "replace")
        if status == SVDMLP_EINVAL:
            raise ValueError(msg)
        raise SvdMlpError(status, msg)


def version() -> int:
    return int(load().svdmlp_version())


def workspace_bytes(T: int, d: int, ff: int, r: int, w_dtype: int) -> int:
    return int(load().svdmlp_workspace_bytes(T, d, ff, r, w_dtype))


class StageProfile:
    """Per-stage GPU time of the library's launches (hipEvents on the
    caller's stream).  ``with StageProfile() as prof: ...`` then
    ``prof.result`` maps stage name -> (total_ms, launches)."""

    def __init__(self):
        self.result: dict[str, tuple[float, int]] = {}

    def __enter__(self):
        lib = load()
        lib.svdmlp_profile_read(None, None, 0)  # drop anything stale
        lib.svdmlp_profile_enable(1)
        return self

    def __exit__(self, *exc):
        lib = load()
        n = lib.svdmlp_profile_enable(0)
        ms = (ctypes.c_double * n)()
        cnt = (ctypes.c_int64 * n)()
        rc = lib.svdmlp_profile_read(ms, cnt, n)
        if rc < 0:
            check(rc)
        self.result = {lib.svdmlp_stage_name(i).decode(): (ms[i], cnt[i]) for i in range(n) if cnt[i]}
        return False
