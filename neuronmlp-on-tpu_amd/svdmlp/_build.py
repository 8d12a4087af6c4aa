"""Build libsvdmlp.so (HIP, gfx950) in-tree.

    python -m svdmlp._build            # from neuronmlp-on-tpu_amd/

Each ``csrc/*.hip`` translation unit is compiled by ``hipcc`` in parallel and
linked into ``svdmlp/libsvdmlp.so`` next to this file, so the library travels
with the source tree.  The shared library links ``libamdhip64.so.7`` by soname;
imported after torch it binds to the HIP runtime torch already loaded, so
streams and device pointers are shared with PyTorch.
"""

from __future__ import annotations

import concurrent.futures as cf
import json
import os
import re
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent  # neuronmlp-on-tpu_amd/
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
BUILD_DIR = ROOT / "_build"
LIB_PATH = PKG_DIR / "libsvdmlp.so"
# per-kernel registers, scratch and occupancy of the last build (the compiler's report)
RESOURCES = BUILD_DIR / "resources.json"
# the benchmark's streaming-read probe (csrc/probe/), its own library outside the SVD-MLP C ABI
PROBE_SRC = CSRC / "probe" / "hbm_read.hip"
PROBE_LIB = PKG_DIR / "libhbmread.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 ops stay disabled for all device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # The 4-wave large-tile kernels unroll 64 MFMA slots per k-step; a lower
    # pragma-unroll threshold leaves that loop rolled and the accumulators in
    # scratch memory.
    "-mllvm", "-pragma-unroll-threshold=100000",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the SVD-MLP HIP library cannot be built")


# The compiler's per-kernel resource report (registers, scratch, occupancy):
# collected into RESOURCES by build() and kept out of the build log.
REMARK_FLAG = "-Rpass-analysis=kernel-resource-usage"
_REMARK = re.compile(r"remark: (?:Function Name: (\S+)|\s+([^:]+): (\S+)) \[" + re.escape(REMARK_FLAG) + r"\]")


def _run(cmd: list[str]) -> str:
    """Run a build command; returns its output with the resource remarks, prints the rest."""
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    lines = [l for l in proc.stdout.splitlines() if noise not in l]
    # (a remark on a kernel defined in a header comes with its include chain)
    text = "\n".join(l for l in lines if REMARK_FLAG not in l and not l.startswith("In file included from"))
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{text}")
    if text.strip():
        print(text, file=sys.stderr)
    return "\n".join(lines)


def resources(text: str) -> dict[str, dict[str, str]]:
    """Kernel (mangled name) -> the resource report's fields, from build output."""
    out: dict[str, dict[str, str]] = {}
    cur = None
    for line in text.splitlines():
        m = _REMARK.search(line)
        if not m:
            continue
        if m.group(1):
            cur = out.setdefault(m.group(1), {})
        elif cur is not None:
            cur[m.group(2).strip()] = m.group(3)
    return out


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compile every HIP translation unit and link libsvdmlp.so; returns its path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [BUILD_DIR / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(8, os.cpu_count() or 1, len(srcs))

    def compile_one(pair):
        src, obj = pair
        cmd = [hipcc, *HIPCC_FLAGS, REMARK_FLAG, "-fno-caret-diagnostics", "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), file=sys.stderr)
        return resources(_run(cmd))

    report: dict[str, dict[str, str]] = {}
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        for r in pool.map(compile_one, zip(srcs, objs)):
            report.update(r)
    RESOURCES.write_text(json.dumps(report, indent=1, sort_keys=True))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, LIB_PATH)
    build_probe(hipcc)
    return LIB_PATH


def build_probe(hipcc: str | None = None) -> Path:
    """Compile and link the benchmark's streaming-read probe, libhbmread.so."""
    hipcc = hipcc or _hipcc()
    tmp = PROBE_LIB.with_suffix(".so.tmp")
    _run([hipcc, *HIPCC_FLAGS, "-shared", str(PROBE_SRC), "-o", str(tmp)])
    os.replace(tmp, PROBE_LIB)
    return PROBE_LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
