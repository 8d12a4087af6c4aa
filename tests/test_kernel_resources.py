"""Register and scratch budgets of the HIP kernels, from the compiler's own
resource report of the last build (``svdmlp._build.RESOURCES``, written by
``__graft_entry__.build()``).

A kernel that spills to scratch memory, or that needs more registers than the
build it was tuned on, runs slower without any test failing: a change to the
large-tile kernel's block-to-tile arithmetic once cost the fp8-factor
instances ~20 VGPRs and made the 256 x 256 ones spill (70B XU_d . Vd 149 ->
202 us).  These tests hold every kernel to no scratch (one listed exception)
and the hot kernels to their recorded register counts.  The baseline
(``tests/kernel_registers_baseline.json``) is rewritten on purpose, with the
timing that justifies the change.
"""

import json
from pathlib import Path

import pytest

from svdmlp import _build

BASELINE = Path(__file__).resolve().parent / "kernel_registers_baseline.json"

# The 4-wave fp8-factor large-tile instance with fp32 slices (BigCfg<8, false,
# 0, true, true, 4, 4, 1, false>): 256 accumulator registers per wave; only
# SVDMLP_TUNE=nw=4 launches it.
SCRATCH_ALLOWED = {"_ZN6svdmlp15big_gemm_kernelINS_6BigCfgILi8ELb0ELi0ELb1ELb1ELi4ELi4ELi1ELb0EEEEEvNS_9BigParamsE"}
SLACK = 4  # VGPRs (or AGPRs) a kernel may grow by without a new baseline


def _report():
    if not _build.RESOURCES.exists():
        pytest.skip("no resource report: run __graft_entry__.build() first")
    return json.loads(_build.RESOURCES.read_text())


def test_report_covers_the_kernels():
    rep = _report()
    names = set(rep)
    for frag in ("big_gemm_kernel", "f8_gemm_kernel", "decode_layer_kernel", "gemv_layer_kernel",
                 "reduce_frag_bf16_kernel"):
        assert any(frag in n for n in names), frag
    for n, r in rep.items():
        assert {"VGPRs", "AGPRs", "ScratchSize [bytes/lane]", "VGPRs Spill"} <= set(r), n


def test_no_scratch_memory():
    rep = _report()
    bad = {n: r["ScratchSize [bytes/lane]"] for n, r in rep.items()
           if n not in SCRATCH_ALLOWED and (int(r["ScratchSize [bytes/lane]"]) > 0 or int(r["VGPRs Spill"]) > 0)}
    assert not bad, f"kernels using scratch memory: {bad}"


def test_hot_kernels_within_register_baseline():
    rep = _report()
    base = json.loads(BASELINE.read_text())
    missing = sorted(n for n in base if n not in rep)
    assert not missing, f"kernels of the baseline no longer built: {missing}"
    grown = {n: (b, {"VGPRs": int(rep[n]["VGPRs"]), "AGPRs": int(rep[n]["AGPRs"])}) for n, b in base.items()
             if int(rep[n]["VGPRs"]) > b["VGPRs"] + SLACK or int(rep[n]["AGPRs"]) > b["AGPRs"] + SLACK}
    assert not grown, f"kernels above their recorded registers (baseline, now): {grown}"
