"""The ``svdflash_tpu.kernels.pallas_ops`` operator API on MI355X.

The reference's benches import these names from a module that is absent from
its snapshot; signatures and keyword arguments follow their call sites:

    svd_mlp(x, ug, vg, uu, vu, ud, vd, gate_up_blocks=...)   bench/speedup.py:142-146,
                                                              models/modeling_llama.py:848-858
    fused_gate_up(x, ug, vg, uu, vu, blocks=...)             bench/smoke.py:79-83, bench/latency.py:373-375
    xuv_matmul(x, u, v)                                      bench/smoke.py:59-67, bench/latency.py:346
    dense_mlp(x, w_gate, w_up, w_down)                       bench/speedup.py:141
    contracted_svd_mlp(x, ug, vg, uu, vu, ud, vd, gate_up_blocks=...)
                                                              models/modeling_llama.py:865-886,
                                                              bench/latency.py:416-432

All take natural layouts and gate-first factor order, as kernels/reference.py
does, and return freshly allocated outputs.

* ``gate_up_blocks`` / ``blocks`` (``config.GateUpBlocks``, the TPU kernels'
  VMEM blocking) are validated as positive integers and otherwise unused: the
  HIP kernels choose their own LDS tiles; the result does not depend on them.
* ``mixed_precision`` is accepted: bf16 inputs always run bf16 MFMA with fp32
  accumulation, fp32 inputs fp32 MFMA (at least the precision of either
  reference mode).
* ``interpret=True`` (the Pallas CPU emulator) has no counterpart and raises.
* ``contracted_svd_mlp`` is the variant whose boundary is the rank-r Down-XU
  instead of h (models/modeling_llama.py:865-886).  At 1-4 tokens it runs the
  contracted decode layer (SVDMLP_CONTRACT): every block computes a 64-column
  strip of h, keeps it in LDS and multiplies it by the matching rows of Ud,
  so h never leaves the block and only fp32 (T, r_d) partials of XU_d cross
  blocks, summed in a fixed order.  Other shapes run the two-kernel layer
  (same y): for prefill, carrying h through the Down-U product on a GPU
  either writes a (rows x r_d) fp32 partial per h strip (64 strips of 224
  columns at 8B, ~740 MB at 1024 tokens, against h's 29 MB) or recomputes h
  once per rank tile; at 5-128 tokens the partials outgrow h's round trip
  inside the persistent layer.
* ``dense_mlp`` is the uncompressed SwiGLU of the dense comparison arm
  (kernels/reference.py:96-106); it runs on the vendor library (hipBLASLt via
  torch) at the input dtype with the SiLU product in fp32.
"""

from __future__ import annotations

import torch

from . import ops
from .config import GateUpBlocks


def _check_blocks(blocks, what: str) -> None:
    if blocks is None:
        return
    fields = blocks._asdict() if isinstance(blocks, GateUpBlocks) else dict(
        zip(GateUpBlocks._fields, tuple(blocks)))
    if len(fields) != len(GateUpBlocks._fields):
        raise ValueError(f"{what} must have the four fields {GateUpBlocks._fields}")
    for name, value in fields.items():
        if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
            raise ValueError(f"{what}.{name} must be a positive integer, got {value}")


def _check_interpret(interpret: bool) -> None:
    if interpret:
        raise NotImplementedError("interpret=True (the Pallas CPU emulator) has no MI355X counterpart; "
                                  "the HIP kernels run only on the GPU")


def svd_mlp(x, u_gate, v_gate, u_up, v_up, u_down, v_down, *, gate_up_blocks=None, mixed_precision=True,
            interpret=False) -> torch.Tensor:
    """The fused SVD-MLP layer (kernels/reference.py:85-93 semantics)."""
    _check_blocks(gate_up_blocks, "gate_up_blocks")
    _check_interpret(interpret)
    return ops.svd_mlp(x, u_gate, v_gate, u_up, v_up, u_down, v_down)


def fused_gate_up(x, u_gate, v_gate, u_up, v_up, *, blocks=None, mixed_precision=True,
                  interpret=False) -> torch.Tensor:
    """SiLU(x.ug.vg) * (x.uu.vu), natural (S, I) output (kernels/reference.py:54-72)."""
    _check_blocks(blocks, "blocks")
    _check_interpret(interpret)
    return ops.fused_gate_up(x, u_gate, v_gate, u_up, v_up)


def xuv_matmul(x, u, v, *, mixed_precision=True, interpret=False) -> torch.Tensor:
    """(x.u).v with the rank-r intermediate rounded to x.dtype (kernels/reference.py:75-82)."""
    _check_interpret(interpret)
    return ops.fused_xuv(x, u, v)


def contracted_svd_mlp(x, u_gate, v_gate, u_up, v_up, u_down, v_down, *, gate_up_blocks=None,
                       mixed_precision=True, interpret=False) -> torch.Tensor:
    """The contracted variant: h kept inside the kernel, (T, r_d) partials of
    Down-XU as the only cross-block data (same y as :func:`svd_mlp` up to
    fp32 summation order)."""
    _check_blocks(gate_up_blocks, "gate_up_blocks")
    _check_interpret(interpret)
    return ops.svd_mlp(x, u_gate, v_gate, u_up, v_up, u_down, v_down, contracted=True)


def dense_mlp(x, w_gate, w_up, w_down, *, mixed_precision=True, interpret=False) -> torch.Tensor:
    """Dense SwiGLU (kernels/reference.py:96-106): w_gate, w_up (H, I), w_down (I, H)."""
    _check_interpret(interpret)
    ops.validate_arrays(x, w_gate, w_up, w_down)
    H = x.shape[1]
    if w_gate.shape != w_up.shape or w_gate.shape[0] != H or w_down.shape != (w_gate.shape[1], H):
        raise ValueError("dense MLP weight shapes do not match")
    if x.device.type != "cuda":
        raise ValueError(f"the dense arm runs on a ROCm GPU; got tensors on {x.device}")
    gate = x @ w_gate
    up = x @ w_up
    hidden = (torch.nn.functional.silu(gate.float()) * up.float()).to(x.dtype)
    return hidden @ w_down


__all__ = ["svd_mlp", "fused_gate_up", "xuv_matmul", "contracted_svd_mlp", "dense_mlp"]
