"""The launcher API of the reference's test_speedup.py, on MI355X.

Drop-in names and argument meanings for the SVD-MLP path:

    fused_mlp_up_T(X, U, V, U_1, V_1, ...)          test_speedup.py:522-544
        -> (I, S) = [SiLU((X.U).V) * ((X.U_1).V_1)]^T
    fused_three_mm_XTUV(X_T, U, V, ...)             test_speedup.py:500-519
        -> (S, H) = (X_T^T . U) . V
    svd_mlp_with_fused_kernel(x, u_up, v_up, u_gate, v_gate, u_down, v_down,
                              up_T_params, XTUV_params, ...)  :631-655
    nki_mm(x, up_v_proj, up_u_proj, gate_v_proj, gate_u_proj,
           down_v_proj, down_u_proj, ...)          :658-666 (PyTorch layouts)
    get_fused_mlp_up_T_params(S), get_fused_three_mm_XTUV_params(S) :169-191
    jax_low_rank_down(hidden_t, u_down, v_down)     :618-628 (vendor down)
    nki_matmul_fully_optimized_(lhsT, rhs, ...)     :545-615 (plain matmul, lhsT.T . rhs)
    nki_baseline(x, up_proj, gate_proj, down_proj)  :669-678 (dense arm)
    _unfused_reference / _unfused_low_rank          :681-696 (comparison arms)
    _unfused_low_rank_pallas                        :699-735 (unfused arm on the plain matmul)

Block parameters (``*_tiles_in_block``) describe the TPU kernels' VMEM
blocking.  They are validated exactly as the reference does -- positive
integers and the 16 MiB x 0.8 VMEM working-set budget -- so callers see the
same ValueErrors; the HIP kernels then use their own LDS tiling.  The output
is the same either way.  ``interpret=True`` (the Pallas CPU emulator) has no
counterpart: the HIP kernels run only on the GPU, so it raises.
``async_dma`` and ``mixed_precision`` are accepted; the HIP kernels always
double-buffer and accumulate in fp32 (fp32 inputs are computed with fp32
MFMA, i.e. at least the precision of either reference mode).
"""

from __future__ import annotations

import functools
from typing import NamedTuple

import numpy as np
import torch

from . import ops

# Software tile sizes of the reference kernels (test_speedup.py:25-30).
M_TILE = 256
R_TILE = 256
K_TILE = 128
N_TILE = 512
VMEM_LIMIT = 16 * 1024 * 1024
VMEM_HEADROOM = 0.8

_ITEMSIZE = {torch.bfloat16: 2, torch.float32: 4, torch.float16: 2}


def _round_up(n: int, tile: int) -> int:
    return ((n + tile - 1) // tile) * tile


def _positive(name: str, value) -> None:
    """test_speedup.py:37-39."""
    if isinstance(value, bool) or not isinstance(value, (int, np.integer)) or value <= 0:
        raise ValueError(f"{name} must be a positive integer, got {value}")


def get_fused_mlp_up_T_params(S: int) -> dict:
    """Block counts of the Gate/Up launcher for S tokens (test_speedup.py:169-177)."""
    _positive("S", S)
    if S % 512 == 0:
        return dict(M_tiles_in_block=2, r_tiles_in_block=2, K_tiles_in_block=4, N_tiles_in_block=1)
    return dict(M_tiles_in_block=4, r_tiles_in_block=2, K_tiles_in_block=1 if S < 512 else 2,
                N_tiles_in_block=2)


def get_fused_three_mm_XTUV_params(S: int) -> dict:
    """Block counts of the Down launcher for S tokens (test_speedup.py:180-191)."""
    _positive("S", S)
    if S % 512 == 0:
        return dict(M_tiles_in_block=4, r_tiles_in_block=2, K_tiles_in_block=2 if S < 2048 else 4,
                    N_tiles_in_block=2)
    return dict(M_tiles_in_block=4, r_tiles_in_block=2, K_tiles_in_block=1 if S < 512 else 2,
                N_tiles_in_block=2)


class FusionShape(NamedTuple):
    """Block sizes, padded extents and VMEM estimate (test_speedup.py:195-204)."""

    M_block: int
    r_block: int
    K_block: int
    N_block: int
    M_padded: int
    r_padded: int
    K_padded: int
    N_padded: int
    vmem_bytes: int


def vmem_plan(mb, rb, kb, nb, mp, rp, npad, itemsize, gate, async_dma) -> dict:
    """The reference kernels' peak live VMEM (test_speedup.py:208-258): XU
    scratch lives across both stages; the U stage adds the input cache, the
    transpose staging and its weight slots, the V stage its weight slots and
    output staging; fp32 accumulators and per-tile temporaries on top."""
    nbr = 2 if gate else 1
    rank_blocks = -(-rp // rb)
    slots_u = 2 if async_dma and (mp // mb) * rank_blocks > 1 else 1
    slots_v = 2 if async_dma and (npad // nb) * rank_blocks > 1 else 1
    xu_scratch = nbr * rp * kb * itemsize
    staging_t = kb * M_TILE * itemsize if gate else 0
    out_tile = (N_TILE * kb if gate else K_TILE * nb) * itemsize
    u_stage = nbr * (slots_u * mb * rb * itemsize + min(rb, rp) * kb * 4)
    v_stage = nbr * (slots_v * rb * nb * itemsize + nb * kb * 4)
    scratch = nbr * max(R_TILE * K_TILE, N_TILE * K_TILE) * 8
    v_peak = xu_scratch + out_tile + v_stage + scratch

    def u_peak(rows):
        return xu_scratch + rows * kb * itemsize + staging_t + u_stage + scratch

    budget = VMEM_LIMIT * VMEM_HEADROOM
    cache_rows = mp if max(u_peak(mp), v_peak) < budget else mb
    return dict(estimated_vmem_bytes=max(u_peak(cache_rows), v_peak), input_cache_rows=cache_rows,
                xu_stage_peak_bytes=u_peak(cache_rows), xuv_stage_peak_bytes=v_peak)


def _check_vmem(estimate: int) -> None:
    """test_speedup.py:303-317: reject working sets over 16 MiB x 0.8."""
    budget = VMEM_LIMIT * VMEM_HEADROOM
    if estimate >= budget:
        raise ValueError(
            f"Estimated VMEM {estimate / 2**20:.2f} MiB exceeds {budget / 2**20:.2f} MiB budget "
            f"(overage: {(estimate - budget) / 2**20:.2f} MiB). Reduce tile counts to fit within budget.")


def _fusion_shape(M, r, K, N, dtype, M_count, r_count, K_count, N_count, gate, async_dma=True) -> FusionShape:
    """test_speedup.py:267-299: validate block counts, pad, check VMEM.  The
    plan is a pure function of its arguments and is remembered per argument
    tuple (the launchers validate on every call); a failing check raises
    every time."""
    try:
        return _fusion_shape_cached(M, r, K, N, dtype, M_count, r_count, K_count, N_count, gate, async_dma)
    except TypeError as exc:  # unhashable arguments: plan without the cache
        if "unhashable" not in str(exc):
            raise
        return _fusion_shape_plan(M, r, K, N, dtype, M_count, r_count, K_count, N_count, gate, async_dma)


@functools.lru_cache(maxsize=4096)
def _fusion_shape_cached(M, r, K, N, dtype, M_count, r_count, K_count, N_count, gate, async_dma):
    return _fusion_shape_plan(M, r, K, N, dtype, M_count, r_count, K_count, N_count, gate, async_dma)


def _fusion_shape_plan(M, r, K, N, dtype, M_count, r_count, K_count, N_count, gate, async_dma) -> FusionShape:
    for name, value in zip(("M_tiles_in_block", "r_tiles_in_block", "K_tiles_in_block", "N_tiles_in_block"),
                           (M_count, r_count, K_count, N_count)):
        _positive(name, value)
    mb, rb, kb, nb = M_TILE * M_count, R_TILE * r_count, K_TILE * K_count, N_TILE * N_count
    mp, rp, kp, npad = _round_up(M, mb), _round_up(r, R_TILE), _round_up(K, kb), _round_up(N, nb)
    itemsize = _ITEMSIZE.get(dtype, 2)
    est = vmem_plan(mb, rb, kb, nb, mp, rp, npad, itemsize, gate, async_dma)["estimated_vmem_bytes"]
    _check_vmem(est)
    return FusionShape(mb, rb, kb, nb, mp, rp, kp, npad, est)


def _no_interpret(interpret: bool) -> None:
    if interpret:
        raise NotImplementedError(
            "interpret=True selects the Pallas CPU emulator; the MI355X kernels run on the GPU only")


def fused_mlp_up_T(X_ref, U_ref, V_ref, U_ref_1, V_ref_1, mixed_precision=True, r_tiles_in_block=2,
                   K_tiles_in_block=1, N_tiles_in_block=2, M_tiles_in_block=4, *, interpret=False,
                   async_dma=True):
    """Return transposed SiLU((X U) V) * ((X U_1) V_1), shape (I, S)
    (test_speedup.py:522-544)."""
    ops.validate_arrays(X_ref, U_ref, V_ref, U_ref_1, V_ref_1)
    K, M = X_ref.shape
    if U_ref.shape[0] != M or V_ref.shape[0] != U_ref.shape[1]:
        raise ValueError("X, U, V contraction dimensions do not match")
    if tuple(U_ref_1.shape) != tuple(U_ref.shape) or tuple(V_ref_1.shape) != tuple(V_ref.shape):
        raise ValueError("gate/up factors must have matching shapes")
    r, N = V_ref.shape
    _fusion_shape(M, r, K, N, X_ref.dtype, M_tiles_in_block, r_tiles_in_block, K_tiles_in_block,
                  N_tiles_in_block, gate=True, async_dma=async_dma)
    _no_interpret(interpret)
    return ops.fused_gate_up(X_ref, U_ref, V_ref, U_ref_1, V_ref_1, out_transposed=True)


def fused_three_mm_XTUV(X_ref, U_ref, V_ref, mixed_precision=True, r_tiles_in_block=2, K_tiles_in_block=1,
                        N_tiles_in_block=2, M_tiles_in_block=4, *, interpret=False, async_dma=True):
    """Return X_ref.T @ U_ref @ V_ref with X_ref given as (I, S)
    (test_speedup.py:500-519)."""
    ops.validate_arrays(X_ref, U_ref, V_ref)
    M, K = X_ref.shape
    if U_ref.shape[0] != M or V_ref.shape[0] != U_ref.shape[1]:
        raise ValueError("X, U, V contraction dimensions do not match")
    r, N = V_ref.shape
    _fusion_shape(M, r, K, N, X_ref.dtype, M_tiles_in_block, r_tiles_in_block, K_tiles_in_block,
                  N_tiles_in_block, gate=False, async_dma=async_dma)
    _no_interpret(interpret)
    return ops.fused_xuv(X_ref, U_ref, V_ref, x_transposed=True)


def jax_low_rank_down(hidden_t, u_down, v_down):
    """Vendor-library Down from (I, S) (test_speedup.py:618-628): hipBLASLt
    GEMMs via torch at the input dtype's GEMM boundaries, fp32 accumulate."""
    ops.validate_arrays(hidden_t, u_down, v_down)
    if hidden_t.shape[0] != u_down.shape[0] or u_down.shape[1] != v_down.shape[0]:
        raise ValueError("hidden, U, V contraction dimensions do not match")
    return (hidden_t.t() @ u_down) @ v_down


def svd_mlp_with_fused_kernel(x, u_up, v_up, u_gate, v_gate, u_down, v_down, up_T_params=None,
                              XTUV_params=None, *, mixed_precision=True, interpret=False, async_dma=True,
                              down_backend="pallas"):
    """Gate/Up kernel followed by the Down kernel (test_speedup.py:631-655);
    up-first argument order.  ``down_backend="pallas"`` runs the fused HIP
    layer (h stays on chip-side workspace, natural layout throughout);
    ``"jax"`` runs the Gate/Up kernel then the vendor Down."""
    if down_backend not in ("pallas", "jax"):
        raise ValueError("down_backend must be 'pallas' or 'jax'")
    S = x.shape[0]
    if up_T_params is None:
        up_T_params = get_fused_mlp_up_T_params(S)
    if down_backend == "pallas" and XTUV_params is None:
        XTUV_params = get_fused_three_mm_XTUV_params(S)
    ops.validate_arrays(x, u_gate, v_gate, u_up, v_up)
    H = x.shape[1]
    r, I = v_gate.shape
    _fusion_shape(H, r, S, I, x.dtype, up_T_params["M_tiles_in_block"], up_T_params["r_tiles_in_block"],
                  up_T_params["K_tiles_in_block"], up_T_params["N_tiles_in_block"], gate=True, async_dma=async_dma)
    _no_interpret(interpret)
    if down_backend == "jax":
        hidden_t = ops.fused_gate_up(x, u_gate, v_gate, u_up, v_up, out_transposed=True)
        return jax_low_rank_down(hidden_t, u_down, v_down)
    ops.validate_arrays(u_down, v_down)
    _fusion_shape(I, u_down.shape[1], S, v_down.shape[1], x.dtype, XTUV_params["M_tiles_in_block"],
                  XTUV_params["r_tiles_in_block"], XTUV_params["K_tiles_in_block"],
                  XTUV_params["N_tiles_in_block"], gate=False, async_dma=async_dma)
    return ops.svd_mlp(x, u_gate, v_gate, u_up, v_up, u_down, v_down)


def nki_mm(x, up_v_proj, up_u_proj, gate_v_proj, gate_u_proj, down_v_proj, down_u_proj, *,
           mixed_precision=True, interpret=False, up_T_params=None, XTUV_params=None, async_dma=True,
           down_backend="pallas"):
    """PyTorch ``Linear.weight`` layouts (out, in) (test_speedup.py:658-666).
    The ``.T`` views are handed to the kernels without copies."""
    return svd_mlp_with_fused_kernel(
        x, up_v_proj.T, up_u_proj.T, gate_v_proj.T, gate_u_proj.T, down_v_proj.T, down_u_proj.T,
        up_T_params, XTUV_params, mixed_precision=mixed_precision, interpret=interpret, async_dma=async_dma,
        down_backend=down_backend)


def _unfused_reference(x, u_up, v_up, u_gate, v_gate, u_down, v_down):
    """fp32 comparison arm on the GPU (test_speedup.py:681-687)."""
    x, u_up, v_up, u_gate, v_gate, u_down, v_down = (
        a.float() for a in (x, u_up, v_up, u_gate, v_gate, u_down, v_down))
    gate = (x @ u_gate) @ v_gate
    up = (x @ u_up) @ v_up
    return ((torch.nn.functional.silu(gate) * up) @ u_down) @ v_down


def _unfused_low_rank(x, u_up, v_up, u_gate, v_gate, u_down, v_down):
    """Vendor (hipBLASLt) arm at the input dtype (test_speedup.py:690-696)."""
    gate = (x @ u_gate) @ v_gate
    up = (x @ u_up) @ v_up
    hidden = torch.nn.functional.silu(gate.float()).to(x.dtype) * up
    return (hidden @ u_down) @ v_down


def nki_matmul_fully_optimized_(lhsT, rhs, TILES_IN_BLOCK_M=2, TILES_IN_BLOCK_N=2, TILES_IN_BLOCK_K=4, *,
                                mixed_precision=True, interpret=False):
    """The reference's plain matmul kernel (test_speedup.py:545-615):
    lhsT (K, M), rhs (K, N) -> (M, N) = lhsT^T . rhs at the input dtype.

    It is the building block of the dense and unfused comparison arms, not of
    the SVD-MLP path, so it runs on the vendor library (hipBLASLt via torch;
    the transposed operand is made contiguous first).  The validation and
    the VMEM estimate follow the reference, so the same shapes raise."""
    ops.validate_arrays(lhsT, rhs)
    K, M = lhsT.shape
    if rhs.shape[0] != K:
        raise ValueError("lhsT and rhs must have the same contraction dimension")
    N = rhs.shape[1]
    for name, value in zip(("TILES_IN_BLOCK_M", "TILES_IN_BLOCK_N", "TILES_IN_BLOCK_K"),
                           (TILES_IN_BLOCK_M, TILES_IN_BLOCK_N, TILES_IN_BLOCK_K)):
        _positive(name, value)
    TILE_M, TILE_K, TILE_N = K_TILE, M_TILE, N_TILE
    BLOCK_M, BLOCK_K, BLOCK_N = TILE_M * TILES_IN_BLOCK_M, TILE_K * TILES_IN_BLOCK_K, TILE_N * TILES_IN_BLOCK_N
    Mp = _round_up(M, BLOCK_M)
    itemsize = _ITEMSIZE[lhsT.dtype]
    _check_vmem((Mp * BLOCK_N + BLOCK_K * BLOCK_N + BLOCK_K * BLOCK_M + TILE_M * BLOCK_N) * itemsize
                + TILE_M * TILE_N * 8)
    _no_interpret(interpret)
    if lhsT.device.type != "cuda":
        raise ValueError(f"the matmul arm runs on a ROCm GPU; got tensors on {lhsT.device}")
    return lhsT.t().contiguous() @ rhs


def nki_baseline(x, up_proj, gate_proj, down_proj, *, mixed_precision=True, interpret=False,
                 matmul_params=None):
    """Dense SwiGLU comparison arm with ``Linear.weight`` layouts (out, in)
    (test_speedup.py:669-678): silu(x.Wg) * (x.Wu), then .Wd, with the SiLU
    product in fp32 rounded to x.dtype."""
    params = {} if matmul_params is None else matmul_params
    up = nki_matmul_fully_optimized_(x.t(), up_proj.t(), **params, mixed_precision=mixed_precision,
                                     interpret=interpret)
    gate = nki_matmul_fully_optimized_(x.t(), gate_proj.t(), **params, mixed_precision=mixed_precision,
                                       interpret=interpret)
    act = torch.nn.functional.silu(gate.float()).to(x.dtype) * up
    return nki_matmul_fully_optimized_(act.t(), down_proj.t(), **params, mixed_precision=mixed_precision,
                                       interpret=interpret)


def _unfused_low_rank_pallas(x, u_up, v_up, u_gate, v_gate, u_down, v_down, *, mixed_precision=True,
                             interpret=False):
    """Unfused low-rank arm on the same plain matmul as the dense arm
    (test_speedup.py:699-735): six GEMMs, SiLU in fp32 rounded to x.dtype."""
    mm = lambda a, b: nki_matmul_fully_optimized_(a, b, mixed_precision=mixed_precision,  # noqa: E731
                                                  interpret=interpret)
    gate = mm(mm(x.t(), u_gate).t(), v_gate)
    up = mm(mm(x.t(), u_up).t(), v_up)
    hidden = torch.nn.functional.silu(gate.float()).to(x.dtype) * up
    return mm(mm(hidden.t(), u_down).t(), v_down)


def relative_l2(got, expected) -> float:
    """test_speedup.py:854 / bench/speedup.py:113-119."""
    g = got.float()
    e = expected.float()
    return float(torch.linalg.norm(g - e) / torch.clamp(torch.linalg.norm(e), min=1e-12))


def tflops(T: int, d: int, ff: int, r: int, r_down: int | None = None) -> float:
    """Algorithmic TFLOP of one SVD-MLP layer: 2*T*(2*r*(d+ff) + r_d*(ff+d))."""
    rd = r if r_down is None else r_down
    return 2.0 * T * (2 * r * (d + ff) + rd * (ff + d)) / 1e12


__all__ = [
    "M_TILE", "R_TILE", "K_TILE", "N_TILE", "VMEM_LIMIT", "VMEM_HEADROOM", "FusionShape",
    "get_fused_mlp_up_T_params", "get_fused_three_mm_XTUV_params", "fused_mlp_up_T", "fused_three_mm_XTUV",
    "jax_low_rank_down", "svd_mlp_with_fused_kernel", "nki_mm", "nki_matmul_fully_optimized_", "nki_baseline",
    "relative_l2", "tflops",
]
