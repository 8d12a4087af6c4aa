"""CPU oracle for the SVD-MLP hot path -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the reference's golden math for the path
(``kernels/reference.py`` of n-paradigm/NeuronMLP-on-TPU) plus the number
formats the MI355X build uses.  It is the checker, never the product: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The HIP library never calls into it and the
package ``svdmlp`` never imports it.

Every function cites the reference lines it follows.  What pins each one
(tests/test_oracle.py):

  round_bf16 ......... torch's independent float32->bfloat16 cast (RNE) on
                       every tie/edge class, plus NaN/Inf/overflow cases.
  e4m3_decode ........ exhaustive 256-code table against the closed form and
                       torch.float8_e4m3fn.
  e4m3_encode ........ torch.float8_e4m3fn cast (RNE, saturating) on dense
                       grids incl. midpoints; round-trip of all finite codes.
  quantize_per_channel amax/448 definition; reconstruction error bound.
  quantize_rows_e4m3 . per-row amax/448 scale; codes equal to torch's e4m3fn
                       cast of the row times 448/amax; every element within
                       half an e4m3 step of its code's value; zero rows.
  svd_mlp_fp8_act_ref  equals svd_mlp_ref when h is already on the row grid
                       (quantising a quantised h changes nothing); error
                       against svd_mlp_ref within the e4m3 budget.
  silu ............... closed form x*sigmoid(x) in float64, silu(0)=0, limits,
                       the identity silu(x)-silu(-x)=x, torch silu (<=2 ulp).
  low_rank_dim ....... known answers 1280/1792/2560 (reference.py:29-31),
                       2816 at c=0.9 (models/README.md:67), 3200 at c=1.0
                       (e2e_block.py:324 ratio 0.88), half-even ties.
  fused_gate_up_ref .. float64 triple-loop brute force on tiny shapes;
                       U = I reduces it to dense_mlp's gate/up; zero U -> 0;
                       linearity in V_up.
  fused_xuv_ref ...... brute force; associativity (x.u).v = x.(u.v) in f64.
  svd_mlp_ref ........ equals xuv(round(gate_up(x))) and dense_mlp_ref when
                       W = U.V with identity U.
  rmsnorm_ref ........ closed form on constant rows (output = gain*sign),
                       scale invariance, float64 brute force.
  mlp_block_f64 ...... float64 triple-loop brute force of the whole block on a
                       tiny shape; agrees with mlp_block_ref in float32.
  relative_l2 ........ hand-computed vectors; NaN rejection.
  factor_bytes ....... 311,427,072 B for the 8B layer at r=2816
                       (results/real_layer0_cpu.json:21; profiler test :20).
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "round_bf16",
    "bf16_bits",
    "bf16_from_bits",
    "e4m3_decode",
    "e4m3_encode",
    "quantize_per_channel",
    "quantize_rows_e4m3",
    "svd_mlp_fp8_act_ref",
    "silu",
    "low_rank_dim",
    "fused_gate_up_ref",
    "fused_xuv_ref",
    "svd_mlp_ref",
    "dense_mlp_ref",
    "unfused_reference",
    "rmsnorm_ref",
    "mlp_block_ref",
    "mlp_block_f64",
    "relative_l2",
    "errors",
    "factor_bytes",
    "layer_flops",
]

F32 = np.float32

# ---------------------------------------------------------------------------
# Number formats
# ---------------------------------------------------------------------------


def bf16_bits(a) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even.

    NaN maps to a quiet NaN with its sign; overflow rounds to +-Inf, which is
    what RNE on the top 16 bits gives.  (The reference's ``.astype(x.dtype)``
    to bfloat16 is ml_dtypes' RNE cast.)
    """
    u = np.ascontiguousarray(np.asarray(a, dtype=F32)).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = (u + (0x7FFF + ((u >> 16) & 1))) >> 16
    out = np.where(nan, (u >> 16) | 0x40, rounded)
    return out.astype(np.uint16)


def bf16_from_bits(b) -> np.ndarray:
    """bfloat16 bit patterns (uint16) -> float32 (exact)."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(F32)


def round_bf16(a) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 value, returned as float32."""
    return bf16_from_bits(bf16_bits(a))


def e4m3_decode(bits) -> np.ndarray:
    """fp8 e4m3fn (OCP FN variant: bias 7, no infinities, S.1111.111 = NaN,
    max 448) bit patterns -> float32."""
    b = np.asarray(bits, dtype=np.uint8).astype(np.int32)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 0x7
    sub = s * m * 2.0 ** -9
    norm = s * (1.0 + m / 8.0) * np.exp2(e - 7.0)
    out = np.where(e == 0, sub, norm)
    out = np.where((e == 0xF) & (m == 0x7), np.nan, out)
    return out.astype(F32)


_E4M3_FINITE = None


def _e4m3_table():
    global _E4M3_FINITE
    if _E4M3_FINITE is None:
        codes = np.arange(0, 0x7F, dtype=np.uint8)  # non-negative finite codes 0..126
        _E4M3_FINITE = (codes, e4m3_decode(codes).astype(np.float64))
    return _E4M3_FINITE


def e4m3_encode(x) -> np.ndarray:
    """float32 -> fp8 e4m3fn bits, round to nearest (ties to even code),
    saturating to +-448; NaN -> 0x7F (sign kept)."""
    xs = np.asarray(x, dtype=np.float64)
    codes, vals = _e4m3_table()
    mag = np.minimum(np.abs(xs), 448.0)
    idx = np.searchsorted(vals, mag)  # first value >= mag
    idx = np.clip(idx, 1, len(vals) - 1)
    lo, hi = vals[idx - 1], vals[idx]
    take_hi = (mag - lo > hi - mag) | ((mag - lo == hi - mag) & ((codes[idx] & 1) == 0))
    code = np.where(take_hi, codes[idx], codes[idx - 1]).astype(np.uint8)
    code = np.where(mag == 0.0, 0, code).astype(np.uint8)
    sign = np.where(np.signbit(xs), 0x80, 0).astype(np.uint8)
    out = code | sign
    out = np.where(np.isnan(xs), 0x7F | sign, out)
    return out.astype(np.uint8)


def quantize_per_channel(w, axis: int = 0):
    """Per-output-channel fp8 quantization: scale[c] =
    amax over the reduced axis / 448, q = e4m3(w / scale).  For a factor laid
    out (d_in, d_out) the output channels are columns (axis=0 reduced).
    Returns (bits uint8, scale float32)."""
    w = np.asarray(w, dtype=F32)
    amax = np.max(np.abs(w), axis=axis, keepdims=True)
    scale = np.where(amax > 0, amax / F32(448.0), F32(1.0)).astype(F32)
    q = e4m3_encode((w / scale).astype(F32))
    return q, np.squeeze(scale, axis=axis).astype(F32)


def quantize_rows_e4m3(a):
    """Per-row fp8 quantization of an activation (the MI355X build's
    fp8-activation mode; the reference has no fp8 path): scale[m] =
    amax_m / 448 and q = e4m3(a * (448 / amax_m)), the product in float32; a
    zero row gets scale 1.  Returns (bits uint8, scale float32)."""
    a = np.asarray(a, dtype=F32)
    amax = np.max(np.abs(a), axis=1, keepdims=True)
    inv = np.where(amax > 0, F32(448.0) / np.where(amax > 0, amax, F32(1.0)), F32(1.0)).astype(F32)
    q = e4m3_encode((a * inv).astype(F32))
    scale = np.where(amax > 0, amax / F32(448.0), F32(1.0)).astype(F32)
    return q, scale[:, 0]


# ---------------------------------------------------------------------------
# Reference math (kernels/reference.py)
# ---------------------------------------------------------------------------


def low_rank_dim(hidden_size: int, intermediate_size: int, compress_ratio: float) -> int:
    """kernels/reference.py:21-34 -- rank aligned to 128, Python round
    (half to even)."""
    numer = intermediate_size * hidden_size * compress_ratio
    denom = (intermediate_size + hidden_size) * 128
    return round(numer / denom) * 128


def silu(x) -> np.ndarray:
    """kernels/reference.py:37-51 -- x * sigmoid(x) in float32 with the
    sign-split sigmoid, so every exp argument is <= 0."""
    x32 = np.asarray(x, dtype=F32)
    pos = x32 >= 0
    with np.errstate(over="ignore"):
        z = np.exp(np.where(pos, -x32, x32))  # exp(-|x|)
    sig = np.where(pos, F32(1.0) / (F32(1.0) + z), z / (F32(1.0) + z))
    return (x32 * sig).astype(F32)


def _cast(a, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return round_bf16(a)
    if dtype == "float32":
        return np.asarray(a, dtype=F32)
    raise ValueError(f"unsupported dtype {dtype!r}")


def fused_gate_up_ref(x, u_gate, v_gate, u_up, v_up, dtype: str = "float32") -> np.ndarray:
    """kernels/reference.py:54-72 -- silu(X.Ug.Vg) * (X.Uu.Vu), fp32 GEMMs,
    one cast to the activation dtype at the end.  Inputs are float32 arrays
    holding values of ``dtype``."""
    x = np.asarray(x, F32)
    gate = (x @ np.asarray(u_gate, F32)) @ np.asarray(v_gate, F32)
    up = (x @ np.asarray(u_up, F32)) @ np.asarray(v_up, F32)
    return _cast(silu(gate) * up, dtype)


def fused_xuv_ref(x, u, v, dtype: str = "float32") -> np.ndarray:
    """kernels/reference.py:75-82 -- (X.U).V in fp32, cast at the end."""
    return _cast((np.asarray(x, F32) @ np.asarray(u, F32)) @ np.asarray(v, F32), dtype)


def svd_mlp_ref(x, u_gate, v_gate, u_up, v_up, u_down, v_down, dtype: str = "float32") -> np.ndarray:
    """kernels/reference.py:85-93 -- xuv(gate_up(x)); h carries the
    activation dtype between the two halves."""
    h = fused_gate_up_ref(x, u_gate, v_gate, u_up, v_up, dtype)
    return fused_xuv_ref(h, u_down, v_down, dtype)


def svd_mlp_fp8_act_ref(x, u_gate, v_gate, u_up, v_up, u_down, v_down) -> np.ndarray:
    """svd_mlp_ref in bf16 with the down projection's input h quantized to
    e4m3 per token row (quantize_rows_e4m3), the MI355X fp8-activation mode
    of the h . Ud stage: xuv(dequant(quant(round(gate_up(x))))).  The
    reference's math (kernels/reference.py:85-93) with that one extra
    rounding."""
    h = fused_gate_up_ref(x, u_gate, v_gate, u_up, v_up, "bfloat16")
    q, s = quantize_rows_e4m3(h)
    hq = (e4m3_decode(q).astype(F32) * s[:, None]).astype(F32)
    return fused_xuv_ref(hq, u_down, v_down, "bfloat16")


def dense_mlp_ref(x, w_gate, w_up, w_down, dtype: str = "float32") -> np.ndarray:
    """kernels/reference.py:96-106 -- uncompressed SwiGLU."""
    x = np.asarray(x, F32)
    gate = x @ np.asarray(w_gate, F32)
    up = x @ np.asarray(w_up, F32)
    return _cast((silu(gate) * up) @ np.asarray(w_down, F32), dtype)


def unfused_reference(x, u_up, v_up, u_gate, v_gate, u_down, v_down) -> np.ndarray:
    """test_speedup.py:681-687 -- the fp32 golden arm (up-first argument
    order, no rounding of h)."""
    f = [np.asarray(a, F32) for a in (x, u_up, v_up, u_gate, v_gate, u_down, v_down)]
    x, u_up, v_up, u_gate, v_gate, u_down, v_down = f
    gate = (x @ u_gate) @ v_gate
    up = (x @ u_up) @ v_up
    return ((silu(gate) * up) @ u_down) @ v_down


def rmsnorm_ref(x, weight, eps: float = 1e-5, dtype: str = "float32") -> np.ndarray:
    """models/modeling_llama.py:257-262 (LlamaRMSNorm.forward): fp32
    x * rsqrt(mean(x^2) + eps), times the fp32 gain, cast to the input dtype."""
    x32 = np.asarray(x, F32)
    var = np.mean(np.square(x32), axis=-1, keepdims=True, dtype=F32)
    h = x32 * (F32(1.0) / np.sqrt(var + F32(eps)))
    return _cast(np.asarray(weight, F32) * h, dtype)


def mlp_block_ref(x, gain, factors, eps: float = 1e-5, dtype: str = "float32") -> np.ndarray:
    """One layer of the MLP stack: x + svd_mlp(rmsnorm(x)), the MLP half of
    bench/e2e_block.py:268-278 with LlamaRMSNorm; the residual add rounds to
    the activation dtype (bf16 + bf16 -> bf16)."""
    h = rmsnorm_ref(x, gain, eps, dtype)
    y = svd_mlp_ref(h, *factors, dtype=dtype)
    return _cast(np.asarray(x, F32) + y, dtype)


def mlp_block_f64(x, gain, factors, eps: float = 1e-5) -> np.ndarray:
    """The same block in float64 with no rounding anywhere (the exact math
    that every bf16 implementation approximates): x + svd_mlp(rmsnorm(x)),
    rmsnorm and silu as above.  Used to measure how far a bf16 chain drifts
    from the exact one over many layers."""
    x = np.asarray(x, np.float64)
    ug, vg, uu, vu, ud, vd = (np.asarray(a, np.float64) for a in factors)
    hn = np.asarray(gain, np.float64) * (x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps))
    g = (hn @ ug) @ vg
    u = (hn @ uu) @ vu
    h = g / (1.0 + np.exp(-g)) * u
    return x + (h @ ud) @ vd


# ---------------------------------------------------------------------------
# Metrics and accounting
# ---------------------------------------------------------------------------


def relative_l2(actual, expected) -> float:
    """bench/checkpoint_speedup.py:20-31 / test_speedup.py:854 --
    ||a - b||_2 / max(||b||_2, 1e-12), rejecting non-finite values."""
    return errors(actual, expected)["relative_l2"]


def errors(actual, expected) -> dict:
    """bench/checkpoint_speedup.py:20-31: relative L2, max abs error and the
    reference RMS; raises FloatingPointError on NaN/Inf and ValueError on a
    shape mismatch."""
    a = np.asarray(actual, dtype=F32)
    e = np.asarray(expected, dtype=F32)
    if a.shape != e.shape:
        raise ValueError(f"output shape mismatch: {a.shape} != {e.shape}")
    if not np.isfinite(a).all() or not np.isfinite(e).all():
        raise FloatingPointError("MLP output or reference contains NaN/Inf")
    diff = (a - e).astype(np.float64)
    ref = e.astype(np.float64)
    return {
        "relative_l2": float(np.linalg.norm(diff) / max(np.linalg.norm(ref), 1e-12)),
        "max_abs_error": float(np.max(np.abs(diff))) if diff.size else 0.0,
        "reference_rms": float(np.sqrt(np.mean(ref ** 2))) if ref.size else 0.0,
    }


def factor_bytes(d: int, ff: int, r_gu: int, r_d: int | None = None, w_bytes: int = 2) -> int:
    """Bytes of one layer's six factors: 2*r_gu*(d+ff) + r_d*(ff+d), times
    the element size (tests_test_profiler.py.before:20: 297 MiB at 8B r=2816)."""
    r_d = r_gu if r_d is None else r_d
    return (2 * r_gu * (d + ff) + r_d * (ff + d)) * w_bytes


def layer_flops(T: int, d: int, ff: int, r_gu: int, r_d: int | None = None) -> int:
    """Algorithmic FLOPs of one layer, 2*T*sum_b r_b*(d_in + d_out)."""
    r_d = r_gu if r_d is None else r_d
    return 2 * T * (2 * r_gu * (d + ff) + r_d * (ff + d))
