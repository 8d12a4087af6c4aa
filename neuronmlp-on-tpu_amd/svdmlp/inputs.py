"""Seeded synthetic inputs for the SVD-MLP configurations.

The recipe follows test_speedup.py:803-835: ``numpy.random.default_rng(seed)``,
factors drawn in the order (u_up, v_up, u_gate, v_gate, u_down, v_down) as
``normal(size=(rows, cols)) / sqrt(rows)`` (so U ~ N(0, 1/d_in) and
V ~ N(0, 1/r)), then X ~ N(0, 1) per sequence length.  bf16 inputs are the
RNE rounding of these float32 draws (torch's cast).

Configurations (BASELINE.json ``configs``):
  tiny     T=128,  d=1024, ff=3584,  r=256,  float32
  8b       T=1024, d=4096, ff=14336, r=2816, bfloat16 (prefill)
  8b-dec   T in {1, 8, 32, 64}, same layer
  stack    32 layers, T=4096, per-branch ranks from {2048, 2304, ..., 3072}
  70b-fp8  T=2048, d=8192, ff=28672, r=5632, fp8 e4m3 factors
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch


@dataclass(frozen=True)
class LayerShape:
    d: int
    ff: int
    r: int  # gate/up rank
    r_down: int | None = None

    @property
    def rd(self) -> int:
        return self.r if self.r_down is None else self.r_down


SHAPES = {
    "tiny": LayerShape(1024, 3584, 256),
    "8b": LayerShape(4096, 14336, 2816),
    "70b": LayerShape(8192, 28672, 5632),
}


def random_matrix(rng: np.random.Generator, rows: int, cols: int) -> np.ndarray:
    """test_speedup.py:804-805: N(0,1) / sqrt(rows), float32."""
    return (rng.normal(size=(rows, cols)).astype(np.float32) / np.float32(math.sqrt(rows))).astype(np.float32)


def make_factors(shape: LayerShape, seed: int = 0, rng: np.random.Generator | None = None):
    """Six float32 factors in the reference's draw order, returned in the
    gate-first order of kernels/reference.py: (ug, vg, uu, vu, ud, vd)."""
    rng = np.random.default_rng(seed) if rng is None else rng
    d, ff, r, rd = shape.d, shape.ff, shape.r, shape.rd
    uu = random_matrix(rng, d, r)
    vu = random_matrix(rng, r, ff)
    ug = random_matrix(rng, d, r)
    vg = random_matrix(rng, r, ff)
    ud = random_matrix(rng, ff, rd)
    vd = random_matrix(rng, rd, d)
    return ug, vg, uu, vu, ud, vd


def make_x(rng: np.random.Generator, T: int, d: int) -> np.ndarray:
    """test_speedup.py:835: X ~ N(0, 1), float32."""
    return rng.normal(size=(T, d)).astype(np.float32)


def make_layer(shape: LayerShape, T: int, seed: int = 0):
    """(x, factors) drawn from one generator in the reference's order."""
    rng = np.random.default_rng(seed)
    factors = make_factors(shape, rng=rng)
    return make_x(rng, T, shape.d), factors


def to_torch(a: np.ndarray, dtype: torch.dtype, device="cuda") -> torch.Tensor:
    """float32 numpy -> torch tensor of ``dtype`` (RNE for bfloat16)."""
    t = torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32))
    return t.to(dtype).to(device)


def as_float32(a: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """The float32 values a tensor of ``dtype`` built from ``a`` holds."""
    if dtype == torch.float32:
        return np.asarray(a, np.float32)
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dtype).float().numpy()


def make_outlier_layer(shape: LayerShape, T: int, seed: int = 0, channels=((3, 1e3), (17, 3e3), (250, 1e2)),
                       col_sigma: float = 1.0):
    """A heavy-tailed stand-in for a real checkpoint's layer (no checkpoint is
    available offline; the reference's real-layer check,
    results/kernel_optimizations_1_4_20260916/real_layer0_S512_check.json:2-3,
    reports a max |error| of 3.8e6 next to a relative error of 3.1e-3, i.e.
    outputs in the millions).  x ~ N(0, 1) with a few hidden channels
    (columns) scaled by 1e2..3e3, the massive-activation pattern of LLaMA
    hidden states; every factor's columns multiplied by log-normal scales
    exp(col_sigma * N(0, 1) - col_sigma^2) (heavy-tailed column norms, mean
    square 1).  Float32, factors gate-first as make_factors."""
    rng = np.random.default_rng(seed)
    factors = list(make_factors(shape, rng=rng))
    for i, f in enumerate(factors):
        s = np.exp(col_sigma * rng.normal(size=f.shape[1]) - col_sigma * col_sigma).astype(np.float32)
        factors[i] = (f * s[None, :]).astype(np.float32)
    x = make_x(rng, T, shape.d)
    for c, scale in channels:
        if c < shape.d:
            x[:, c] *= np.float32(scale)
    return x, tuple(factors)
