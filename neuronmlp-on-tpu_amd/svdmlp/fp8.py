"""fp8 e4m3fn factor quantization (LLaMA3-70B configuration).

Each factor (d_in, d_out) gets one fp32 scale per output column,
``scale = amax(|w[:, c]|) / 448``, and ``q = e4m3fn(w / scale)`` with round
to nearest even.  The kernels widen ``q`` to bf16 exactly and apply the scale
to the fp32 accumulator, so ``x . w`` is computed as ``(x . q) * scale``.
"""

from __future__ import annotations

import torch

from .ops import QuantizedFactor

E4M3_MAX = 448.0


def quantize_per_channel(w: torch.Tensor) -> QuantizedFactor:
    """Quantize a (d_in, d_out) factor with per-output-column scales."""
    if w.dim() != 2:
        raise ValueError(f"expected a 2D factor, got {tuple(w.shape)}")
    w32 = w.float()
    amax = w32.abs().amax(dim=0)
    scale = torch.where(amax > 0, amax / E4M3_MAX, torch.ones_like(amax))
    # Clamp before the cast: torch's e4m3fn conversion does not saturate.
    q = (w32 / scale).clamp_(-E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
    return QuantizedFactor(q.contiguous(), scale.to(torch.float32).contiguous())
