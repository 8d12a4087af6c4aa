"""The MLP stack: N layers of x <- x + svd_mlp(RMSNorm(x)), the MLP half of
the model loop of bench/e2e_block.py:264-278 / 343-355 with LlamaRMSNorm
(models/modeling_llama.py:245-262), on libsvdmlp.

Non-uniform compression draws each layer's gate, up and down ranks
independently from ``RANK_CHOICES`` with a seeded generator.  Each branch
runs at its own rank (the library's two-rank entry points; the reference's
TPU launcher takes one rank for gate and up, test_speedup.py:532-533, so it
would zero-pad the smaller branch).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import ops

RANK_CHOICES = (2048, 2304, 2560, 2816, 3072)


@dataclass
class StackLayer:
    gain: torch.Tensor   # (d,) float32 RMSNorm gain
    factors: tuple       # (ug, vg, uu, vu, ud, vd) at the drawn ranks
    ranks: tuple         # drawn (r_gate, r_up, r_down)


def draw_ranks(n_layers: int, seed: int, choices=RANK_CHOICES) -> list[tuple[int, int, int]]:
    """Per-layer (gate, up, down) ranks, drawn independently and seeded."""
    rng = np.random.default_rng(seed)
    picks = rng.choice(np.asarray(choices), size=(n_layers, 3))
    return [tuple(int(v) for v in row) for row in picks]


def make_stack(n_layers: int, d: int, ff: int, *, seed: int, device, dtype=torch.bfloat16,
               choices=RANK_CHOICES) -> list[StackLayer]:
    """Synthetic layers: U ~ N(0, 1/d_in), V ~ N(0, 1/r) (test_speedup.py:803-808
    recipe, drawn on the device), gains ~ U(0.9, 1.1)."""
    ranks = draw_ranks(n_layers, seed, choices)
    layers = []
    for i, (rg, ru, rd) in enumerate(ranks):
        g = torch.Generator(device=device)
        g.manual_seed(seed * 1000 + i)

        def rnd(rows, cols):
            return (torch.randn(rows, cols, generator=g, device=device, dtype=torch.float32)
                    / math.sqrt(rows)).to(dtype)

        ug, vg = rnd(d, rg), rnd(rg, ff)
        uu, vu = rnd(d, ru), rnd(ru, ff)
        ud, vd = rnd(ff, rd), rnd(rd, d)
        gain = torch.rand(d, generator=g, device=device, dtype=torch.float32) * 0.2 + 0.9
        layers.append(StackLayer(gain, (ug, vg, uu, vu, ud, vd), (rg, ru, rd)))
    return layers


def stack_flops(T: int, d: int, ff: int, layers) -> float:
    """Algorithmic FLOPs of the stack, 2*T*sum_b r_b*(d_in + d_out) with the
    drawn ranks."""
    return float(sum(2 * T * ((rg + ru) * (d + ff) + rd * (ff + d)) for rg, ru, rd in
                     (l.ranks for l in layers)))


def stack_workspace(x: torch.Tensor, layers) -> torch.Tensor:
    """One workspace for every layer of the stack (sized for the largest rank)."""
    ff = layers[0].factors[1].shape[1]
    r = max(max(l.ranks) for l in layers)
    return ops.svd_mlp_workspace(x, r=r, ff=ff)


def run_stack(x: torch.Tensor, layers, *, eps: float = 1e-5, workspace: torch.Tensor | None = None,
              buffers: tuple | None = None) -> torch.Tensor:
    """x after every layer's block, ping-ponging between two (T, d) buffers."""
    if workspace is None:
        workspace = stack_workspace(x, layers)
    if buffers is None:
        buffers = (torch.empty_like(x), torch.empty_like(x))
    cur = x
    for i, layer in enumerate(layers):
        out = buffers[i % 2]
        ops.svd_mlp_block(cur, layer.gain, *layer.factors, eps=eps, workspace=workspace, out=out)
        cur = out
    return cur
