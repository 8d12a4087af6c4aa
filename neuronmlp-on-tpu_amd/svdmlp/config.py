"""Model shapes, ranks and block parameters.

The reference imports these names from ``svdflash_tpu.kernels.config``
(bench/speedup.py:20-31, models/modeling_llama.py:62-73), a module absent from
its snapshot; fields follow their use at models/modeling_llama.py:367-375 and
bench/speedup.py:123-133.
"""

from __future__ import annotations

from typing import NamedTuple

from .ops import low_rank_dim


class ModelShape(NamedTuple):
    name: str
    hidden_size: int
    intermediate_size: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    rank_at_080: int


def _shape(name, h, i, layers, heads, kv):
    return ModelShape(name, h, i, layers, heads, kv, low_rank_dim(h, i, 0.8))


MODELS = {
    "llama-3.2-3b": _shape("llama-3.2-3b", 3072, 8192, 28, 24, 8),
    "llama-3.1-8b": _shape("llama-3.1-8b", 4096, 14336, 32, 32, 8),
    "qwen3-8b": _shape("qwen3-8b", 4096, 12288, 36, 32, 8),
    "llama-3.1-70b": _shape("llama-3.1-70b", 8192, 28672, 80, 64, 8),
}


def rank_for(model: ModelShape, compress_ratio: float) -> int:
    """SVD rank of ``model`` at ``compress_ratio`` (128-aligned)."""
    if not 0.0 < compress_ratio <= 1.0:
        raise ValueError("compress-ratio must be in (0, 1]")
    return low_rank_dim(model.hidden_size, model.intermediate_size, compress_ratio)


class GateUpBlocks(NamedTuple):
    """Gate/Up block sizes of the reference API (rows, hidden, rank, output
    columns), e.g. (128, 1024, 512, 512) at bench/speedup.py:131.  The MI355X
    kernels pick their own LDS tiles; the values are validated and recorded."""

    bs: int
    bh: int
    br: int
    bn: int


# Down (XUV) tile constants of the reference's config module (values from
# results/down_static_analysis_8b.json:17-22), kept so that importers of that
# module (bench/diagnose_down.py:23-26) resolve; the HIP kernels pick their own
# tiles and do not read them.
XUV_ROW_TILE = 128
XUV_INPUT_TILE = 1024
XUV_RANK_TILE = 512
XUV_OUTPUT_TILE = 1024
