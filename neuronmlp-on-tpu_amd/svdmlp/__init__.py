"""svdmlp -- the SVD-compressed LLaMA MLP hot path on AMD Instinct MI355X.

Host package over libsvdmlp.so (hand-written HIP kernels for gfx950):

* :mod:`svdmlp.ops`     -- kernels/reference.py operator API
  (``fused_gate_up``, ``fused_xuv``, ``svd_mlp``) on ROCm tensors.
* :mod:`svdmlp.compat`  -- the test_speedup.py launcher API
  (``fused_mlp_up_T``, ``fused_three_mm_XTUV``, ``svd_mlp_with_fused_kernel``,
  ``nki_mm``, ``get_fused_*_params`` ...).
* :mod:`svdmlp.config`  -- model shapes, ranks and block parameters.
* :mod:`svdmlp.inputs`  -- seeded synthetic inputs of the benchmark configs.
* :mod:`svdmlp.fp8`     -- fp8 e4m3fn per-channel factor quantization.
* :mod:`svdmlp.stack`   -- the N-layer MLP stack (RMSNorm, MLP, residual).
* :mod:`svdmlp.checkpoint` -- SVD factors from sharded safetensors checkpoints
  (models/hf_svd.py), and :mod:`svdmlp.checkpoint_speedup`, the per-layer
  real-checkpoint runner (bench/checkpoint_speedup.py).
* :mod:`svdmlp.pallas_ops` -- the pallas_ops operator names and keywords of
  the reference's benches (``svd_mlp``, ``fused_gate_up``, ``xuv_matmul``,
  ``dense_mlp``, ``contracted_svd_mlp``).
* :mod:`svdmlp.speedup` -- the three-way fused / dense / unfused benchmark
  (test_speedup.py's synthetic branch); :mod:`svdmlp.e2e_block` -- the
  N-layer transformer prefill with attention (bench/e2e_block.py).
"""

from ._lib import SvdMlpError, load, version, workspace_bytes  # noqa: F401
from .ops import (  # noqa: F401
    QuantizedFactor,
    clear_workspace_cache,
    fused_gate_up,
    fused_xuv,
    low_rank_dim,
    silu,
    svd_mlp,
    svd_mlp_block,
    svd_mlp_workspace,
    workspace_status,
)

__version__ = "1.0.0"
