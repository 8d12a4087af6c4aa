"""SVD-MLP factors from a sharded Hugging Face safetensors checkpoint
(models/hf_svd.py:1-196).

The checkpoint stores each branch as two PyTorch ``Linear`` weights in
``[out, in]`` order, and names the first projection ``v_proj`` and the second
``u_proj``: ``gate_v_proj.weight`` is ``(r, d)`` and ``gate_u_proj.weight``
``(ff, r)``.  The kernels take natural matmul operands, ``U (d_in, r)`` and
``V (r, d_out)``, so each stored tensor is transposed and the v/u names swap:
``Ug = gate_v_proj.T``, ``Vg = gate_u_proj.T`` and so on.  Factors come back
gate-first, ``(Ug, Vg, Uu, Vu, Ud, Vd)``, ready for ``svdmlp.svd_mlp``.

Two device layouts are offered:

* ``"natural"`` (default): each factor is copied to the device and transposed
  there once into a contiguous ``(in, out)`` tensor, the layout every fast path
  (large-tile prefill, persistent decode layers) reads;
* ``"linear"``: each factor is copied as stored and returned as a transposed
  view; the library reads the ``(out, in)`` storage in place (no transpose
  pass, no second copy), on its Linear-layout kernels.

Validation and its exceptions follow the reference: missing config or index
-> ``FileNotFoundError``; index without ``weight_map`` -> ``ValueError``;
missing factor keys -> ``KeyError``; missing shards -> ``FileNotFoundError``;
factor shapes or dtypes that disagree with the config -> ``ValueError`` /
``TypeError``.
"""

from __future__ import annotations

import json
from contextlib import ExitStack
from pathlib import Path
from typing import Sequence

FACTOR_SUFFIXES = (
    "gate_v_proj.weight",
    "gate_u_proj.weight",
    "up_v_proj.weight",
    "up_u_proj.weight",
    "down_v_proj.weight",
    "down_u_proj.weight",
)

_SAFETENSORS_DTYPES = ("BF16", "F32", "F16")


def checkpoint_metadata(model_path: str | Path) -> tuple[dict, dict]:
    """``config.json`` and ``model.safetensors.index.json`` of a checkpoint
    directory, minimally validated (models/hf_svd.py:23-37)."""
    model_path = Path(model_path)
    config_path = model_path / "config.json"
    index_path = model_path / "model.safetensors.index.json"
    if not config_path.is_file():
        raise FileNotFoundError(f"missing checkpoint config: {config_path}")
    if not index_path.is_file():
        raise FileNotFoundError(f"missing safetensors index: {index_path}")
    config = json.loads(config_path.read_text(encoding="utf-8"))
    index = json.loads(index_path.read_text(encoding="utf-8"))
    if "weight_map" not in index:
        raise ValueError(f"safetensors index has no weight_map: {index_path}")
    return config, index


def factor_keys(layer_index: int) -> tuple[str, ...]:
    """The six tensor names of one layer's MLP (models/hf_svd.py:40-44)."""
    if layer_index < 0:
        raise ValueError(f"layer index must be non-negative, got {layer_index}")
    prefix = f"model.layers.{layer_index}.mlp."
    return tuple(prefix + suffix for suffix in FACTOR_SUFFIXES)


def validate_factor_shapes(factors: Sequence, *, hidden_size: int, intermediate_size: int) -> int:
    """Check the natural-layout (transposed) shapes and a common dtype; return
    the rank (models/hf_svd.py:47-73).  ``factors`` may be tensors or any
    objects with ``shape`` and ``dtype``."""
    if len(factors) != 6:
        raise ValueError(f"expected six MLP factors, got {len(factors)}")
    rank = int(factors[0].shape[1])
    expected = (
        (hidden_size, rank),
        (rank, intermediate_size),
        (hidden_size, rank),
        (rank, intermediate_size),
        (intermediate_size, rank),
        (rank, hidden_size),
    )
    actual = tuple(tuple(int(v) for v in f.shape) for f in factors)
    if actual != expected:
        raise ValueError(f"invalid transposed MLP factor shapes; expected {expected}, got {actual}")
    dtypes = {str(f.dtype) for f in factors}
    if len(dtypes) != 1:
        raise TypeError(f"MLP factor dtypes differ: {sorted(dtypes)}")
    return rank


def _selected(config: dict, layer_indices) -> tuple[int, ...]:
    num_layers = int(config["num_hidden_layers"])
    selected = tuple(range(num_layers)) if layer_indices is None else tuple(int(i) for i in layer_indices)
    if not selected or len(set(selected)) != len(selected):
        raise ValueError("select at least one layer, without duplicates")
    if min(selected) < 0 or max(selected) >= num_layers:
        raise ValueError(f"layer indices must be in [0, {num_layers})")
    return selected


def _required_shards(model_path: Path, weight_map: dict, keys) -> list[str]:
    missing = [key for key in keys if key not in weight_map]
    if missing:
        raise KeyError(f"checkpoint is missing MLP factors: {missing}")
    names = sorted({weight_map[key] for key in keys})
    absent = [name for name in names if not (model_path / name).is_file()]
    if absent:
        raise FileNotFoundError("checkpoint shards required by the selected layers are missing: " + ", ".join(absent))
    return names


class _Shape:
    def __init__(self, shape, dtype):
        self.shape, self.dtype = shape, dtype


def inspect_mlp_checkpoint(model_path: str | Path, layer_indices: Sequence[int] | None = None) -> dict:
    """Validate shard headers without loading payloads (models/hf_svd.py:76-129):
    per selected layer its rank, dtype, factor bytes and tensor locations."""
    from safetensors import safe_open

    model_path = Path(model_path)
    config, index = checkpoint_metadata(model_path)
    if config.get("hidden_act", "silu") != "silu" or config.get("mlp_bias", False):
        raise ValueError("the fused kernel requires bias-free SwiGLU MLPs")
    hidden, intermediate = int(config["hidden_size"]), int(config["intermediate_size"])
    selected = _selected(config, layer_indices)
    weight_map = index["weight_map"]
    keys = tuple(key for layer in selected for key in factor_keys(layer))
    names = _required_shards(model_path, weight_map, keys)
    itemsize = {"BF16": 2, "F16": 2, "F32": 4}
    layers = []
    with ExitStack() as stack:
        shards = {name: stack.enter_context(safe_open(str(model_path / name), framework="pt")) for name in names}
        for layer in selected:
            descriptors, info = [], []
            for key in factor_keys(layer):
                view = shards[weight_map[key]].get_slice(key)
                shape, dtype = tuple(view.get_shape()), view.get_dtype()
                if len(shape) != 2 or dtype not in _SAFETENSORS_DTYPES or min(shape) <= 0:
                    raise ValueError(f"unsupported MLP tensor {key}: {shape}, {dtype}")
                descriptors.append(_Shape(shape[::-1], dtype))
                info.append({"key": key, "shape": list(shape), "dtype": dtype, "shard": weight_map[key]})
            rank = validate_factor_shapes(descriptors, hidden_size=hidden, intermediate_size=intermediate)
            nbytes = sum(d.shape[0] * d.shape[1] * itemsize[d.dtype] for d in descriptors)
            layers.append({"layer": layer, "rank": rank, "dtype": info[0]["dtype"], "factor_bytes": nbytes,
                           "tensors": info})
    return {"model_path": str(model_path.resolve()), "num_hidden_layers": int(config["num_hidden_layers"]),
            "hidden_size": hidden, "intermediate_size": intermediate, "selected_layers": list(selected),
            "shards": names, "layers": layers}


def load_mlp_factors(model_path: str | Path, layer_indices: Sequence[int], *, device="cuda",
                     layout: str = "natural", dtype=None) -> tuple[tuple, ...]:
    """Selected layers' factors on ``device``, gate-first ``(Ug, Vg, Uu, Vu, Ud,
    Vd)`` per layer (models/hf_svd.py:132-196).  ``layout`` is ``"natural"``
    (contiguous ``(in, out)``, transposed on the device), ``"padded"`` (natural,
    with the V factors' rows 64 elements longer in memory: the row pitch the
    decode kernels stream fastest, see ``ops.pad_rows``) or ``"linear"``
    (transposed views of the stored ``(out, in)`` tensors).  ``dtype``
    optionally converts (e.g. ``torch.bfloat16``) on the device."""
    import torch
    from safetensors import safe_open

    from .ops import pad_rows

    if layout not in ("natural", "padded", "linear"):
        raise ValueError(f"layout must be 'natural', 'padded' or 'linear', got {layout!r}")
    model_path = Path(model_path)
    config, index = checkpoint_metadata(model_path)
    layer_indices = tuple(layer_indices)
    if not layer_indices:
        raise ValueError("at least one layer must be selected")
    weight_map = index["weight_map"]
    keys = tuple(key for layer in layer_indices for key in factor_keys(layer))
    names = _required_shards(model_path, weight_map, keys)
    dev = torch.device(device)
    layers = []
    with ExitStack() as stack:
        shards = {name: stack.enter_context(safe_open(str(model_path / name), framework="pt")) for name in names}
        for layer in layer_indices:
            factors = []
            for i, key in enumerate(factor_keys(layer)):
                stored = shards[weight_map[key]].get_tensor(key).to(dev)  # (out, in)
                if dtype is not None:
                    stored = stored.to(dtype)
                if layout == "linear":
                    factors.append(stored.t())
                elif layout == "padded" and i % 2:   # Vg, Vu, Vd
                    factors.append(pad_rows(stored.t()))
                else:
                    factors.append(stored.t().contiguous())
                del stored
            validate_factor_shapes(factors, hidden_size=int(config["hidden_size"]),
                                   intermediate_size=int(config["intermediate_size"]))
            layers.append(tuple(factors))
    return tuple(layers)


def save_mlp_checkpoint(model_path: str | Path, layers: Sequence[Sequence], *, hidden_size: int,
                        intermediate_size: int, shard_layers: int = 1, extra_config: dict | None = None) -> Path:
    """Write gate-first natural-layout factors as a sharded checkpoint in the
    format ``load_mlp_factors`` reads (stored transposed, v/u names swapped):
    for synthetic test checkpoints and for exporting factors."""
    import torch
    from safetensors.torch import save_file

    model_path = Path(model_path)
    model_path.mkdir(parents=True, exist_ok=True)
    weight_map = {}
    for s0 in range(0, len(layers), shard_layers):
        name = f"model-{s0 // shard_layers + 1:05d}.safetensors"
        tensors = {}
        for layer in range(s0, min(len(layers), s0 + shard_layers)):
            validate_factor_shapes(layers[layer], hidden_size=hidden_size, intermediate_size=intermediate_size)
            for key, f in zip(factor_keys(layer), layers[layer]):
                tensors[key] = torch.as_tensor(f).detach().to("cpu").t().contiguous()
                weight_map[key] = name
        save_file(tensors, str(model_path / name))
    config = {"hidden_size": hidden_size, "intermediate_size": intermediate_size, "num_hidden_layers": len(layers),
              "hidden_act": "silu", "mlp_bias": False}
    config.update(extra_config or {})
    (model_path / "config.json").write_text(json.dumps(config), encoding="utf-8")
    (model_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}), encoding="utf-8")
    return model_path
