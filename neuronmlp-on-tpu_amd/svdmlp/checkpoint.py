"""SVD-MLP factors stored in a sharded Hugging Face safetensors checkpoint.

The on-disk format is the reference's (models/hf_svd.py:13-20, 130-196) and
is kept exactly, so its checkpoints load unchanged:

* ``config.json`` gives ``hidden_size``, ``intermediate_size`` and
  ``num_hidden_layers``; ``model.safetensors.index.json`` maps every tensor
  name to its shard file (``weight_map``);
* each MLP branch (gate, up, down) is two PyTorch ``Linear`` weights stored
  ``(out, in)``: ``model.layers.{i}.mlp.{branch}_v_proj.weight`` is the first
  projection, ``(r, d_in)``, and ``{branch}_u_proj.weight`` the second,
  ``(d_out, r)``.

The kernels take natural matmul operands, ``U (d_in, r)`` and ``V (r,
d_out)``: the first projection is U transposed, the second V transposed
(hence the v -> U, u -> V naming swap).  Everything below works on a table of
the six factor slots, each knowing its branch, its projection and how its
shapes follow from (rank, hidden, intermediate); layers are returned
gate-first, ``(Ug, Vg, Uu, Vu, Ud, Vd)``, ready for ``svdmlp.svd_mlp``.

Device layouts: ``"natural"`` (contiguous ``(in, out)``, one transpose on the
device), ``"padded"`` (natural, V rows 64 elements longer in memory, the pitch
the decode kernels stream fastest) and ``"linear"`` (transposed views of the
stored tensors: the library reads the ``(out, in)`` storage in place).

Errors keep the reference's exception types and message wording, so callers
that match on them behave the same: missing config / index / shards
(FileNotFoundError), an index without ``weight_map`` or a bad layer selection
(ValueError), absent tensor names (KeyError), inconsistent shapes
(ValueError) or dtypes (TypeError).
"""

from __future__ import annotations

import json
from contextlib import ExitStack
from dataclasses import dataclass
from pathlib import Path
from typing import Iterable, Sequence

CONFIG_FILE = "config.json"
INDEX_FILE = "model.safetensors.index.json"
_ITEMSIZE = {"BF16": 2, "F16": 2, "F32": 4}


@dataclass(frozen=True)
class FactorSlot:
    """One of a layer's six factors: ``branch`` gate / up / down, ``proj``
    "v" (first projection; natural operand U) or "u" (second; natural V)."""

    branch: str
    proj: str

    def key(self, layer: int) -> str:
        return f"model.layers.{layer}.mlp.{self.branch}_{self.proj}_proj.weight"

    def natural_shape(self, rank: int, hidden: int, intermediate: int) -> tuple[int, int]:
        d_in, d_out = (intermediate, hidden) if self.branch == "down" else (hidden, intermediate)
        return (d_in, rank) if self.proj == "v" else (rank, d_out)


SLOTS = tuple(FactorSlot(b, p) for b in ("gate", "up", "down") for p in ("v", "u"))
FACTOR_SUFFIXES = tuple(s.key(0).split(".mlp.", 1)[1] for s in SLOTS)


def factor_keys(layer_index: int) -> tuple[str, ...]:
    """Tensor names of one layer's factors, in slot (gate-first) order."""
    if layer_index < 0:
        raise ValueError(f"layer index must be non-negative, got {layer_index}")
    return tuple(s.key(layer_index) for s in SLOTS)


def validate_factor_shapes(factors: Sequence, *, hidden_size: int, intermediate_size: int) -> int:
    """Rank of six natural-layout factors (anything with ``shape`` and
    ``dtype``) after checking every shape against the slot table and that one
    dtype is shared (the contract of models/hf_svd.py:47-73)."""
    if len(factors) != len(SLOTS):
        raise ValueError(f"expected six MLP factors, got {len(factors)}")
    shapes = tuple(tuple(int(n) for n in f.shape) for f in factors)
    rank = shapes[0][1] if len(shapes[0]) == 2 else -1
    want = tuple(s.natural_shape(rank, hidden_size, intermediate_size) for s in SLOTS)
    if shapes != want:
        raise ValueError(f"invalid transposed MLP factor shapes; expected {want}, got {shapes}")
    kinds = sorted({str(f.dtype) for f in factors})
    if len(kinds) > 1:
        raise TypeError(f"MLP factor dtypes differ: {kinds}")
    return rank


class SvdCheckpoint:
    """A checkpoint directory, parsed once: its MLP geometry and tensor map."""

    def __init__(self, root: str | Path):
        self.root = Path(root)
        cfg_path, idx_path = self.root / CONFIG_FILE, self.root / INDEX_FILE
        for path, what in ((cfg_path, "checkpoint config"), (idx_path, "safetensors index")):
            if not path.is_file():
                raise FileNotFoundError(f"missing {what}: {path}")
        self.config = json.loads(cfg_path.read_text(encoding="utf-8"))
        self.index = json.loads(idx_path.read_text(encoding="utf-8"))
        if "weight_map" not in self.index:
            raise ValueError(f"safetensors index has no weight_map: {idx_path}")
        self.weight_map: dict = self.index["weight_map"]

    @property
    def hidden(self) -> int:
        return int(self.config["hidden_size"])

    @property
    def intermediate(self) -> int:
        return int(self.config["intermediate_size"])

    @property
    def num_layers(self) -> int:
        return int(self.config["num_hidden_layers"])

    def selection(self, layers: Iterable[int] | None) -> tuple[int, ...]:
        """Validated layer list (``None``: every layer)."""
        sel = tuple(range(self.num_layers)) if layers is None else tuple(int(i) for i in layers)
        if not sel or len(set(sel)) != len(sel):
            raise ValueError("select at least one layer, without duplicates")
        if not all(0 <= i < self.num_layers for i in sel):
            raise ValueError(f"layer indices must be in [0, {self.num_layers})")
        return sel

    def shards_for(self, layers: Sequence[int]) -> list[str]:
        """Shard files holding the layers' factors, after checking that every
        tensor name is mapped and every shard exists."""
        keys = [k for i in layers for k in factor_keys(i)]
        unmapped = [k for k in keys if k not in self.weight_map]
        if unmapped:
            raise KeyError(f"checkpoint is missing MLP factors: {unmapped}")
        shards = sorted({self.weight_map[k] for k in keys})
        gone = [s for s in shards if not (self.root / s).is_file()]
        if gone:
            raise FileNotFoundError("checkpoint shards required by the selected layers are missing: " + ", ".join(gone))
        return shards

    def _handles(self, stack: ExitStack, shards: Sequence[str]) -> dict:
        from safetensors import safe_open

        return {s: stack.enter_context(safe_open(str(self.root / s), framework="pt")) for s in shards}

    def headers(self, layers: Sequence[int]) -> list[dict]:
        """Per layer: rank, dtype, factor bytes and where each tensor lives,
        from the shard headers alone (no payload is read)."""
        rows = []
        with ExitStack() as stack:
            handles = self._handles(stack, self.shards_for(layers))
            for i in layers:
                tensors, natural = [], []
                for slot in SLOTS:
                    key = slot.key(i)
                    view = handles[self.weight_map[key]].get_slice(key)
                    stored, kind = tuple(view.get_shape()), view.get_dtype()
                    if len(stored) != 2 or kind not in _ITEMSIZE or min(stored) <= 0:
                        raise ValueError(f"unsupported MLP tensor {key}: {stored}, {kind}")
                    natural.append(_Header((stored[1], stored[0]), kind))
                    tensors.append({"key": key, "shape": list(stored), "dtype": kind, "shard": self.weight_map[key]})
                rank = validate_factor_shapes(natural, hidden_size=self.hidden, intermediate_size=self.intermediate)
                size = sum(h.shape[0] * h.shape[1] * _ITEMSIZE[h.dtype] for h in natural)
                rows.append({"layer": i, "rank": rank, "dtype": tensors[0]["dtype"], "factor_bytes": size,
                             "tensors": tensors})
        return rows

    def tensors(self, layers: Sequence[int], *, device, layout: str, dtype=None) -> tuple[tuple, ...]:
        """The layers' factors on ``device`` in the requested layout."""
        import torch

        from .ops import pad_rows

        place = {
            "natural": lambda w, slot: w.t().contiguous(),
            "padded": lambda w, slot: pad_rows(w.t()) if slot.proj == "u" else w.t().contiguous(),
            "linear": lambda w, slot: w.t(),
        }
        if layout not in place:
            raise ValueError(f"layout must be 'natural', 'padded' or 'linear', got {layout!r}")
        dev = torch.device(device)
        out = []
        with ExitStack() as stack:
            handles = self._handles(stack, self.shards_for(layers))
            for i in layers:
                layer = []
                for slot in SLOTS:
                    key = slot.key(i)
                    w = handles[self.weight_map[key]].get_tensor(key).to(dev)   # stored (out, in)
                    if dtype is not None:
                        w = w.to(dtype)
                    layer.append(place[layout](w, slot))
                validate_factor_shapes(layer, hidden_size=self.hidden, intermediate_size=self.intermediate)
                out.append(tuple(layer))
        return tuple(out)


@dataclass(frozen=True)
class _Header:
    shape: tuple
    dtype: str


def checkpoint_metadata(model_path: str | Path) -> tuple[dict, dict]:
    """``(config, index)`` of a checkpoint directory (models/hf_svd.py:23-37)."""
    ck = SvdCheckpoint(model_path)
    return ck.config, ck.index


def inspect_mlp_checkpoint(model_path: str | Path, layer_indices: Sequence[int] | None = None) -> dict:
    """Header-only validation of the selected layers (models/hf_svd.py:76-129):
    geometry, shards and, per layer, rank, dtype, factor bytes and tensors."""
    ck = SvdCheckpoint(model_path)
    if ck.config.get("hidden_act", "silu") != "silu" or ck.config.get("mlp_bias", False):
        raise ValueError("the fused kernel requires bias-free SwiGLU MLPs")
    layers = ck.selection(layer_indices)
    return {"model_path": str(ck.root.resolve()), "num_hidden_layers": ck.num_layers, "hidden_size": ck.hidden,
            "intermediate_size": ck.intermediate, "selected_layers": list(layers), "shards": ck.shards_for(layers),
            "layers": ck.headers(layers)}


def load_mlp_factors(model_path: str | Path, layer_indices: Sequence[int], *, device="cuda",
                     layout: str = "natural", dtype=None) -> tuple[tuple, ...]:
    """Selected layers' factors on ``device``, gate-first ``(Ug, Vg, Uu, Vu, Ud,
    Vd)`` per layer (models/hf_svd.py:132-196); ``layout`` is "natural",
    "padded" or "linear" (module docstring); ``dtype`` optionally converts
    on the device."""
    ck = SvdCheckpoint(model_path)
    layers = tuple(layer_indices)
    if not layers:
        raise ValueError("at least one layer must be selected")
    return ck.tensors(layers, device=device, layout=layout, dtype=dtype)


def save_mlp_checkpoint(model_path: str | Path, layers: Sequence[Sequence], *, hidden_size: int,
                        intermediate_size: int, shard_layers: int = 1, extra_config: dict | None = None) -> Path:
    """Write gate-first natural-layout factors in the format above (stored
    transposed, v/u roles as the reference names them), ``shard_layers``
    layers per shard: for synthetic test checkpoints and exported factors."""
    import torch
    from safetensors.torch import save_file

    root = Path(model_path)
    root.mkdir(parents=True, exist_ok=True)
    weight_map = {}
    for first in range(0, len(layers), shard_layers):
        shard = f"model-{first // shard_layers + 1:05d}.safetensors"
        payload = {}
        for i in range(first, min(len(layers), first + shard_layers)):
            validate_factor_shapes(layers[i], hidden_size=hidden_size, intermediate_size=intermediate_size)
            for slot, f in zip(SLOTS, layers[i]):
                payload[slot.key(i)] = torch.as_tensor(f).detach().to("cpu").t().contiguous()
                weight_map[slot.key(i)] = shard
        save_file(payload, str(root / shard))
    config = {"hidden_size": hidden_size, "intermediate_size": intermediate_size, "num_hidden_layers": len(layers),
              "hidden_act": "silu", "mlp_bias": False, **(extra_config or {})}
    (root / CONFIG_FILE).write_text(json.dumps(config), encoding="utf-8")
    (root / INDEX_FILE).write_text(json.dumps({"weight_map": weight_map}), encoding="utf-8")
    return root
