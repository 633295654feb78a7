"""FP8 checkpoint ingestion: safetensors tensors -> loaded FP8 linear layers.

One call takes a linear layer from a checkpoint on disk to a layer ready for
``quant_method.apply``, with the reference's pieces in the reference's order:

1. ``quantization_config`` (from ``config.json``, or given) -> recipe and method
   (``FP8Config.from_config`` / ``get_quant_method``; an ignored layer gives ``None``);
2. the checkpoint's scale tensor names checked against the recipe
   (``validate_scale_key_set``, reference ``model_loader/fp8.py:366-379``);
3. ``create_weights`` with one output partition per packed projection (q/k/v,
   gate/up), whose ``F8_E4M3`` weights stream from disk straight into their row
   slice of the packed weight in HBM;
4. each projection's scale normalised (an inverse checkpoint scale inverted exactly
   once, ``normalize_scale``, :387) and loaded through the scale parameter's
   ``weight_loader`` with the projection as ``shard_id``, which narrows it to the
   projection's rows or 128-row blocks (reference ``layers/linear/fp8.py:139-180``);
   a static ``input_scale`` loads the same way, each projection's in turn, as the
   reference's loader does. ``scale_direction`` applies to the weight scales only (the
   reference defines it but has no call site; activation ``input_scale`` tensors are
   dequant scales in the checkpoint formats that ship them);
5. ``process_weights_after_loading``.

Checkpoint names follow the usual layout: ``<parent>.<projection>.weight`` with
``weight_scale`` / ``weight_scale_inv`` / ``input_scale`` beside it.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from typing import Any

import torch
from torch import nn

from ayaka.exceptions import CheckpointCorruptError, UnsupportedWeightFormatError
from ayaka.model_loader.fp8 import FP8_SCALE_KEY_SUFFIXES, normalize_scale, parse_fp8_config, validate_scale_key_set
from ayaka.model_loader.reader import CheckpointReader
from ayaka.types import DType

__all__ = ["PackedLayout", "PackedProjection", "load_fp8_linear"]


@dataclass(frozen=True, slots=True)
class PackedProjection:
    """One logical projection inside a packed output dimension."""

    name: str
    local_offset: int
    local_size: int


class PackedLayout:
    """Row layout of a packed linear layer (``layer.layout``), looked up by
    projection name or index, as the FP8 scale loader expects."""

    def __init__(self, parts: Sequence[PackedProjection]) -> None:
        self.parts = tuple(parts)

    @property
    def names(self) -> tuple[str, ...]:
        return tuple(p.name for p in self.parts)

    def __getitem__(self, shard_id: object) -> PackedProjection:
        if isinstance(shard_id, int):
            return self.parts[shard_id]
        for part in self.parts:
            if part.name == shard_id:
                return part
        raise KeyError(f"no projection {shard_id!r}; have {self.names}")


def _quantization_config(reader: CheckpointReader, config: Mapping[str, Any] | None) -> Mapping[str, Any]:
    if config is not None:
        return config
    qc = reader.config.get("quantization_config")
    if not isinstance(qc, Mapping):
        raise CheckpointCorruptError(f"{reader.path}: config.json has no quantization_config object")
    return qc


def load_fp8_linear(
    reader: CheckpointReader,
    target: str,
    projections: Sequence[str] | None = None,
    *,
    config: Mapping[str, Any] | None = None,
    device: torch.device | str | None = None,
) -> nn.Module | None:
    """Build and load the FP8 linear layer ``target`` from ``reader``'s checkpoint.

    Args:
        reader: the checkpoint.
        target: the layer's module path, e.g. ``model.layers.0.self_attn.qkv_proj``.
        projections: checkpoint projections packed into it, e.g.
            ``("q_proj", "k_proj", "v_proj")``, siblings of ``target``; ``None``
            loads ``target`` itself.
        config: the ``quantization_config``; default ``config.json``'s.
        device: where the weights live (the GPU for ``apply``).

    Returns:
        The loaded layer (``layer.quant_method`` set), or ``None`` when the config
        excludes ``target`` from FP8 (it is then loaded as a plain linear elsewhere).
    """
    from ayaka.layers.linear.fp8 import FP8Config

    qc = _quantization_config(reader, config)
    parsed = parse_fp8_config(qc)
    method = FP8Config.from_config(qc).get_quant_method(None, target)
    if method is None:
        return None
    parent = target.rsplit(".", 1)[0] if "." in target else ""
    prefixes = [target] if not projections else [f"{parent}.{p}" if parent else p for p in projections]
    names = list(projections) if projections else [target]

    # weights: e4m3 [rows, K] per projection
    sizes, k = [], None
    for prefix in prefixes:
        entry = reader.entry(f"{prefix}.weight")
        if entry.dtype is not DType.FP8_E4M3:
            raise UnsupportedWeightFormatError(f"{prefix}.weight: FP8 layers need F8_E4M3 weights, got {entry.dtype.label}")
        if len(entry.shape) != 2:
            raise CheckpointCorruptError(f"{prefix}.weight: FP8 weights are [out, in], got shape {entry.shape}")
        if k is not None and entry.shape[1] != k:
            raise CheckpointCorruptError(f"{prefix}.weight: input size {entry.shape[1]} differs from {k} of its siblings")
        k = entry.shape[1]
        sizes.append(entry.shape[0])
        candidates = (f"{prefix}.{suffix}" for suffixes in FP8_SCALE_KEY_SUFFIXES.values() for suffix in suffixes)
        validate_scale_key_set([key for key in candidates if key in reader], parsed.recipe.recipe)

    layer = nn.Module()
    method.create_weights(layer, output_partition_sizes=sizes, input_size_per_partition=int(k), device=device)
    packed = projections is not None and len(prefixes) > 1
    if packed:
        offsets = [sum(sizes[:i]) for i in range(len(sizes))]
        layer.layout = PackedLayout([PackedProjection(n, o, s) for n, o, s in zip(names, offsets, sizes)])

    direction = parsed.recipe.scale_direction
    scale_name = method.weight_scale_name
    row = 0
    for name, prefix, size in zip(names, prefixes, sizes):
        reader.read_into(f"{prefix}.weight", layer.weight.data[row:row + size])
        row += size
        shard = name if packed else None
        scale = normalize_scale(reader.read(f"{prefix}.{scale_name}", device), direction=direction)
        param = getattr(layer, scale_name)
        param.weight_loader(layer, param, scale, shard)
        if getattr(layer, "input_scale", None) is not None:
            key = f"{prefix}.input_scale"
            if key not in reader:
                raise CheckpointCorruptError(f"{key}: a static-activation checkpoint must ship input_scale")
            value = reader.read(key, device)  # activation scales are dequant scales in every producer
            if value.numel() == 1:
                value = value.reshape(())  # a [1] scalar fits the layer's 0-d input_scale
            layer.input_scale.weight_loader(layer, layer.input_scale, value, shard)
    method.process_weights_after_loading(layer)
    layer.quant_method = method
    return layer
