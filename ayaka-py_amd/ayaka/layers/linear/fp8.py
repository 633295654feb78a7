"""Dense FP8 linear quantization methods and checkpoint scale loading.

Drop-in for the reference's ``python/ayaka/layers/linear/fp8.py`` (``:67-664``). The
public surface is the reference's: class names, constructor arguments, parameter
names / shapes / dtypes / sentinels (NaN, or 0xFF for UE8M0), the packed-projection
scale loader and every error message. The structure is this module's own:

* each method *declares* its scale parameters as ``_ScaleSlot`` records (name, shape
  rule, dtype, sentinel, how a loaded value is checked); one generic routine creates
  them and one validates them after loading, in declaration order;
* the scale loader first resolves *where* a checkpoint tensor goes (the whole
  parameter, one projection's entry, or one projection's rows / 128-row blocks) and
  then writes it with one broadcasting rule;
* ``apply`` hands the activation to the recipe's entry point in
  ``ayaka.kernel.hip`` (gfx950 HIP kernels).
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from dataclasses import dataclass
from typing import Any, ClassVar, Literal, cast

import torch
from torch import nn

from ayaka.kernel.hip.gemm.fp8_linear import fp8_block_linear, fp8_pertensor_linear, fp8_rowwise_linear
from ayaka.layers.linear.methods import LinearMethodBase
from ayaka.layers.linear.weight_loading import WeightLoadError, set_weight_attrs
from ayaka.layers.quantization.base import (
    BaseQuantization,
    QuantizationCapabilities,
    QuantizationTarget,
    QuantizeMethodBase,
)
from ayaka.types import compute_torch_dtypes
from ayaka.utils.import_utils import CapabilityError
from ayaka.utils.math_utils import div_ceil
from ayaka.weights.spec import FP8Recipe

FP8 = torch.float8_e4m3fn
BLOCK128 = 128
UE8M0_UNSET = 0xFF  # the UE8M0 NaN code doubles as the "not loaded" sentinel

ActivationScheme = Literal["dynamic", "static", "weight_only"]
_ACTIVATION_SCHEMES: tuple[str, ...] = ("dynamic", "static", "weight_only")

#: layer construction attributes that stay on the layer, not on the weight parameter
_LAYER_ONLY_ATTRS = frozenset(
    {"output_partition_sizes", "input_size_per_partition", "input_size", "output_size", "params_dtype", "device"}
)

#: non-persistent buffer holding an fp32 copy of a bf16 block-128 weight-scale table
_BLOCK_SCALE_F32 = "_fp8_block_scale_f32"

_SCALE_DTYPE_NAMES = {torch.uint8: "e8m0", torch.float32: "float32", torch.bfloat16: "bfloat16"}


# ------------------------------------------------------------------ scale checks
def _not_loaded(name: str) -> ValueError:
    return ValueError(f"{name} not loaded from the checkpoint")


def _check_float_scale(name: str, tensor: torch.Tensor) -> None:
    """A float scale must be loaded (no NaN sentinel left), finite and positive."""
    if tensor.is_meta:
        raise _not_loaded(name)
    values = tensor.detach().float()
    finite = torch.isfinite(values)
    if not bool(finite.all().item()):
        if bool(torch.isnan(values).any().item()):
            raise _not_loaded(name)
        raise ValueError(f"{name} must be finite; found an infinite checkpoint value")
    if not bool((values > 0).all().item()):
        raise ValueError(f"{name} must be positive; found a zero or negative checkpoint value")


def _check_code_scale(name: str, tensor: torch.Tensor) -> None:
    """A UE8M0 scale is loaded once no 0xFF code (sentinel and NaN code) is left."""
    if tensor.is_meta or bool(tensor.eq(UE8M0_UNSET).any().item()):
        raise _not_loaded(name)


@dataclass(frozen=True)
class _ScaleSlot:
    """One checkpoint scale parameter of a method."""

    name: str
    shape: tuple[int, ...]
    dtype: torch.dtype
    check: Callable[[str, torch.Tensor], None]

    @property
    def sentinel(self) -> float | int:
        return UE8M0_UNSET if self.dtype is torch.uint8 else float("nan")


# ------------------------------------------------------------------ scale loader
def _layout_of(layer: nn.Module) -> Any:
    return getattr(layer, "layout", None)


def _projection_names(layer: nn.Module) -> tuple[str, ...]:
    """Logical projection names of a packed layer (``layout.names``, else the names of
    ``layout.parts``); empty for an unpacked layer."""
    layout = _layout_of(layer)
    if layout is None:
        return ()
    declared = getattr(layout, "names", None)
    if declared:
        return tuple(map(str, declared))
    return tuple(part if isinstance(part, str) else str(part.name) for part in getattr(layout, "parts", ()))


def _parts_are_plain_names(layer: nn.Module) -> bool:
    layout = _layout_of(layer)
    parts = () if layout is None else getattr(layout, "parts", ())
    return len(parts) > 0 and all(isinstance(part, str) for part in parts)


def _projection_span(layer: nn.Module, shard_id: object) -> tuple[int, int, int]:
    """``(position, first_row, end_row)`` of the projection ``shard_id`` names; a plain-name
    projection spans the single row at its position."""
    layout = _layout_of(layer)
    if layout is None:
        raise WeightLoadError("scale loading requires the layer's projection layout")
    names = _projection_names(layer)
    entry = layout[shard_id]  # type: ignore[index]
    label = entry if isinstance(entry, str) else str(entry.name)
    if label not in names:
        raise WeightLoadError(f"unknown projection {label!r}; expected one of {names}")
    position = names.index(label)
    if isinstance(entry, str):
        return position, position, position + 1
    first = int(entry.local_offset)
    return position, first, first + int(entry.local_size)


def _scale_destination(layer: nn.Module, data: torch.Tensor, loaded: torch.Tensor, shard_id: object) -> torch.Tensor | None:
    """The part of ``data`` one checkpoint scale is written to, or ``None`` when the
    tensor replaces ``data`` outright (a projection-tagged tensor of the full shape)."""
    if shard_id is None:
        return data
    if tuple(loaded.shape) == tuple(data.shape):
        return None
    names = _projection_names(layer)
    if not names:
        return data
    position, first, end = _projection_span(layer, shard_id)
    if _parts_are_plain_names(layer) and data.ndim >= 1 and data.shape[0] == len(names):
        return data[position]
    rows_per_scale = int(getattr(layer, "fp8_scale_block_y", 1) or 1)
    if rows_per_scale > 1:  # 128-row block scales: the blocks the projection's rows touch
        first, end = first // rows_per_scale, div_ceil(end, rows_per_scale)
    if data.ndim < 1:
        raise WeightLoadError("packed scale storage must have at least one dimension")
    return data[first:end]


def _write_scale(destination: torch.Tensor, loaded: torch.Tensor) -> None:
    """Copy ``loaded`` into ``destination``: same shape or same element count copies,
    a single value broadcasts, anything else does not fit."""
    if loaded.numel() == destination.numel():
        destination.copy_(loaded if loaded.shape == destination.shape else loaded.reshape(destination.shape))
    elif loaded.numel() == 1:
        destination.fill_(loaded.reshape(()))
    else:
        raise WeightLoadError(
            f"scale: checkpoint shape {tuple(loaded.shape)} does not fit destination shape {tuple(destination.shape)}"
        )


def _scale_loader(layer: nn.Module, parameter: torch.Tensor, loaded_weight: torch.Tensor, shard_id: object = None) -> None:
    """Load one checkpoint scale into a (possibly packed) scale parameter.

    A scalar broadcasts over its destination; a fused QKV / gate-up layer loads one
    scale per logical projection (``shard_id``) into that projection's entry, rows, or
    128-row scale blocks (``layer.fp8_scale_block_y``).
    """
    if not isinstance(parameter, torch.Tensor):
        raise TypeError("parameter must be a torch.Tensor")
    if loaded_weight.is_meta:
        raise WeightLoadError("scale loading requires a materialized checkpoint tensor")
    if getattr(layer, _BLOCK_SCALE_F32, None) is not None:
        setattr(layer, _BLOCK_SCALE_F32, None)  # stale once the scale parameter is written
    destination = _scale_destination(layer, parameter.data, loaded_weight, shard_id)
    if destination is None:
        parameter.data.copy_(loaded_weight)
    else:
        _write_scale(destination, loaded_weight)


# ------------------------------------------------------------------ methods
class _FP8LinearMethodBase(LinearMethodBase):
    """FP8 weight storage plus the declared scale slots of a recipe."""

    weight_scale_name: ClassVar[str] = "weight_scale"

    def __init__(self, *, activation_bits: int) -> None:
        self._activation_bits = activation_bits

    # -- declarations each recipe provides
    def _scale_slots(self, total_output: int, input_size: int) -> list[_ScaleSlot]:
        raise NotImplementedError

    def _rows_per_scale(self, input_size: int) -> int:
        return 1

    def _run(self, layer: nn.Module, x: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
        raise NotImplementedError

    # -- shared machinery
    def get_capabilities(self) -> QuantizationCapabilities:
        return QuantizationCapabilities(
            supported_devices=frozenset({"cuda"}),  # gfx950 HIP kernels only; no CPU path
            supported_act_dtypes=compute_torch_dtypes(),
            supported_targets=frozenset({QuantizationTarget.LINEAR}),
            storage_format="fp8_e4m3",
            weight_bits=8,
            activation_bits=self._activation_bits,
            supports_dynamic_activation=True,
            supports_static_activation=True,
        )

    def create_weights(self, layer: nn.Module, *weight_args: Any, **attrs: Any) -> None:
        if weight_args:
            raise TypeError("FP8 linear weight dimensions must be passed by name")
        partitions = attrs.get("output_partition_sizes")
        input_size = attrs.get("input_size_per_partition")
        if not partitions:
            raise ValueError("output_partition_sizes is required for FP8 linear weights")
        if not isinstance(input_size, int) or input_size < 1:
            raise ValueError("input_size_per_partition must be a positive integer")
        device = attrs.get("device")
        total_output = sum(map(int, partitions))
        weight = nn.Parameter(torch.empty(total_output, input_size, dtype=FP8, device=device), requires_grad=False)
        layer.register_parameter("weight", weight)
        set_weight_attrs(weight, {key: value for key, value in attrs.items() if key not in _LAYER_ONLY_ATTRS})
        layer.fp8_total_output = total_output
        layer.fp8_input_size = input_size
        layer.fp8_scale_block_y = 1
        self.create_scale_parameters(layer, total_output, input_size, device)

    def create_scale_parameters(self, layer: nn.Module, total_output: int, input_size: int, device) -> None:
        for slot in self._scale_slots(total_output, input_size):
            param = nn.Parameter(torch.full(slot.shape, slot.sentinel, dtype=slot.dtype, device=device),
                                 requires_grad=False)
            layer.register_parameter(slot.name, param)
            set_weight_attrs(param, {"weight_loader": _scale_loader})
        layer.fp8_scale_block_y = self._rows_per_scale(input_size)

    def process_weights_after_loading(self, layer: nn.Module) -> None:
        for slot in self._scale_slots(layer.fp8_total_output, layer.fp8_input_size):
            slot.check(slot.name, getattr(layer, slot.name))

    def apply(self, layer: nn.Module, *args: Any, **kwargs: Any) -> torch.Tensor:
        bias = args[1] if len(args) > 1 else kwargs.get("bias")
        return self._run(layer, args[0], cast("torch.Tensor | None", bias))


class FP8PerTensorLinearMethod(_FP8LinearMethodBase):
    """Per-tensor / per-output-row FP8 with static, dynamic or weight-only activation.

    ``"static"`` runs W8A8 with the checkpoint's ``input_scale`` at ``M > 1``;
    ``"dynamic"`` quantizes per token at ``M > 1``; ``"weight_only"`` never quantizes
    the activation. ``M == 1`` always runs the weight-only GEMV.
    """

    def __init__(self, activation_scheme: ActivationScheme = "dynamic") -> None:
        scheme = str(activation_scheme)
        if scheme not in _ACTIVATION_SCHEMES:
            raise ValueError(f"activation_scheme must be one of {_ACTIVATION_SCHEMES}")
        super().__init__(activation_bits=16 if scheme == "weight_only" else 8)
        self.activation_scheme: ActivationScheme = cast(ActivationScheme, scheme)

    def _scale_slots(self, total_output, input_size):
        slots = [_ScaleSlot("weight_scale", (total_output,), torch.float32, _check_float_scale)]
        if self.activation_scheme == "static":
            slots.append(_ScaleSlot("input_scale", (), torch.float32, _check_float_scale))
        return slots

    def create_scale_parameters(self, layer, total_output, input_size, device) -> None:
        super().create_scale_parameters(layer, total_output, input_size, device)
        if self.activation_scheme != "static":
            layer.register_parameter("input_scale", None)

    def process_weights_after_loading(self, layer: nn.Module) -> None:
        super().process_weights_after_loading(layer)
        scale = layer.weight_scale
        # A piecewise-constant [N] scale lets the static GEMM take it as a scalar.
        layer._fp8_uniform_scale = bool(scale.eq(scale[0]).all().item())

    def _run(self, layer, x, bias):
        if self.activation_scheme == "dynamic":
            return fp8_rowwise_linear(x, layer.weight, layer.weight_scale, bias)
        if self.activation_scheme == "weight_only":
            return fp8_pertensor_linear(x, layer.weight, layer.weight_scale, bias)
        return fp8_pertensor_linear(x, layer.weight, layer.weight_scale, bias, input_scale=layer.input_scale,
                                    uniform_scale=bool(getattr(layer, "_fp8_uniform_scale", False)))


class FP8RowwiseLinearMethod(_FP8LinearMethodBase):
    """Dynamic per-token activation quant with per-output-row weight scales."""

    def __init__(self) -> None:
        super().__init__(activation_bits=8)

    def _scale_slots(self, total_output, input_size):
        return [_ScaleSlot("weight_scale", (total_output,), torch.float32, _check_float_scale)]

    def _run(self, layer, x, bias):
        return fp8_rowwise_linear(x, layer.weight, layer.weight_scale, bias)


class FP8BlockLinearMethod(_FP8LinearMethodBase):
    """DeepSeek-V3-style 128x128 block scales with dynamic per-token-group activations."""

    weight_scale_name = "weight_scale_inv"

    def __init__(self, scale_dtype: torch.dtype = torch.bfloat16) -> None:
        if scale_dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("scale_dtype must be bfloat16 or float32")
        super().__init__(activation_bits=8)
        self.scale_dtype = scale_dtype

    def _scale_slots(self, total_output, input_size):
        shape = (div_ceil(total_output, BLOCK128), div_ceil(input_size, BLOCK128))
        return [_ScaleSlot("weight_scale_inv", shape, self.scale_dtype, _check_float_scale)]

    def _rows_per_scale(self, input_size):
        return BLOCK128

    def process_weights_after_loading(self, layer: nn.Module) -> None:
        super().process_weights_after_loading(layer)
        # The W8A8 GEMM's decode-batch kernel (M <= 64) reads fp32 block scales. A bf16
        # table widens to fp32 exactly, so a widened copy, made once here, gives the same
        # products; the parameter itself keeps the checkpoint's dtype. The scale loader
        # drops the copy whenever it writes the parameter again.
        scale = layer.weight_scale_inv
        layer.register_buffer(_BLOCK_SCALE_F32, scale.detach().float() if scale.dtype != torch.float32 else None,
                              persistent=False)

    def _run(self, layer, x, bias):
        scale = layer.weight_scale_inv
        widened = getattr(layer, _BLOCK_SCALE_F32, None)
        if widened is not None and x.numel() > x.shape[-1]:  # M > 1: the W8A8 GEMM
            scale = widened
        return fp8_block_linear(x, layer.weight, scale, bias)


class FP8W8A16LinearMethod(_FP8LinearMethodBase):
    """Weight-only e4m3 with fp32 / bf16 / UE8M0 scales, per-channel or blocked.

    ``M == 1`` runs the decode GEMV, ``M > 1`` the W8A16 GEMM; the activation is
    never quantized.
    """

    def __init__(self, scale_dtype: torch.dtype = torch.float32, weight_block: tuple[int, int] | None = None) -> None:
        if scale_dtype not in _SCALE_DTYPE_NAMES:
            raise ValueError("scale_dtype must be float32, bfloat16, or uint8 (UE8M0)")
        if weight_block is not None and min(weight_block) < 1:
            raise ValueError("weight_block sizes must be positive")
        super().__init__(activation_bits=16)
        self.scale_dtype = scale_dtype
        self.weight_block = weight_block

    def _scale_geometry(self, input_size: int) -> tuple[int, int]:
        """(rows, columns) of weight covered by one scale: per-channel without a block."""
        return (1, input_size) if self.weight_block is None else self.weight_block

    def _scale_slots(self, total_output, input_size):
        rows, cols = self._scale_geometry(input_size)
        check = _check_code_scale if self.scale_dtype is torch.uint8 else _check_float_scale
        return [_ScaleSlot("weight_scale", (div_ceil(total_output, rows), div_ceil(input_size, cols)),
                           self.scale_dtype, check)]

    def _rows_per_scale(self, input_size):
        return self._scale_geometry(input_size)[0]

    def create_scale_parameters(self, layer, total_output, input_size, device) -> None:
        super().create_scale_parameters(layer, total_output, input_size, device)
        layer.fp8_weight_block = self._scale_geometry(input_size)

    def _run(self, layer, x, bias):
        from ayaka.kernel.hip.gemm.fp8_gemv import fp8_weight_only_gemv
        from ayaka.kernel.hip.gemm.fp8_w8a16_gemm import fp8_weight_only_gemm

        k = int(x.shape[-1])
        rows, cols = self._scale_geometry(k)
        geometry = dict(scale_row_stride=div_ceil(k, cols), block_size_y=rows, block_size_x=cols,
                        scale_dtype=_SCALE_DTYPE_NAMES[self.scale_dtype])
        # One token (any lead shape) is a GEMV and returns [N], as the reference's method.
        if x.numel() == k:
            out = fp8_weight_only_gemv(x.reshape(k), layer.weight, layer.weight_scale, **geometry)
        else:
            out = fp8_weight_only_gemm(x, layer.weight, layer.weight_scale, **geometry)
        return out if bias is None else out + bias


class FP8Mxfp8LinearMethod(_FP8LinearMethodBase):
    """MXFP8: e4m3 activations and weights with UE8M0 scales per 32-wide K group."""

    MX_GROUP = 32

    def __init__(self) -> None:
        super().__init__(activation_bits=8)

    def _scale_slots(self, total_output, input_size):
        if input_size % self.MX_GROUP:
            raise ValueError("MXFP8 requires the weight K to be divisible by 32")
        return [_ScaleSlot("weight_scale", (total_output, input_size // self.MX_GROUP), torch.uint8, _check_code_scale)]

    def _run(self, layer, x, bias):
        from ayaka.kernel.hip.gemm.fp8_mxfp8_gemm import mxfp8_scaled_mm
        from ayaka.kernel.hip.quant.fp8_quant import per_token_group_quant_mxfp8

        k = int(x.shape[-1])
        if k % self.MX_GROUP:
            raise ValueError("MXFP8 requires the activation K to be divisible by 32")
        rows = x.reshape(-1, k)
        rows = rows if rows.is_contiguous() else rows.contiguous()
        q, codes = per_token_group_quant_mxfp8(rows, self.MX_GROUP)
        n = int(layer.weight.shape[0])
        out = torch.empty((rows.shape[0], n), dtype=x.dtype, device=x.device)
        mxfp8_scaled_mm(q, codes, layer.weight, layer.weight_scale, bias, out=out)
        return out.reshape(*x.shape[:-1], n)


# ------------------------------------------------------------------ config
_METHOD_BUILDERS: dict[FP8Recipe, Callable[[torch.dtype, Any], QuantizeMethodBase]] = {
    FP8Recipe.W8A8_STATIC_PER_TENSOR: lambda sdt, blk: FP8PerTensorLinearMethod(activation_scheme="static"),
    FP8Recipe.W8A8_DYNAMIC_PER_TENSOR: lambda sdt, blk: FP8PerTensorLinearMethod(activation_scheme="dynamic"),
    FP8Recipe.W8A8_ROWWISE: lambda sdt, blk: FP8RowwiseLinearMethod(),
    FP8Recipe.W8A8_BLOCK128: lambda sdt, blk: FP8BlockLinearMethod(scale_dtype=sdt),
    FP8Recipe.W8A16: lambda sdt, blk: FP8W8A16LinearMethod(scale_dtype=sdt, weight_block=blk),
    FP8Recipe.MXFP8: lambda sdt, blk: FP8Mxfp8LinearMethod(),
}


def _method_for(recipe: FP8Recipe, scale_dtype: torch.dtype, weight_block) -> QuantizeMethodBase:
    builder = _METHOD_BUILDERS.get(recipe)
    if builder is None:
        raise CapabilityError(
            "quantization.fp8_recipe",
            detail=f"recipe {recipe.value!r} has no dense linear method",
            remedy="use the KV-cache quantization owner for cache recipes",
        )
    return builder(scale_dtype, weight_block)


def method_from_recipe(parsed: Any) -> QuantizeMethodBase:
    """Dense FP8 method of a parsed checkpoint recipe (``ParsedFP8Config``)."""
    return _method_for(parsed.recipe.recipe, parsed.scale_dtype, parsed.recipe.weight_block)


class FP8Config(BaseQuantization):
    """Select a dense FP8 linear method from a validated recipe descriptor; every
    ``get_quant_method`` call returns a fresh method."""

    def __init__(
        self,
        recipe_name: str,
        *,
        scale_dtype: torch.dtype = torch.bfloat16,
        weight_block: tuple[int, int] | None = None,
        ignored_layers: tuple[str, ...] = (),
        method_factory: Callable[[], QuantizeMethodBase] | None = None,
    ) -> None:
        self.recipe_name = str(recipe_name)
        self.scale_dtype = scale_dtype
        self.weight_block = weight_block
        self.ignored_layers = tuple(ignored_layers)
        self._method_factory = method_factory

    @classmethod
    def get_name(cls) -> str:
        return "fp8"

    @classmethod
    def from_config(cls, config: Mapping[str, Any]) -> FP8Config:
        from ayaka.model_loader.fp8 import parse_fp8_config

        parsed = parse_fp8_config(config)
        return cls(parsed.recipe.recipe.value, scale_dtype=parsed.scale_dtype, weight_block=parsed.recipe.weight_block,
                   ignored_layers=parsed.ignored_layers, method_factory=lambda: method_from_recipe(parsed))

    def _make_method(self) -> QuantizeMethodBase:
        if self._method_factory is not None:
            return self._method_factory()
        return _method_for(FP8Recipe(self.recipe_name), self.scale_dtype, self.weight_block)

    def get_capabilities(self) -> QuantizationCapabilities:
        return self._make_method().get_capabilities()

    def _ignores(self, prefix: str) -> bool:
        return any(prefix == name or prefix.startswith(name + ".") for name in self.ignored_layers)

    def get_quant_method(self, layer: nn.Module, prefix: str) -> QuantizeMethodBase | None:
        del layer
        return None if self._ignores(prefix) else self._make_method()


__all__ = [
    "BLOCK128",
    "FP8BlockLinearMethod",
    "FP8Config",
    "FP8Mxfp8LinearMethod",
    "FP8PerTensorLinearMethod",
    "FP8RowwiseLinearMethod",
    "FP8W8A16LinearMethod",
    "_scale_loader",
    "method_from_recipe",
]
