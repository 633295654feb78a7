"""Dense FP8 linear quantization methods and checkpoint scale loading.

Drop-in for the reference's ``python/ayaka/layers/linear/fp8.py`` (``:67-664``):
same classes, constructor arguments, parameter names / shapes / dtypes / NaN
(or 0xFF) sentinels, loader hooks and error messages.

* ``create_weights`` allocates the ``[N, K]`` e4m3 weight and the recipe's scale
  parameters, named as checkpoints ship them (``weight_scale``,
  ``weight_scale_inv``, ``input_scale``) and filled with sentinels so a missing
  checkpoint tensor can never act as a scale;
* ``process_weights_after_loading`` rejects unloaded, non-finite, zero and negative
  scales (0xFF for UE8M0) once per layer;
* ``apply`` runs the recipe on the gfx950 HIP operators of ``ayaka.kernel.hip``.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
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

ActivationScheme = Literal["dynamic", "static", "weight_only"]
_ACTIVATION_SCHEMES: tuple[str, ...] = ("dynamic", "static", "weight_only")

#: layer construction attributes that are not copied onto the weight parameter
_WEIGHT_ATTR_EXCLUSIONS = frozenset(
    {"output_partition_sizes", "input_size_per_partition", "input_size", "output_size", "params_dtype", "device"}
)


def _not_loaded(name: str) -> ValueError:
    return ValueError(f"{name} not loaded from the checkpoint")


def _require_loaded_scale(name: str, tensor: torch.Tensor) -> None:
    """Reject a scale that is absent (NaN sentinel), non-finite, or non-positive."""
    if tensor.is_meta:
        raise _not_loaded(name)
    values = tensor.detach().float()
    if bool(torch.isnan(values).any().item()):
        raise _not_loaded(name)
    if not bool(torch.isfinite(values).all().item()):
        raise ValueError(f"{name} must be finite; found an infinite checkpoint value")
    if bool((values <= 0).any().item()):
        raise ValueError(f"{name} must be positive; found a zero or negative checkpoint value")


# ------------------------------------------------------------------ scale loader
def _projection_names(layer: nn.Module) -> tuple[str, ...]:
    layout = getattr(layer, "layout", None)
    if layout is None:
        return ()
    names = getattr(layout, "names", None)
    if names:
        return tuple(str(n) for n in names)
    return tuple(p if isinstance(p, str) else str(p.name) for p in getattr(layout, "parts", ()))


def _parts_are_names(layer: nn.Module) -> bool:
    layout = getattr(layer, "layout", None)
    parts = getattr(layout, "parts", ()) if layout is not None else ()
    return bool(parts) and all(isinstance(p, str) for p in parts)


def _locate_projection(layer: nn.Module, shard_id: object) -> tuple[int, int, int]:
    """``(index, row_start, row_stop)`` of one projection inside the packed output."""
    layout = getattr(layer, "layout", None)
    if layout is None:
        raise WeightLoadError("scale loading requires the layer's projection layout")
    names = _projection_names(layer)
    projection = layout[shard_id]  # type: ignore[index]
    name = projection if isinstance(projection, str) else str(projection.name)
    if name not in names:
        raise WeightLoadError(f"unknown projection {name!r}; expected one of {names}")
    index = names.index(name)
    if isinstance(projection, str):
        return index, index, index + 1
    start = int(projection.local_offset)
    return index, start, start + int(projection.local_size)


def _assign_scale(destination: torch.Tensor, loaded: torch.Tensor, label: str) -> None:
    if tuple(loaded.shape) == tuple(destination.shape):
        destination.copy_(loaded)
    elif loaded.numel() == destination.numel():
        destination.copy_(loaded.reshape(destination.shape))
    elif loaded.numel() == 1:
        destination.fill_(loaded.reshape(()))
    else:
        raise WeightLoadError(
            f"{label}: checkpoint shape {tuple(loaded.shape)} does not fit destination shape {tuple(destination.shape)}"
        )


def _scale_loader(layer: nn.Module, parameter: torch.Tensor, loaded_weight: torch.Tensor, shard_id: object = None) -> None:
    """Load one projection's scale into a (possibly packed) scale parameter.

    A per-tensor checkpoint's scalar broadcasts; a fused QKV / gate-up layer loads
    one scale per logical projection, narrowed to that projection's rows (or its
    128-row blocks for block scales, ``layer.fp8_scale_block_y``).
    """
    if not isinstance(parameter, torch.Tensor):
        raise TypeError("parameter must be a torch.Tensor")
    if loaded_weight.is_meta:
        raise WeightLoadError("scale loading requires a materialized checkpoint tensor")
    data = parameter.data
    if shard_id is None or tuple(loaded_weight.shape) == tuple(data.shape):
        if shard_id is not None:
            data.copy_(loaded_weight)
        else:
            _assign_scale(data, loaded_weight, "scale")
        return
    names = _projection_names(layer)
    if not names:
        _assign_scale(data, loaded_weight, "scale")
        return
    index, start, stop = _locate_projection(layer, shard_id)
    if _parts_are_names(layer) and data.ndim >= 1 and data.shape[0] == len(names):
        destination = data[index]
    else:
        rows_per_scale = int(getattr(layer, "fp8_scale_block_y", 1) or 1)
        if rows_per_scale > 1:
            start, stop = start // rows_per_scale, div_ceil(stop, rows_per_scale)
        if data.ndim < 1:
            raise WeightLoadError("packed scale storage must have at least one dimension")
        destination = data[start:stop]
    _assign_scale(destination, loaded_weight, "scale")


# ------------------------------------------------------------------ methods
class _FP8LinearMethodBase(LinearMethodBase):
    """Shared FP8 storage creation and capability declaration."""

    weight_scale_name: ClassVar[str] = "weight_scale"

    def __init__(self, *, activation_bits: int) -> None:
        self._activation_bits = activation_bits

    def get_capabilities(self) -> QuantizationCapabilities:
        return QuantizationCapabilities(
            supported_devices=frozenset({"cpu", "cuda"}),
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
        output_partition_sizes = attrs.get("output_partition_sizes")
        input_size = attrs.get("input_size_per_partition")
        if not output_partition_sizes:
            raise ValueError("output_partition_sizes is required for FP8 linear weights")
        if not isinstance(input_size, int) or input_size < 1:
            raise ValueError("input_size_per_partition must be a positive integer")
        device = attrs.get("device")
        total_output = sum(int(size) for size in output_partition_sizes)
        weight = nn.Parameter(torch.empty(total_output, input_size, dtype=FP8, device=device), requires_grad=False)
        layer.register_parameter("weight", weight)
        weight_attrs = {k: v for k, v in attrs.items() if k not in _WEIGHT_ATTR_EXCLUSIONS}
        set_weight_attrs(weight, weight_attrs)
        layer.fp8_total_output = total_output
        layer.fp8_input_size = input_size
        layer.fp8_scale_block_y = 1
        self.create_scale_parameters(layer, total_output, input_size, device)

    def create_scale_parameters(self, layer: nn.Module, total_output: int, input_size: int, device) -> None:
        raise NotImplementedError

    def apply(self, layer: nn.Module, *args: Any, **kwargs: Any) -> torch.Tensor:
        raise NotImplementedError

    @staticmethod
    def _bias(args: tuple[Any, ...], kwargs: Mapping[str, Any]) -> torch.Tensor | None:
        return cast("torch.Tensor | None", args[1] if len(args) > 1 else kwargs.get("bias"))

    @staticmethod
    def _scale_param(layer: nn.Module, name: str, shape, dtype: torch.dtype, sentinel, device) -> None:
        param = nn.Parameter(torch.full(shape, sentinel, dtype=dtype, device=device), requires_grad=False)
        layer.register_parameter(name, param)
        set_weight_attrs(param, {"weight_loader": _scale_loader})


class FP8PerTensorLinearMethod(_FP8LinearMethodBase):
    """Per-tensor / per-output-row FP8 with static, dynamic or weight-only activation.

    ``"static"`` runs W8A8 with the checkpoint's ``input_scale`` at ``M > 1``;
    ``"dynamic"`` quantizes per token at ``M > 1``; ``"weight_only"`` never
    quantizes the activation. ``M == 1`` always runs the weight-only GEMV.
    """

    def __init__(self, activation_scheme: ActivationScheme = "dynamic") -> None:
        scheme = str(activation_scheme)
        if scheme not in _ACTIVATION_SCHEMES:
            raise ValueError(f"activation_scheme must be one of {_ACTIVATION_SCHEMES}")
        super().__init__(activation_bits=16 if scheme == "weight_only" else 8)
        self.activation_scheme: ActivationScheme = cast(ActivationScheme, scheme)

    def create_scale_parameters(self, layer, total_output, input_size, device) -> None:
        self._scale_param(layer, "weight_scale", (total_output,), torch.float32, float("nan"), device)
        if self.activation_scheme == "static":
            self._scale_param(layer, "input_scale", (), torch.float32, float("nan"), device)
        else:
            layer.register_parameter("input_scale", None)

    def process_weights_after_loading(self, layer: nn.Module) -> None:
        _require_loaded_scale("weight_scale", layer.weight_scale)
        if self.activation_scheme == "static":
            _require_loaded_scale("input_scale", layer.input_scale)
        scale = layer.weight_scale
        layer._fp8_uniform_scale = bool((scale == scale[0]).all().item())

    def apply(self, layer: nn.Module, *args: Any, **kwargs: Any) -> torch.Tensor:
        x, bias = args[0], self._bias(args, kwargs)
        if self.activation_scheme == "weight_only":
            return fp8_pertensor_linear(x, layer.weight, layer.weight_scale, bias)
        if self.activation_scheme == "static":
            return fp8_pertensor_linear(x, layer.weight, layer.weight_scale, bias, input_scale=layer.input_scale,
                                        uniform_scale=bool(getattr(layer, "_fp8_uniform_scale", False)))
        return fp8_rowwise_linear(x, layer.weight, layer.weight_scale, bias)


class FP8RowwiseLinearMethod(_FP8LinearMethodBase):
    """Dynamic per-token activation quant with per-output-row weight scales."""

    def __init__(self) -> None:
        super().__init__(activation_bits=8)

    def create_scale_parameters(self, layer, total_output, input_size, device) -> None:
        self._scale_param(layer, "weight_scale", (total_output,), torch.float32, float("nan"), device)

    def process_weights_after_loading(self, layer: nn.Module) -> None:
        _require_loaded_scale("weight_scale", layer.weight_scale)

    def apply(self, layer: nn.Module, *args: Any, **kwargs: Any) -> torch.Tensor:
        return fp8_rowwise_linear(args[0], layer.weight, layer.weight_scale, self._bias(args, kwargs))


class FP8BlockLinearMethod(_FP8LinearMethodBase):
    """DeepSeek-V3-style 128x128 block scales with dynamic per-token-group activations."""

    weight_scale_name = "weight_scale_inv"

    def __init__(self, scale_dtype: torch.dtype = torch.bfloat16) -> None:
        if scale_dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("scale_dtype must be bfloat16 or float32")
        super().__init__(activation_bits=8)
        self.scale_dtype = scale_dtype

    def create_scale_parameters(self, layer, total_output, input_size, device) -> None:
        shape = (div_ceil(total_output, BLOCK128), div_ceil(input_size, BLOCK128))
        self._scale_param(layer, "weight_scale_inv", shape, self.scale_dtype, float("nan"), device)
        layer.fp8_scale_block_y = BLOCK128

    def process_weights_after_loading(self, layer: nn.Module) -> None:
        _require_loaded_scale("weight_scale_inv", layer.weight_scale_inv)

    def apply(self, layer: nn.Module, *args: Any, **kwargs: Any) -> torch.Tensor:
        return fp8_block_linear(args[0], layer.weight, layer.weight_scale_inv, self._bias(args, kwargs))


class FP8W8A16LinearMethod(_FP8LinearMethodBase):
    """Weight-only e4m3 with fp32 / bf16 / UE8M0 scales, per-channel or blocked.

    ``M == 1`` runs the decode GEMV, ``M > 1`` the W8A16 GEMM; the activation is
    never quantized.
    """

    def __init__(self, scale_dtype: torch.dtype = torch.float32, weight_block: tuple[int, int] | None = None) -> None:
        if scale_dtype not in (torch.float32, torch.bfloat16, torch.uint8):
            raise ValueError("scale_dtype must be float32, bfloat16, or uint8 (UE8M0)")
        if weight_block is not None:
            by, bx = weight_block
            if by < 1 or bx < 1:
                raise ValueError("weight_block sizes must be positive")
        super().__init__(activation_bits=16)
        self.scale_dtype = scale_dtype
        self.weight_block = weight_block

    def _scale_geometry(self, input_size: int) -> tuple[int, int]:
        return (1, input_size) if self.weight_block is None else self.weight_block

    def create_scale_parameters(self, layer, total_output, input_size, device) -> None:
        by, bx = self._scale_geometry(input_size)
        sentinel: float | int = 0xFF if self.scale_dtype is torch.uint8 else float("nan")
        self._scale_param(layer, "weight_scale", (div_ceil(total_output, by), div_ceil(input_size, bx)),
                          self.scale_dtype, sentinel, device)
        layer.fp8_scale_block_y = by
        layer.fp8_weight_block = (by, bx)

    def process_weights_after_loading(self, layer: nn.Module) -> None:
        scale = layer.weight_scale
        if self.scale_dtype is torch.uint8:
            if scale.is_meta or bool((scale == 0xFF).any().item()):
                raise _not_loaded("weight_scale")
        else:
            _require_loaded_scale("weight_scale", scale)

    def apply(self, layer: nn.Module, *args: Any, **kwargs: Any) -> torch.Tensor:
        from ayaka.kernel.hip.gemm.fp8_gemv import fp8_weight_only_gemv
        from ayaka.kernel.hip.gemm.fp8_w8a16_gemm import fp8_weight_only_gemm

        x = args[0]
        inner = int(x.shape[-1])
        by, bx = self._scale_geometry(inner)
        scale_dtype = {torch.uint8: "e8m0", torch.float32: "float32", torch.bfloat16: "bfloat16"}[self.scale_dtype]
        stride = div_ceil(inner, bx)
        if x.numel() == inner:
            result = fp8_weight_only_gemv(x.reshape(inner), layer.weight, layer.weight_scale, scale_row_stride=stride,
                                          block_size_y=by, block_size_x=bx, scale_dtype=scale_dtype)
        else:
            result = fp8_weight_only_gemm(x, layer.weight, layer.weight_scale, scale_row_stride=stride,
                                          block_size_y=by, block_size_x=bx, scale_dtype=scale_dtype)
        bias = self._bias(args, kwargs)
        return result + bias if bias is not None else result


class FP8Mxfp8LinearMethod(_FP8LinearMethodBase):
    """MXFP8: e4m3 activations and weights with UE8M0 scales per 32-wide K group."""

    MX_GROUP = 32

    def __init__(self) -> None:
        super().__init__(activation_bits=8)

    def create_scale_parameters(self, layer, total_output, input_size, device) -> None:
        if input_size % self.MX_GROUP:
            raise ValueError("MXFP8 requires the weight K to be divisible by 32")
        self._scale_param(layer, "weight_scale", (total_output, input_size // self.MX_GROUP), torch.uint8, 0xFF, device)

    def process_weights_after_loading(self, layer: nn.Module) -> None:
        scale = layer.weight_scale
        # 0xFF is both the sentinel and the UE8M0 NaN code: never a valid scale.
        if scale.is_meta or bool((scale == 0xFF).any().item()):
            raise _not_loaded("weight_scale")

    def apply(self, layer: nn.Module, *args: Any, **kwargs: Any) -> torch.Tensor:
        from ayaka.kernel.hip.gemm.fp8_mxfp8_gemm import mxfp8_scaled_mm
        from ayaka.kernel.hip.quant.fp8_quant import per_token_group_quant_mxfp8

        x = args[0]
        lead, inner = tuple(x.shape[:-1]), int(x.shape[-1])
        if inner % self.MX_GROUP:
            raise ValueError("MXFP8 requires the activation K to be divisible by 32")
        x2d = x.reshape(-1, inner)
        if not x2d.is_contiguous():
            x2d = x2d.contiguous()
        weight = layer.weight
        quantized, activation_scale = per_token_group_quant_mxfp8(x2d, self.MX_GROUP)
        out = torch.empty((x2d.shape[0], int(weight.shape[0])), dtype=x.dtype, device=x.device)
        result = mxfp8_scaled_mm(quantized, activation_scale, weight, layer.weight_scale, self._bias(args, kwargs), out=out)
        return result.reshape(*lead, result.shape[-1])


# ------------------------------------------------------------------ config
def method_from_recipe(parsed: Any) -> QuantizeMethodBase:
    """Dense FP8 method of a parsed checkpoint recipe (``ParsedFP8Config``)."""
    recipe = parsed.recipe.recipe
    return _method_for(recipe, parsed.scale_dtype, parsed.recipe.weight_block)


def _method_for(recipe: FP8Recipe, scale_dtype: torch.dtype, weight_block) -> QuantizeMethodBase:
    if recipe is FP8Recipe.W8A8_STATIC_PER_TENSOR:
        return FP8PerTensorLinearMethod(activation_scheme="static")
    if recipe is FP8Recipe.W8A8_DYNAMIC_PER_TENSOR:
        return FP8PerTensorLinearMethod(activation_scheme="dynamic")
    if recipe is FP8Recipe.W8A8_ROWWISE:
        return FP8RowwiseLinearMethod()
    if recipe is FP8Recipe.W8A8_BLOCK128:
        return FP8BlockLinearMethod(scale_dtype=scale_dtype)
    if recipe is FP8Recipe.W8A16:
        return FP8W8A16LinearMethod(scale_dtype=scale_dtype, weight_block=weight_block)
    if recipe is FP8Recipe.MXFP8:
        return FP8Mxfp8LinearMethod()
    raise CapabilityError(
        "quantization.fp8_recipe",
        detail=f"recipe {recipe.value!r} has no dense linear method",
        remedy="use the KV-cache quantization owner for cache recipes",
    )


class FP8Config(BaseQuantization):
    """Select a dense FP8 linear method from a validated recipe descriptor."""

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

    def get_quant_method(self, layer: nn.Module, prefix: str) -> QuantizeMethodBase | None:
        del layer
        if any(prefix == ignored or prefix.startswith(f"{ignored}.") for ignored in self.ignored_layers):
            return None
        return self._make_method()


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
