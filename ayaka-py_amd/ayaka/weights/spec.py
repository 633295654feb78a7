"""FP8 recipe contract types (reference ``ayaka/weights/spec.py:154-486``).

Same enum values, dataclass fields and validation rules, so a recipe built by a
reference checkpoint adapter validates identically here. Python 3.10 has no
``enum.StrEnum``; :class:`_StrEnum` gives the same ``str``-valued behaviour.
"""

from __future__ import annotations

import enum
import json
import math
from dataclasses import dataclass

from ayaka.types import DType


class _StrEnum(str, enum.Enum):
    def __str__(self) -> str:
        return str(self.value)


class FP8Recipe(_StrEnum):
    W8A8_STATIC_PER_TENSOR = "w8a8_static_per_tensor"
    W8A8_DYNAMIC_PER_TENSOR = "w8a8_dynamic_per_tensor"
    W8A8_ROWWISE = "w8a8_rowwise"
    W8A8_BLOCK128 = "w8a8_block128"
    MXFP8 = "mxfp8"
    W8A16 = "w8a16"
    KV_CACHE = "kv_cache"


class FP8ValueFormat(_StrEnum):
    E4M3 = "e4m3"
    E5M2 = "e5m2"


class FP8ActivationScheme(_StrEnum):
    NONE = "none"
    STATIC = "static"
    DYNAMIC = "dynamic"
    CALIBRATED = "calibrated"


class FP8ScaleFormat(_StrEnum):
    FP32 = "float32"
    BF16 = "bfloat16"
    UE8M0 = "ue8m0"


class FP8ScaleDirection(_StrEnum):
    DEQUANT = "dequant"
    INVERSE = "inverse"


class FP8ZeroPolicy(_StrEnum):
    AMAX_FLOOR = "amax_floor"
    CHECKPOINT_SCALE = "checkpoint_scale"


_A = FP8ActivationScheme
_F = FP8ScaleFormat
_Z = FP8ZeroPolicy

#: recipe -> (activation scheme, activation block, weight block, scale format, zero policy)
RECIPE_CONTRACTS: dict[FP8Recipe, tuple] = {
    FP8Recipe.W8A8_STATIC_PER_TENSOR: (_A.STATIC, None, None, _F.FP32, _Z.CHECKPOINT_SCALE),
    FP8Recipe.W8A8_DYNAMIC_PER_TENSOR: (_A.DYNAMIC, None, None, _F.FP32, _Z.AMAX_FLOOR),
    FP8Recipe.W8A8_ROWWISE: (_A.DYNAMIC, None, None, _F.FP32, _Z.AMAX_FLOOR),
    FP8Recipe.W8A8_BLOCK128: (_A.DYNAMIC, (1, 128), (128, 128), _F.FP32, _Z.AMAX_FLOOR),
    FP8Recipe.MXFP8: (_A.DYNAMIC, (1, 32), (1, 32), _F.UE8M0, _Z.AMAX_FLOOR),
}


def _check_block(name: str, block) -> None:
    if block is None:
        return
    if not isinstance(block, tuple) or len(block) != 2:
        raise TypeError(f"{name} must be a (rows, K) tuple or None")
    if any(isinstance(v, bool) or not isinstance(v, int) for v in block):
        raise TypeError(f"{name} entries must be integers")
    if any(v < 1 for v in block):
        raise ValueError(f"{name} entries must be positive")


@dataclass(frozen=True, slots=True)
class FP8RecipeSpec:
    """Immutable description of one FP8 inference recipe (logical ``(rows, K)`` blocks)."""

    recipe: FP8Recipe
    value_format: FP8ValueFormat
    activation_scheme: FP8ActivationScheme
    activation_block: tuple[int, int] | None
    weight_block: tuple[int, int] | None
    scale_format: FP8ScaleFormat
    scale_direction: FP8ScaleDirection
    logical_scale_layout: str
    physical_scale_layout: str
    zero_policy: FP8ZeroPolicy
    amax_floor: float | None = None
    calibration_source: str | None = None
    excluded_layers: tuple[str, ...] = ()
    version: int = 1

    def __post_init__(self) -> None:
        for name, kind in (("recipe", FP8Recipe), ("value_format", FP8ValueFormat),
                           ("activation_scheme", FP8ActivationScheme), ("scale_format", FP8ScaleFormat),
                           ("scale_direction", FP8ScaleDirection), ("zero_policy", FP8ZeroPolicy)):
            try:
                object.__setattr__(self, name, kind(getattr(self, name)))
            except ValueError as error:
                allowed = ", ".join(member.value for member in kind)
                raise ValueError(f"{name} must be one of: {allowed}") from error
        _check_block("activation_block", self.activation_block)
        _check_block("weight_block", self.weight_block)
        for name in ("logical_scale_layout", "physical_scale_layout"):
            value = getattr(self, name)
            if not isinstance(value, str) or not value.strip():
                raise ValueError(f"{name} must be a non-empty metadata identifier")
            object.__setattr__(self, name, value.strip())
        if self.zero_policy is FP8ZeroPolicy.AMAX_FLOOR:
            if isinstance(self.amax_floor, bool) or not isinstance(self.amax_floor, (int, float)):
                raise TypeError("amax_floor must be a finite positive number for dynamic recipes")
            try:
                floor = float(self.amax_floor)
            except OverflowError as error:
                raise ValueError("amax_floor must be finite and positive") from error
            if not math.isfinite(floor) or floor <= 0.0:
                raise ValueError("amax_floor must be finite and positive")
            object.__setattr__(self, "amax_floor", floor)
        elif self.amax_floor is not None:
            raise ValueError("amax_floor is only valid when zero_policy='amax_floor'")
        if self.calibration_source is not None:
            if not isinstance(self.calibration_source, str) or not self.calibration_source.strip():
                raise ValueError("calibration_source must be None or a non-empty string")
            object.__setattr__(self, "calibration_source", self.calibration_source.strip())
        if not isinstance(self.excluded_layers, tuple):
            raise TypeError("excluded_layers must be a tuple of layer names")
        if any(not isinstance(x, str) or not x.strip() for x in self.excluded_layers):
            raise ValueError("excluded_layers entries must be non-empty strings")
        layers = tuple(x.strip() for x in self.excluded_layers)
        if len(set(layers)) != len(layers):
            raise ValueError("excluded_layers must not contain duplicates")
        object.__setattr__(self, "excluded_layers", layers)
        if isinstance(self.version, bool) or not isinstance(self.version, int):
            raise TypeError("version must be an integer")
        if self.version < 1:
            raise ValueError("version must be >= 1")
        calibrated = self.activation_scheme in (_A.STATIC, _A.CALIBRATED) or self.recipe is FP8Recipe.W8A16
        if calibrated and self.calibration_source is None:
            raise ValueError("static, calibrated, and W8A16 recipes require calibration_source")
        self._validate_recipe_contract()

    def _validate_recipe_contract(self) -> None:
        recipe = self.recipe
        if recipe is FP8Recipe.KV_CACHE:
            if self.activation_scheme is not _A.CALIBRATED:
                raise ValueError("KV cache FP8 requires activation_scheme='calibrated'")
            if self.activation_block is not None or self.weight_block is not None:
                raise ValueError("KV cache FP8 uses per-layer/per-plane scales, not GEMM blocks")
            if self.scale_format is not _F.FP32:
                raise ValueError("KV cache FP8 scales must use float32")
            if self.zero_policy is not _Z.CHECKPOINT_SCALE:
                raise ValueError("KV cache FP8 requires a calibrated checkpoint scale policy")
            return
        if self.value_format is not FP8ValueFormat.E4M3:
            raise ValueError("E5M2 is supported only by the KV cache recipe")
        if recipe is FP8Recipe.W8A16:
            if self.activation_scheme is not _A.NONE:
                raise ValueError("W8A16 requires activation_scheme='none'")
            if self.activation_block is not None:
                raise ValueError("W8A16 does not quantize activations")
            if self.zero_policy is not _Z.CHECKPOINT_SCALE:
                raise ValueError("W8A16 requires checkpoint weight scales")
            return
        scheme, a_block, w_block, fmt, policy = RECIPE_CONTRACTS[recipe]
        if recipe is FP8Recipe.W8A8_BLOCK128 and self.scale_format is _F.BF16:
            fmt = _F.BF16  # block-128 checkpoints may ship bf16 scales
        required = (scheme, a_block, w_block, fmt, policy)
        actual = (self.activation_scheme, self.activation_block, self.weight_block, self.scale_format, self.zero_policy)
        if actual != required:
            raise ValueError(
                f"recipe {recipe.value!r} requires activation scheme/block, weight block, "
                f"scale format, and zero policy {required}; got {actual}"
            )

    @property
    def cache_key(self) -> str:
        """Stable recipe metadata for weight-plan digests."""
        payload = {
            "activation_block": self.activation_block,
            "activation_scheme": self.activation_scheme.value,
            "amax_floor": self.amax_floor,
            "calibration_source": self.calibration_source,
            "excluded_layers": self.excluded_layers,
            "logical_scale_layout": self.logical_scale_layout,
            "physical_scale_layout": self.physical_scale_layout,
            "recipe": self.recipe.value,
            "scale_direction": self.scale_direction.value,
            "scale_format": self.scale_format.value,
            "version": self.version,
            "value_format": self.value_format.value,
            "weight_block": self.weight_block,
            "zero_policy": self.zero_policy.value,
        }
        return json.dumps(payload, ensure_ascii=True, sort_keys=True, separators=(",", ":"))


_SCALE_DTYPE_FOR_FORMAT = {_F.UE8M0: DType.UINT8, _F.BF16: DType.BF16, _F.FP32: DType.FP32}


@dataclass(frozen=True, slots=True)
class QuantSpec:
    """Quantization of one weight. ``group_size`` -1 = per-channel, 0 = per-tensor; FP8
    weights carry their granularity in ``fp8_recipe`` and keep ``group_size`` at 0."""

    method: str = "none"
    weight_dtype: DType = DType.BF16
    scale_dtype: DType = DType.FP32
    group_size: int = 0
    symmetric: bool = True
    has_zero_point: bool = False
    fp8_recipe: FP8RecipeSpec | None = None

    def __post_init__(self) -> None:
        if not isinstance(self.method, str) or not self.method:
            raise ValueError("method must be a non-empty string")
        if not isinstance(self.weight_dtype, DType) or not isinstance(self.scale_dtype, DType):
            raise TypeError("weight_dtype and scale_dtype must be DType values")
        if isinstance(self.group_size, bool) or not isinstance(self.group_size, int):
            raise TypeError("group_size must be an integer")
        if self.group_size < -1:
            raise ValueError("group_size must be -1, 0, or a positive integer")
        if not isinstance(self.symmetric, bool) or not isinstance(self.has_zero_point, bool):
            raise TypeError("symmetric and has_zero_point must be bool values")
        if self.method == "fp8" and self.fp8_recipe is None:
            raise ValueError("FP8 QuantSpec requires an explicit fp8_recipe")
        if self.fp8_recipe is None:
            return
        if self.method != "fp8":
            raise ValueError("fp8_recipe may only be set when method='fp8'")
        if not isinstance(self.fp8_recipe, FP8RecipeSpec):
            raise TypeError("fp8_recipe must be an FP8RecipeSpec")
        if self.fp8_recipe.recipe is FP8Recipe.KV_CACHE:
            raise ValueError("KV cache quantization is owned by KVQuantization, not WeightSpec")
        if self.fp8_recipe.value_format is not FP8ValueFormat.E4M3:
            raise ValueError("FP8 weight recipes in QuantSpec require E4M3 storage")
        if self.weight_dtype is not DType.FP8_E4M3:
            raise ValueError("FP8 weight recipes require weight_dtype=FP8_E4M3")
        expected = _SCALE_DTYPE_FOR_FORMAT[self.fp8_recipe.scale_format]
        if self.scale_dtype is not expected:
            raise ValueError(f"{self.fp8_recipe.scale_format.value} scales require scale_dtype={expected.label}")
        if not self.symmetric or self.has_zero_point:
            raise ValueError("FP8 inference recipes require symmetric values without a zero point")
        if self.group_size != 0:
            raise ValueError("FP8RecipeSpec owns FP8 scale granularity; leave generic group_size at 0")

    @property
    def cache_key(self) -> str:
        payload = {
            "fp8_recipe": self.fp8_recipe.cache_key if self.fp8_recipe is not None else None,
            "group_size": self.group_size,
            "has_zero_point": self.has_zero_point,
            "method": self.method,
            "scale_dtype": self.scale_dtype.label,
            "symmetric": self.symmetric,
            "weight_dtype": self.weight_dtype.label,
        }
        return json.dumps(payload, ensure_ascii=True, sort_keys=True, separators=(",", ":"))

    @property
    def is_quantized(self) -> bool:
        return self.method != "none"
