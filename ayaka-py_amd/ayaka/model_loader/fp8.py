"""FP8 checkpoint adapter: ``quantization_config`` -> explicit recipe contract.

Same functions, keys, decision order and errors as the reference
(``python/ayaka/model_loader/fp8.py:53-437``):

* :func:`parse_fp8_config` detects the recipe (explicit name, then KV-only, then
  W8A16 before any MX hint, then MXFP8, block-128, rowwise hint, static, and the
  dynamic per-tensor default), resolves the scale dtype (block-128 defaults to
  bf16), the amax floor (1e-10) and the calibration provenance, and returns a
  validated :class:`ParsedFP8Config`;
* :func:`expected_scale_keys` / :func:`validate_scale_key_set` enforce the
  checkpoint's scale tensor names;
* :func:`normalize_scale` inverts an inverse scale exactly once;
* :func:`shard_scale_k` slices a block scale's K axis for one rank.
"""

from __future__ import annotations

from collections.abc import Mapping, Sequence
from dataclasses import dataclass
from typing import Any

import torch

from ayaka.types import DType
from ayaka.utils.math_utils import div_ceil
from ayaka.weights.spec import (
    FP8ActivationScheme,
    FP8Recipe,
    FP8RecipeSpec,
    FP8ScaleDirection,
    FP8ScaleFormat,
    FP8ValueFormat,
    FP8ZeroPolicy,
    QuantSpec,
)

__all__ = [
    "FP8_SCALE_KEY_SUFFIXES",
    "ParsedFP8Config",
    "classify_scale_key",
    "expected_scale_keys",
    "normalize_scale",
    "parse_fp8_config",
    "recipe_from_config",
    "scale_blocks_for_k",
    "shard_scale_k",
    "validate_scale_key_set",
]

_DYNAMIC_FLOOR = 1e-10

#: scale kind -> checkpoint tensor suffixes
FP8_SCALE_KEY_SUFFIXES: dict[str, tuple[str, ...]] = {
    "weight_scale": ("weight_scale",),
    "weight_scale_inv": ("weight_scale_inv",),
    "input_scale": ("input_scale",),
    "kv_scale": ("k_scale", "v_scale"),
}

_FORMAT_OF_DTYPE = {torch.float32: FP8ScaleFormat.FP32, torch.bfloat16: FP8ScaleFormat.BF16, torch.uint8: FP8ScaleFormat.UE8M0}
_DTYPE_OF_FORMAT = {v: k for k, v in _FORMAT_OF_DTYPE.items()}
_DTYPE_ENUM_OF_FORMAT = {FP8ScaleFormat.FP32: DType.FP32, FP8ScaleFormat.BF16: DType.BF16, FP8ScaleFormat.UE8M0: DType.UINT8}

_WEIGHT_ONLY = ("none", "weight_only", "weight-only")


def _first(config: Mapping[str, Any], *keys: str, default: Any = None) -> Any:
    """Value of the first key present with a non-None value."""
    for key in keys:
        value = config.get(key)
        if value is not None:
            return value
    return default


def _int_pair(value: Any, name: str) -> tuple[int, int] | None:
    if value is None:
        return None
    if isinstance(value, (list, tuple)) and len(value) == 2 and all(
        isinstance(v, int) and not isinstance(v, bool) for v in value
    ):
        return int(value[0]), int(value[1])
    raise ValueError(f"{name} must be a (rows, K) integer pair, got {value!r}")


def _scale_format(value: Any) -> FP8ScaleFormat | None:
    if value is None:
        return None
    token = str(value).lower().replace("torch.", "")
    for fmt, names in ((FP8ScaleFormat.UE8M0, ("ue8m0", "e8m0", "uint8")),
                       (FP8ScaleFormat.BF16, ("bfloat16", "bf16")),
                       (FP8ScaleFormat.FP32, ("float32", "fp32", "float"))):
        if token in names:
            return fmt
    raise ValueError(f"unknown scale format {value!r}")


def _is_inverse(config: Mapping[str, Any], explicit: Any) -> bool:
    if explicit is not None:
        return str(explicit).lower() in ("inverse", "inv", "scale_inv")
    return bool(_first(config, "use_scale_inv", "scale_inv", default=False)) or bool(
        _first(config, "weight_scale_inv", default=False)
    )


def _weight_block(config: Mapping[str, Any]) -> tuple[int, int] | None:
    return _int_pair(_first(config, "weight_block_size", "weight_block", "weight_blocks"), "weight_block_size")


def _detect_recipe(config: Mapping[str, Any]) -> FP8Recipe:
    """Recipe of a ``quantization_config``; the order of the checks is the contract."""
    explicit = _first(config, "fp8_recipe", "recipe")
    if explicit is not None:
        try:
            return FP8Recipe(str(explicit))
        except ValueError as error:
            allowed = ", ".join(member.value for member in FP8Recipe)
            raise ValueError(f"unknown fp8 recipe {explicit!r}; expected one of: {allowed}") from error
    algo = str(_first(config, "quant_algo", "quantization", "quant_method", "method", default="")).lower()
    block = _weight_block(config)
    activation = str(_first(config, "activation_scheme", "activation", default="")).lower()
    fmt = _scale_format(_first(config, "scale_format", "scale_dtype", "scale_fmt"))
    serialized = bool(_first(config, "is_checkpoint_fp8_serialized", "serialized", default=False))
    kv_scheme = _first(config, "kv_cache_scheme", "kv_scheme")
    weight_quant = bool(activation) or block is not None or serialized or any(
        token in algo for token in ("mxfp8", "w8a8", "w8a16"))
    if kv_scheme is not None and not weight_quant:
        return FP8Recipe.KV_CACHE
    # weight-only first: a W8A16 checkpoint may carry UE8M0 scales and a weight block
    if activation in _WEIGHT_ONLY or "w8a16" in algo:
        return FP8Recipe.W8A16
    if "mxfp8" in algo or block == (1, 32) or fmt is FP8ScaleFormat.UE8M0:
        return FP8Recipe.MXFP8
    if block == (128, 128) or "block" in algo:
        if block != (128, 128):
            raise ValueError("block FP8 requires weight_block_size=[128, 128]")
        return FP8Recipe.W8A8_BLOCK128
    if block is not None:
        raise ValueError(f"unsupported weight_block_size {block}; expected [128, 128] or [1, 32]")
    hint = str(_first(config, "weight_scheme", "weight_granularity", "weight_strategy", default="")).lower()
    if "rowwise" in activation or "rowwise" in hint:
        return FP8Recipe.W8A8_ROWWISE
    if activation in ("static", "calibrated"):
        return FP8Recipe.W8A8_STATIC_PER_TENSOR
    return FP8Recipe.W8A8_DYNAMIC_PER_TENSOR


def _scale_dtype(recipe: FP8Recipe, fmt: FP8ScaleFormat | None) -> torch.dtype:
    if recipe is FP8Recipe.KV_CACHE:
        return torch.float32
    if recipe is FP8Recipe.MXFP8:
        return torch.uint8
    if fmt is not None:
        return _DTYPE_OF_FORMAT[fmt]
    return torch.bfloat16 if recipe is FP8Recipe.W8A8_BLOCK128 else torch.float32


def _activation_scheme(recipe: FP8Recipe) -> FP8ActivationScheme:
    return {FP8Recipe.W8A16: FP8ActivationScheme.NONE,
            FP8Recipe.W8A8_STATIC_PER_TENSOR: FP8ActivationScheme.STATIC,
            FP8Recipe.KV_CACHE: FP8ActivationScheme.CALIBRATED}.get(recipe, FP8ActivationScheme.DYNAMIC)


def _blocks(recipe: FP8Recipe):
    if recipe is FP8Recipe.W8A8_BLOCK128:
        return (1, 128), (128, 128)
    if recipe is FP8Recipe.MXFP8:
        return (1, 32), (1, 32)
    return None, None


@dataclass(frozen=True, slots=True)
class ParsedFP8Config:
    """Checkpoint metadata normalised into the FP8 contract (``quant`` is None for KV)."""

    recipe: FP8RecipeSpec
    quant: QuantSpec | None
    scale_dtype: torch.dtype
    ignored_layers: tuple[str, ...]

    @property
    def method_name(self) -> str:
        return self.recipe.recipe.value


def parse_fp8_config(config: Mapping[str, Any]) -> ParsedFP8Config:
    """Parse and validate one ``quantization_config`` mapping.

    Raises:
        TypeError: ``config`` is not a mapping.
        ValueError: unknown or contradictory recipe, block, scale format or provenance.
    """
    if not isinstance(config, Mapping):
        raise TypeError("quantization_config must be a mapping")
    recipe = _detect_recipe(config)
    fmt = _scale_format(_first(config, "scale_format", "scale_dtype", "scale_fmt"))
    if recipe is FP8Recipe.W8A8_BLOCK128 and fmt is None:
        fmt = FP8ScaleFormat.BF16
    scale_dtype = _scale_dtype(recipe, fmt)
    fmt = FP8ScaleFormat.FP32 if recipe is FP8Recipe.KV_CACHE else _FORMAT_OF_DTYPE[scale_dtype]

    activation_block, weight_block = _blocks(recipe)
    if recipe is FP8Recipe.W8A16:
        weight_block = _weight_block(config)
    scheme = _activation_scheme(recipe)
    if recipe not in (FP8Recipe.W8A16, FP8Recipe.KV_CACHE):
        configured = str(_first(config, "activation_scheme", "activation", default="")).lower()
        if configured in _WEIGHT_ONLY:
            raise ValueError(f"recipe {recipe.value!r} requires an activation scheme, got 'none'")

    checkpoint_scaled = scheme in (FP8ActivationScheme.STATIC, FP8ActivationScheme.CALIBRATED) or recipe is FP8Recipe.W8A16
    zero_policy = FP8ZeroPolicy.CHECKPOINT_SCALE if checkpoint_scaled else FP8ZeroPolicy.AMAX_FLOOR
    amax_floor = float(_first(config, "amax_floor", default=_DYNAMIC_FLOOR)) if zero_policy is FP8ZeroPolicy.AMAX_FLOOR else None
    calibration = (str(_first(config, "calibration_source", "calibration", "calibrated_by", default="quantization_config"))
                   if checkpoint_scaled else None)
    direction = FP8ScaleDirection.INVERSE if _is_inverse(config, _first(config, "scale_direction")) else FP8ScaleDirection.DEQUANT
    layout = str(_first(config, "logical_scale_layout", "scale_layout", default="row_major"))
    spec = FP8RecipeSpec(
        recipe=recipe,
        value_format=FP8ValueFormat.E4M3,
        activation_scheme=scheme,
        activation_block=activation_block,
        weight_block=weight_block,
        scale_format=fmt,
        scale_direction=direction,
        logical_scale_layout=layout,
        physical_scale_layout=str(_first(config, "physical_scale_layout", default=layout)),
        zero_policy=zero_policy,
        amax_floor=amax_floor,
        calibration_source=calibration,
        excluded_layers=tuple(str(n) for n in _first(config, "ignored_layers", "ignored", "exclude", default=())),
    )
    quant = None if recipe is FP8Recipe.KV_CACHE else QuantSpec(
        method="fp8", weight_dtype=DType.FP8_E4M3, scale_dtype=_DTYPE_ENUM_OF_FORMAT[spec.scale_format], fp8_recipe=spec)
    return ParsedFP8Config(recipe=spec, quant=quant, scale_dtype=scale_dtype, ignored_layers=spec.excluded_layers)


def recipe_from_config(config: Mapping[str, Any]) -> tuple[FP8Recipe, torch.dtype, tuple[str, ...]]:
    """``(recipe, scale dtype, ignored layers)`` of a ``quantization_config``."""
    parsed = parse_fp8_config(config)
    return parsed.recipe.recipe, parsed.scale_dtype, parsed.ignored_layers


def expected_scale_keys(recipe: FP8Recipe) -> tuple[str, ...]:
    """Scale tensor kinds a checkpoint of ``recipe`` must ship."""
    if recipe is FP8Recipe.KV_CACHE:
        return ("k_scale", "v_scale")
    if recipe not in FP8Recipe:
        raise ValueError(f"unknown FP8 recipe {recipe!r}")
    keys = ["weight_scale_inv" if recipe is FP8Recipe.W8A8_BLOCK128 else "weight_scale"]
    if recipe is FP8Recipe.W8A8_STATIC_PER_TENSOR:
        keys.append("input_scale")
    return tuple(keys)


def classify_scale_key(key: str) -> str | None:
    """Scale kind carried by a checkpoint tensor name, or None."""
    leaf = key.rsplit(".", 1)[-1]
    for kind, suffixes in FP8_SCALE_KEY_SUFFIXES.items():
        if leaf in suffixes:
            return kind
    return None


def validate_scale_key_set(keys: Sequence[str], recipe: FP8Recipe) -> None:
    """Reject a checkpoint whose scale tensors do not match ``recipe``."""
    present = {classify_scale_key(k) for k in keys} - {None}
    expected = set(expected_scale_keys(recipe))
    missing = expected - present
    if missing:
        raise ValueError(f"{recipe.value} checkpoint is missing scale tensors: {sorted(missing)}")
    for kind in present:
        if kind not in expected and kind != "kv_scale":
            raise ValueError(f"{recipe.value} checkpoint carries an unexpected scale tensor kind {kind!r}")


def normalize_scale(scale: torch.Tensor, *, direction: FP8ScaleDirection) -> torch.Tensor:
    """Dequant scale; an inverse scale is inverted exactly once. UE8M0 codes pass through."""
    if scale.dtype is torch.uint8 or direction is FP8ScaleDirection.DEQUANT:
        return scale
    values = scale.float()
    if not bool(torch.isfinite(values).all().item()) or bool((values <= 0).any().item()):
        raise ValueError("inverse scale must be finite and positive")
    return 1.0 / scale


def shard_scale_k(scale: torch.Tensor, *, rank: int, world_size: int, block: int = 128) -> torch.Tensor:
    """K-axis slice of a ``[rows, K / block]`` block scale owned by one rank."""
    if world_size < 1:
        raise ValueError("world_size must be >= 1")
    if not 0 <= rank < world_size:
        raise ValueError("rank must be smaller than world_size")
    if block < 1:
        raise ValueError("block must be positive")
    if scale.ndim != 2:
        raise ValueError("scale must be 2-D [rows, K / block]")
    columns = int(scale.shape[1])
    if columns % world_size:
        raise ValueError(f"scale K blocks {columns} must divide by world_size={world_size}")
    if world_size == 1:
        return scale
    local = columns // world_size
    return scale[:, rank * local:(rank + 1) * local]


def scale_blocks_for_k(inner: int, block: int) -> int:
    """Scale columns a ``block``-wide K axis needs."""
    return div_ceil(inner, block)
