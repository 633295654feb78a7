"""FP8 checkpoint adapter: ``quantization_config`` -> explicit recipe contract.

The public contract is the reference's (``python/ayaka/model_loader/fp8.py:53-437``):
function names, accepted keys and aliases, the recipe decision order, defaults
(block-128 scales default to bf16, dynamic amax floor 1e-10) and every error message.

The implementation is table-driven:

* ``_Keys`` reads a mapping through alias lists (``_ALIASES``): the first alias present
  with a non-None value wins;
* ``_DETECTION`` is the ordered list of recipe rules -- explicit name, a check of the
  block / scale-format hints, KV-only,
  weight-only (before any MX hint: a W8A16 checkpoint may carry UE8M0 scales),
  MXFP8, block-128, any other block (an error), rowwise hint, static, and the dynamic
  per-tensor default; the first rule that fires decides;
* ``_TRAITS`` holds each recipe's fixed facts: activation scheme, activation / weight
  blocks, default scale dtype and the checkpoint scale tensors it ships.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping, Sequence
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

#: logical field -> the config keys that may carry it, in priority order
_ALIASES: dict[str, tuple[str, ...]] = {
    "recipe": ("fp8_recipe", "recipe"),
    "algo": ("quant_algo", "quantization", "quant_method", "method"),
    "block": ("weight_block_size", "weight_block", "weight_blocks"),
    "activation": ("activation_scheme", "activation"),
    "scale_format": ("scale_format", "scale_dtype", "scale_fmt"),
    "serialized": ("is_checkpoint_fp8_serialized", "serialized"),
    "kv_scheme": ("kv_cache_scheme", "kv_scheme"),
    "weight_hint": ("weight_scheme", "weight_granularity", "weight_strategy"),
    "direction": ("scale_direction",),
    "inverse_flag": ("use_scale_inv", "scale_inv"),
    "inverse_key": ("weight_scale_inv",),
    "amax_floor": ("amax_floor",),
    "calibration": ("calibration_source", "calibration", "calibrated_by"),
    "logical_layout": ("logical_scale_layout", "scale_layout"),
    "physical_layout": ("physical_scale_layout",),
    "ignored": ("ignored_layers", "ignored", "exclude"),
}

#: scale-format spellings (lower case, "torch." stripped)
_FORMAT_SPELLINGS: dict[str, FP8ScaleFormat] = {
    **dict.fromkeys(("ue8m0", "e8m0", "uint8"), FP8ScaleFormat.UE8M0),
    **dict.fromkeys(("bfloat16", "bf16"), FP8ScaleFormat.BF16),
    **dict.fromkeys(("float32", "fp32", "float"), FP8ScaleFormat.FP32),
}
_FORMAT_OF_DTYPE = {torch.float32: FP8ScaleFormat.FP32, torch.bfloat16: FP8ScaleFormat.BF16, torch.uint8: FP8ScaleFormat.UE8M0}
_DTYPE_OF_FORMAT = {fmt: dtype for dtype, fmt in _FORMAT_OF_DTYPE.items()}
_DTYPE_ENUM_OF_FORMAT = {FP8ScaleFormat.FP32: DType.FP32, FP8ScaleFormat.BF16: DType.BF16, FP8ScaleFormat.UE8M0: DType.UINT8}

_WEIGHT_ONLY_SCHEMES = frozenset({"none", "weight_only", "weight-only"})
_INVERSE_DIRECTIONS = frozenset({"inverse", "inv", "scale_inv"})
_WEIGHT_QUANT_ALGOS = ("mxfp8", "w8a8", "w8a16")


class _Keys:
    """Alias-aware, normalising reads of one ``quantization_config`` mapping."""

    def __init__(self, config: Mapping[str, Any]) -> None:
        self._config = config

    def get(self, field: str, default: Any = None) -> Any:
        for key in _ALIASES[field]:
            value = self._config.get(key)
            if value is not None:
                return value
        return default

    def text(self, field: str) -> str:
        return str(self.get(field, "")).lower()

    def block(self) -> tuple[int, int] | None:
        value = self.get("block")
        if value is None:
            return None
        if (isinstance(value, (list, tuple)) and len(value) == 2
                and all(isinstance(v, int) and not isinstance(v, bool) for v in value)):
            return int(value[0]), int(value[1])
        raise ValueError(f"weight_block_size must be a (rows, K) integer pair, got {value!r}")

    def scale_format(self) -> FP8ScaleFormat | None:
        value = self.get("scale_format")
        if value is None:
            return None
        fmt = _FORMAT_SPELLINGS.get(str(value).lower().replace("torch.", ""))
        if fmt is None:
            raise ValueError(f"unknown scale format {value!r}")
        return fmt

    def inverse_scales(self) -> bool:
        direction = self.get("direction")
        if direction is not None:
            return str(direction).lower() in _INVERSE_DIRECTIONS
        return bool(self.get("inverse_flag", False)) or bool(self.get("inverse_key", False))


# ------------------------------------------------------------------ recipe detection
def _explicit(keys: _Keys) -> FP8Recipe | None:
    named = keys.get("recipe")
    if named is None:
        return None
    try:
        return FP8Recipe(str(named))
    except ValueError as error:
        allowed = ", ".join(member.value for member in FP8Recipe)
        raise ValueError(f"unknown fp8 recipe {named!r}; expected one of: {allowed}") from error


def _malformed_hints(keys: _Keys) -> FP8Recipe | None:
    """Never decides; rejects a malformed weight block or scale format before any
    recipe is inferred (whichever recipe the config would otherwise name)."""
    keys.block()
    keys.scale_format()
    return None


def _kv_only(keys: _Keys) -> FP8Recipe | None:
    algo = keys.text("algo")
    quantizes_weights = (bool(keys.text("activation")) or keys.block() is not None or bool(keys.get("serialized", False))
                         or any(token in algo for token in _WEIGHT_QUANT_ALGOS))
    return FP8Recipe.KV_CACHE if keys.get("kv_scheme") is not None and not quantizes_weights else None


def _weight_only(keys: _Keys) -> FP8Recipe | None:
    hit = keys.text("activation") in _WEIGHT_ONLY_SCHEMES or "w8a16" in keys.text("algo")
    return FP8Recipe.W8A16 if hit else None


def _mx(keys: _Keys) -> FP8Recipe | None:
    hit = "mxfp8" in keys.text("algo") or keys.block() == (1, 32) or keys.scale_format() is FP8ScaleFormat.UE8M0
    return FP8Recipe.MXFP8 if hit else None


def _block128(keys: _Keys) -> FP8Recipe | None:
    block = keys.block()
    if block != (128, 128) and "block" not in keys.text("algo"):
        return None
    if block != (128, 128):
        raise ValueError("block FP8 requires weight_block_size=[128, 128]")
    return FP8Recipe.W8A8_BLOCK128


def _other_block(keys: _Keys) -> FP8Recipe | None:
    block = keys.block()
    if block is not None:
        raise ValueError(f"unsupported weight_block_size {block}; expected [128, 128] or [1, 32]")
    return None


def _rowwise(keys: _Keys) -> FP8Recipe | None:
    hit = "rowwise" in keys.text("activation") or "rowwise" in keys.text("weight_hint")
    return FP8Recipe.W8A8_ROWWISE if hit else None


def _static(keys: _Keys) -> FP8Recipe | None:
    return FP8Recipe.W8A8_STATIC_PER_TENSOR if keys.text("activation") in ("static", "calibrated") else None


#: the decision order is the contract: the first rule returning a recipe decides
_DETECTION: tuple[Callable[[_Keys], FP8Recipe | None], ...] = (
    _explicit, _malformed_hints, _kv_only, _weight_only, _mx, _block128, _other_block, _rowwise, _static,
)


def _detect_recipe(config: Mapping[str, Any]) -> FP8Recipe:
    keys = _Keys(config)
    for rule in _DETECTION:
        recipe = rule(keys)
        if recipe is not None:
            return recipe
    return FP8Recipe.W8A8_DYNAMIC_PER_TENSOR


# ------------------------------------------------------------------ per-recipe facts
@dataclass(frozen=True)
class _RecipeTraits:
    scheme: FP8ActivationScheme
    activation_block: tuple[int, int] | None = None
    weight_block: tuple[int, int] | None = None
    default_scale: torch.dtype = torch.float32
    fixed_scale: torch.dtype | None = None  # the recipe admits no other scale dtype
    scale_keys: tuple[str, ...] = ("weight_scale",)


_DYNAMIC = FP8ActivationScheme.DYNAMIC
_TRAITS: dict[FP8Recipe, _RecipeTraits] = {
    FP8Recipe.W8A8_STATIC_PER_TENSOR: _RecipeTraits(FP8ActivationScheme.STATIC, scale_keys=("weight_scale", "input_scale")),
    FP8Recipe.W8A8_DYNAMIC_PER_TENSOR: _RecipeTraits(_DYNAMIC),
    FP8Recipe.W8A8_ROWWISE: _RecipeTraits(_DYNAMIC),
    FP8Recipe.W8A8_BLOCK128: _RecipeTraits(_DYNAMIC, (1, 128), (128, 128), default_scale=torch.bfloat16,
                                           scale_keys=("weight_scale_inv",)),
    FP8Recipe.MXFP8: _RecipeTraits(_DYNAMIC, (1, 32), (1, 32), fixed_scale=torch.uint8),
    FP8Recipe.W8A16: _RecipeTraits(FP8ActivationScheme.NONE),
    FP8Recipe.KV_CACHE: _RecipeTraits(FP8ActivationScheme.CALIBRATED, fixed_scale=torch.float32,
                                      scale_keys=("k_scale", "v_scale")),
}


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
    keys = _Keys(config)
    traits = _TRAITS[recipe]
    requested = keys.scale_format()
    if traits.fixed_scale is not None:
        scale_dtype = traits.fixed_scale
    else:
        scale_dtype = _DTYPE_OF_FORMAT[requested] if requested is not None else traits.default_scale

    if traits.scheme is not FP8ActivationScheme.NONE and recipe is not FP8Recipe.KV_CACHE:
        if keys.text("activation") in _WEIGHT_ONLY_SCHEMES:
            raise ValueError(f"recipe {recipe.value!r} requires an activation scheme, got 'none'")
    weight_block = keys.block() if recipe is FP8Recipe.W8A16 else traits.weight_block

    scale_from_checkpoint = traits.scheme in (FP8ActivationScheme.STATIC, FP8ActivationScheme.CALIBRATED,
                                              FP8ActivationScheme.NONE)
    layout = str(keys.get("logical_layout", "row_major"))
    spec = FP8RecipeSpec(
        recipe=recipe,
        value_format=FP8ValueFormat.E4M3,
        activation_scheme=traits.scheme,
        activation_block=traits.activation_block,
        weight_block=weight_block,
        scale_format=_FORMAT_OF_DTYPE[scale_dtype],
        scale_direction=FP8ScaleDirection.INVERSE if keys.inverse_scales() else FP8ScaleDirection.DEQUANT,
        logical_scale_layout=layout,
        physical_scale_layout=str(keys.get("physical_layout", layout)),
        zero_policy=FP8ZeroPolicy.CHECKPOINT_SCALE if scale_from_checkpoint else FP8ZeroPolicy.AMAX_FLOOR,
        amax_floor=None if scale_from_checkpoint else float(keys.get("amax_floor", _DYNAMIC_FLOOR)),
        calibration_source=str(keys.get("calibration", "quantization_config")) if scale_from_checkpoint else None,
        excluded_layers=tuple(str(name) for name in keys.get("ignored", ())),
    )
    quant = None if recipe is FP8Recipe.KV_CACHE else QuantSpec(
        method="fp8", weight_dtype=DType.FP8_E4M3, scale_dtype=_DTYPE_ENUM_OF_FORMAT[spec.scale_format], fp8_recipe=spec)
    return ParsedFP8Config(recipe=spec, quant=quant, scale_dtype=scale_dtype, ignored_layers=spec.excluded_layers)


def recipe_from_config(config: Mapping[str, Any]) -> tuple[FP8Recipe, torch.dtype, tuple[str, ...]]:
    """``(recipe, scale dtype, ignored layers)`` of a ``quantization_config``."""
    parsed = parse_fp8_config(config)
    return parsed.recipe.recipe, parsed.scale_dtype, parsed.ignored_layers


# ------------------------------------------------------------------ scale tensors
def expected_scale_keys(recipe: FP8Recipe) -> tuple[str, ...]:
    """Scale tensor kinds a checkpoint of ``recipe`` must ship."""
    traits = _TRAITS.get(recipe)
    if traits is None:
        raise ValueError(f"unknown FP8 recipe {recipe!r}")
    return traits.scale_keys


def classify_scale_key(key: str) -> str | None:
    """Scale kind carried by a checkpoint tensor name, or None."""
    leaf = key.rpartition(".")[2]
    return next((kind for kind, suffixes in FP8_SCALE_KEY_SUFFIXES.items() if leaf in suffixes), None)


def validate_scale_key_set(keys: Sequence[str], recipe: FP8Recipe) -> None:
    """Reject a checkpoint whose scale tensors do not match ``recipe``."""
    present = {kind for kind in map(classify_scale_key, keys) if kind is not None}
    expected = set(expected_scale_keys(recipe))
    missing = expected - present
    if missing:
        raise ValueError(f"{recipe.value} checkpoint is missing scale tensors: {sorted(missing)}")
    unexpected = present - expected - {"kv_scale"}
    if unexpected:
        kind = next(iter(unexpected))
        raise ValueError(f"{recipe.value} checkpoint carries an unexpected scale tensor kind {kind!r}")


def normalize_scale(scale: torch.Tensor, *, direction: FP8ScaleDirection) -> torch.Tensor:
    """Dequant scale; an inverse scale is inverted exactly once. UE8M0 codes pass through."""
    if scale.dtype is torch.uint8 or direction is FP8ScaleDirection.DEQUANT:
        return scale
    values = scale.float()
    if not (bool(torch.isfinite(values).all().item()) and bool((values > 0).all().item())):
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
    blocks = int(scale.shape[1])
    if blocks % world_size:
        raise ValueError(f"scale K blocks {blocks} must divide by world_size={world_size}")
    per_rank = blocks // world_size
    return scale if world_size == 1 else scale.narrow(1, rank * per_rank, per_rank)


def scale_blocks_for_k(inner: int, block: int) -> int:
    """Scale columns a ``block``-wide K axis needs."""
    return div_ceil(inner, block)
