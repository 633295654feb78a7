"""Quantization method hooks the FP8 linear methods implement.

The subset of the reference's ``ayaka/layers/quantization/base.py`` (targets
``:35-45``, capabilities ``:229-259``, ``QuantizeMethodBase`` ``:347``,
``BaseQuantization`` ``:457``) that a linear layer's quantization lifecycle uses:
create weights -> load -> ``process_weights_after_loading`` -> ``apply``.
"""

from __future__ import annotations

import enum
from abc import ABC, abstractmethod
from collections.abc import Mapping
from dataclasses import dataclass
from typing import Any

import torch
from torch import nn


class QuantizationTarget(str, enum.Enum):
    LINEAR = "linear"
    EMBEDDING = "embedding"
    LM_HEAD = "lm_head"
    KV_CACHE = "kv_cache"
    MOE = "moe"

    def __str__(self) -> str:
        return str(self.value)


@dataclass(frozen=True)
class QuantizationCapabilities:
    """Static capability declaration of a quantization method."""

    supported_act_dtypes: tuple[torch.dtype, ...] = ()
    supported_devices: frozenset[str] = frozenset({"cpu", "cuda"})
    supported_targets: frozenset[QuantizationTarget] = frozenset({QuantizationTarget.LINEAR})
    min_cuda_capability: int | None = None
    required_modules: tuple[str, ...] = ()
    storage_format: str | None = None
    weight_bits: int | None = None
    activation_bits: int | None = None
    supports_tensor_parallel: bool = True
    supports_expert_parallel: bool = False
    supports_dynamic_activation: bool = False
    supports_static_activation: bool = True
    supports_online_quantization: bool = False

    def __post_init__(self) -> None:
        devices = frozenset(d.lower() for d in self.supported_devices)
        object.__setattr__(self, "supported_devices", devices)
        object.__setattr__(self, "supported_act_dtypes", tuple(self.supported_act_dtypes))
        object.__setattr__(self, "required_modules", tuple(self.required_modules))
        object.__setattr__(self, "supported_targets", frozenset(QuantizationTarget(t) for t in self.supported_targets))
        if not devices:
            raise ValueError("supported_devices must not be empty")
        if not self.supported_targets:
            raise ValueError("supported_targets must not be empty")


class QuantizeMethodBase(ABC):
    """Storage creation and execution of one quantized layer."""

    @abstractmethod
    def create_weights(self, layer: nn.Module, *weight_args: Any, **extra_weight_attrs: Any) -> None: ...

    @abstractmethod
    def apply(self, layer: nn.Module, *args: Any, **kwargs: Any) -> torch.Tensor: ...

    def process_weights_after_loading(self, layer: nn.Module) -> None:
        """Validate / repack loaded weights once, before the first ``apply``."""
        return None

    def get_capabilities(self) -> QuantizationCapabilities:
        return QuantizationCapabilities()

    def supports(self, target: QuantizationTarget) -> bool:
        return QuantizationTarget(target) in self.get_capabilities().supported_targets


class BaseQuantization(ABC):
    """A quantization configuration: picks a method per layer."""

    @classmethod
    @abstractmethod
    def get_name(cls) -> str: ...

    @classmethod
    @abstractmethod
    def from_config(cls, config: Mapping[str, Any]) -> BaseQuantization: ...

    @abstractmethod
    def get_capabilities(self) -> QuantizationCapabilities: ...

    @abstractmethod
    def get_quant_method(self, layer: nn.Module, prefix: str) -> QuantizeMethodBase | None: ...
