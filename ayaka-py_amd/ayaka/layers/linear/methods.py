"""Linear specialisation of the quantization method contract
(reference ``ayaka/layers/linear/methods.py:26-37``)."""

from __future__ import annotations

from typing import ClassVar

from ayaka.layers.quantization.base import QuantizationCapabilities, QuantizeMethodBase
from ayaka.types import compute_torch_dtypes


class LinearMethodBase(QuantizeMethodBase):
    uses_weight_loader_v2: ClassVar[bool] = False

    def get_capabilities(self) -> QuantizationCapabilities:
        return QuantizationCapabilities(supported_devices=frozenset({"cuda"}),
                                        supported_act_dtypes=compute_torch_dtypes())
