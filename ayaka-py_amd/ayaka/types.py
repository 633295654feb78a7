"""Element-type registry of the FP8 linear path (subset of the reference's
``ayaka/types.py:8-60`` ``DType``: the same members, labels and attributes for the
types this path stores or computes in)."""

from __future__ import annotations

import enum


class DType(enum.Enum):
    """``(label, bits, sub_byte, torch_name, safetensors_token, max_finite)`` per type."""

    FP32 = ("fp32", 32, False, "float32", "F32", 3.4028234663852886e38)
    FP16 = ("fp16", 16, False, "float16", "F16", 65504.0)
    BF16 = ("bf16", 16, False, "bfloat16", "BF16", 3.3895313892515355e38)
    FP8_E4M3 = ("fp8_e4m3", 8, False, "float8_e4m3fn", "F8_E4M3", 448.0)
    FP8_E5M2 = ("fp8_e5m2", 8, False, "float8_e5m2", "F8_E5M2", 57344.0)
    UINT8 = ("uint8", 8, False, "uint8", "U8", None)

    def __init__(self, label, bits, sub_byte, torch_name, safetensors_token, max_finite):
        self.label = label
        self.bits = bits
        self.sub_byte = sub_byte
        self.torch_name = torch_name
        self.safetensors_token = safetensors_token
        self.max_finite = max_finite

    @property
    def torch_dtype(self):
        import torch

        return getattr(torch, self.torch_name)


#: dtypes every compute layer of this path accepts as activations.
COMPUTE_DTYPES = (DType.FP16, DType.BF16, DType.FP32)


def compute_torch_dtypes() -> tuple:
    """Torch dtypes of :data:`COMPUTE_DTYPES`."""
    return tuple(dtype.torch_dtype for dtype in COMPUTE_DTYPES)
