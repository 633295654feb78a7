"""Element-type registry of the FP8 linear path: the reference's ``DType``
(``ayaka/types.py:8-60``) with the same members, labels, bit widths, torch names,
safetensors tokens (``F8_E4M3`` / ``U8`` for FP8 weights and UE8M0 scale codes,
``types.py:32,40``) and finite maxima, so checkpoint headers map onto it."""

from __future__ import annotations

import enum


class DType(enum.Enum):
    """``(label, bits, sub_byte, torch_name, safetensors_token, max_finite)`` per type."""

    FP64 = ("fp64", 64, False, "float64", "F64", None)
    FP32 = ("fp32", 32, False, "float32", "F32", 3.4028234663852886e38)
    FP16 = ("fp16", 16, False, "float16", "F16", 65504.0)
    BF16 = ("bf16", 16, False, "bfloat16", "BF16", 3.3895313892515355e38)
    FP8_E4M3 = ("fp8_e4m3", 8, False, "float8_e4m3fn", "F8_E4M3", 448.0)
    FP8_E5M2 = ("fp8_e5m2", 8, False, "float8_e5m2", "F8_E5M2", 57344.0)
    FP4_E2M1 = ("fp4_e2m1", 4, True, None, "F4", None)
    INT64 = ("int64", 64, False, "int64", "I64", None)
    INT32 = ("int32", 32, False, "int32", "I32", None)
    INT8 = ("int8", 8, False, "int8", "I8", None)
    UINT8 = ("uint8", 8, False, "uint8", "U8", None)
    INT4 = ("int4", 4, True, None, "I4", None)
    BOOL = ("bool", 8, False, "bool", "BOOL", None)

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

        if self.torch_name is None:
            raise TypeError(f"{self.label} has no torch dtype (sub-byte, stored packed)")
        return getattr(torch, self.torch_name)

    def nbytes(self, numel: int) -> int:
        """Bytes that ``numel`` elements occupy (sub-byte types packed, rounded up)."""
        return (int(numel) * self.bits + 7) // 8

    @classmethod
    def from_str(cls, name: str) -> "DType":
        """Member by label, enum name, torch name or safetensors token (case-insensitive)."""
        key = name.strip().lower()
        for member in cls:
            names = (member.label, member.name.lower(), member.safetensors_token.lower())
            if key in names or (member.torch_name is not None and key == member.torch_name):
                return member
        raise ValueError(f"unknown dtype {name!r}")


#: dtypes every compute layer of this path accepts as activations.
COMPUTE_DTYPES = (DType.FP16, DType.BF16, DType.FP32)


def compute_torch_dtypes() -> tuple:
    """Torch dtypes of :data:`COMPUTE_DTYPES`."""
    return tuple(dtype.torch_dtype for dtype in COMPUTE_DTYPES)
