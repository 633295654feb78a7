"""Integer helpers."""

from __future__ import annotations


def div_ceil(a: int, b: int) -> int:
    """``ceil(a / b)`` for integers of any sign (``b != 0``)."""
    return -(-a // b)


def validate_output_dtype(dtype) -> None:
    """Require a supported kernel output dtype (``float16``, ``bfloat16`` or ``float32``).

    Raises ``ValueError`` otherwise, as the reference's ``utils/math_utils.py:210``.
    """
    import torch

    if dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("out_dtype must be float16, bfloat16, or float32")
