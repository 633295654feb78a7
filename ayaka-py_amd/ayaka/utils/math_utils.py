"""Integer helpers."""

from __future__ import annotations


def div_ceil(a: int, b: int) -> int:
    """``ceil(a / b)`` for integers of any sign (``b != 0``)."""
    return -(-a // b)
