"""Host-side contract checks shared by the operator wrappers.

Mirrors the guards of the reference (``python/ayaka/kernel/triton/_host.py:18-207``)
so callers see the same exception types and message fragments: ``TypeError`` for a
non-tensor or a wrong dtype, ``ValueError`` for device, rank, shape and stride.
"""

from __future__ import annotations

from collections.abc import Iterable

import torch


def dtype_list(dtypes: Iterable[torch.dtype]) -> str:
    """Human-readable enumeration, e.g. ``"float16, bfloat16, or float32"``."""
    names = [str(dtype).replace("torch.", "", 1) for dtype in dtypes]
    if len(names) == 1:
        return names[0]
    if len(names) == 2:
        return f"{names[0]} or {names[1]}"
    return ", ".join(names[:-1]) + f", or {names[-1]}"


def require_tensor(x: object, name: str) -> None:
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")


def require_cuda(x: torch.Tensor, name: str) -> None:
    require_tensor(x, name)
    if not x.is_cuda:
        raise ValueError(f"{name} must be a CUDA tensor")


def require_dtype(x: torch.Tensor, name: str, dtypes: tuple[torch.dtype, ...]) -> None:
    if x.dtype not in dtypes:
        raise TypeError(f"{name} must have dtype {dtype_list(dtypes)}; got {x.dtype}")


def require_shape(x: torch.Tensor, name: str, shape: tuple[int, ...]) -> None:
    if tuple(x.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(x.shape)}")


def require_same_device(x: torch.Tensor, name: str, reference: torch.Tensor, reference_name: str) -> None:
    if x.device != reference.device:
        raise ValueError(f"{name} and {reference_name} must be on the same CUDA device")


def require_last_dim_stride1(x: torch.Tensor, name: str) -> None:
    if x.dim() == 0 or x.stride(-1) != 1:
        raise ValueError(f"{name} must have stride(-1) == 1")


def prepare_output(
    like: torch.Tensor,
    out: torch.Tensor | None,
    *,
    shape: tuple[int, ...] | None = None,
    dtype: torch.dtype | None = None,
    dtypes: tuple[torch.dtype, ...] | None = None,
    name: str = "out",
    like_name: str = "input",
) -> torch.Tensor:
    """Validate a caller's ``out`` or allocate a fresh one on ``like``'s device."""
    resolved_shape = tuple(like.shape) if shape is None else tuple(shape)
    resolved_dtype = like.dtype if dtype is None else dtype
    if out is None:
        return torch.empty(resolved_shape, device=like.device, dtype=resolved_dtype)
    require_tensor(out, name)
    require_same_device(out, name, like, like_name)
    allowed = (resolved_dtype,) if dtypes is None else tuple(dtypes)
    if out.dtype not in allowed:
        raise TypeError(f"{name} must have dtype {dtype_list(allowed)}; got {out.dtype}")
    require_shape(out, name, resolved_shape)
    return out


def fake_tensor(like: torch.Tensor, *, shape: tuple[int, ...] | None = None, dtype: torch.dtype | None = None) -> torch.Tensor:
    """Uninitialised meta-kernel output."""
    return torch.empty(
        tuple(like.shape) if shape is None else tuple(shape),
        dtype=like.dtype if dtype is None else dtype,
        device=like.device,
    )
