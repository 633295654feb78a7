"""Operand / scale / bias contracts shared by the GEMM and GEMV wrappers.

Same checks, exception types and message fragments as the reference
(``python/ayaka/kernel/triton/gemm/_common.py:316-479``), so a caller switching
to this package sees identical failures for bad inputs.
"""

from __future__ import annotations

import torch

from ayaka.kernel.hip._host import dtype_list, require_cuda, require_dtype, require_same_device, require_tensor
from ayaka.utils.math_utils import div_ceil

#: Dtypes accepted for scales, biases and GEMM outputs.
FLOAT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
OUTPUT_DTYPES = FLOAT_DTYPES

#: K width (and N height) of one block-FP8 scale.
SCALE_BLOCK_K = 128

FP8 = torch.float8_e4m3fn


def require_fp8_dtype() -> torch.dtype:
    """The OCP e4m3fn dtype (present in every supported torch build)."""
    return FP8


def validate_operand(tensor: torch.Tensor, name: str, *, dtype: torch.dtype, allow_transposed: bool) -> None:
    """2-D operand of ``dtype``, row-major (or column-major when ``allow_transposed``)."""
    require_tensor(tensor, name)
    require_dtype(tensor, name, (dtype,))
    require_cuda(tensor, name)
    if tensor.ndim != 2:
        raise ValueError(f"{name} must be 2-D")
    if tensor.stride(1) != 1 and not (allow_transposed and tensor.stride(0) == 1):
        layout = "stride(1) == 1 or stride(0) == 1" if allow_transposed else "stride(1) == 1"
        raise ValueError(f"{name} must have {layout}")


def validate_scale(
    scale: torch.Tensor,
    name: str,
    reference: torch.Tensor,
    size: int,
    *,
    dtypes: tuple[torch.dtype, ...] = FLOAT_DTYPES,
    scalar_ok: bool = True,
    reference_name: str = "a",
) -> None:
    """Scalar or contiguous ``[size]`` dequantization scale."""
    require_tensor(scale, name)
    require_same_device(scale, name, reference, reference_name)
    if scale.dtype not in dtypes:
        raise TypeError(f"{name} must have dtype {dtype_list(dtypes)}")
    if scale.ndim == 0:
        if scalar_ok:
            return
        raise ValueError(f"{name} must have shape [{size}]")
    if scale.ndim != 1 or scale.numel() != size:
        if scalar_ok:
            raise ValueError(f"{name} must be a scalar or a vector of shape [{size}]")
        raise ValueError(f"{name} must have shape [{size}]")
    if scale.stride(0) != 1:
        raise ValueError(f"{name} must be contiguous")


def validate_block_scale(
    scale: torch.Tensor,
    name: str,
    reference: torch.Tensor,
    shape: tuple[int, int],
    *,
    dtypes: tuple[torch.dtype, ...] = FLOAT_DTYPES,
    reference_name: str = "a",
) -> None:
    """Contiguous 2-D block scale of exactly ``shape``."""
    require_tensor(scale, name)
    require_same_device(scale, name, reference, reference_name)
    if scale.dtype not in dtypes:
        raise TypeError(f"{name} must have dtype {dtype_list(dtypes)}")
    if tuple(scale.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {shape}")
    if not scale.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def validate_bias(
    bias: torch.Tensor | None,
    reference: torch.Tensor,
    size: int,
    *,
    dtypes: tuple[torch.dtype, ...] = FLOAT_DTYPES,
    reference_name: str = "a",
) -> None:
    """Optional ``[size]`` additive bias."""
    if bias is None:
        return
    require_tensor(bias, "bias")
    require_same_device(bias, "bias", reference, reference_name)
    if bias.dtype not in dtypes:
        raise TypeError(f"bias must have dtype {dtype_list(dtypes)}")
    if tuple(bias.shape) != (size,):
        raise ValueError(f"bias must have shape [{size}]")


_W8A16_SCALE_DTYPES = {"e8m0": torch.uint8, "float32": torch.float32, "bfloat16": torch.bfloat16}


def validate_w8a16_scale(
    weight_scale: torch.Tensor,
    reference: torch.Tensor,
    *,
    scale_dtype: str,
    block_size_y: int,
    scale_row_stride: int,
    columns: int,
    reference_name: str = "input",
) -> None:
    """Packed UE8M0 / fp32 / bf16 weight-scale storage of the weight-only path."""
    require_tensor(weight_scale, "weight_scale")
    require_same_device(weight_scale, "weight_scale", reference, reference_name)
    expected = _W8A16_SCALE_DTYPES[scale_dtype]
    if weight_scale.dtype is not expected:
        raise TypeError(f"{scale_dtype} weight_scale must have dtype {expected}")
    if weight_scale.numel() < div_ceil(columns, block_size_y) * scale_row_stride:
        raise ValueError("weight_scale storage is too small for the requested block layout")


def weight_bytes(weight: torch.Tensor) -> torch.Tensor:
    """``uint8`` view of a uint8 / e4m3 ``[N, K]`` weight with ``stride(1) == 1``."""
    require_tensor(weight, "weight")
    require_cuda(weight, "weight")
    if weight.ndim != 2:
        raise ValueError("weight must be 2-D")
    if weight.dtype is torch.uint8:
        byte_view = weight
    elif weight.dtype is FP8:
        byte_view = weight.view(torch.uint8)
    else:
        raise TypeError("weight must have dtype uint8 or torch.float8_e4m3fn")
    if byte_view.stride(1) != 1:
        raise ValueError("weight must have stride(1) == 1")
    return byte_view
