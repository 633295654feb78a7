"""Dense FP8 linear entry points used by the FP8 linear methods.

Same functions, arguments and dispatch as the reference's
``python/ayaka/kernel/triton/gemm/fp8_linear.py:102-260``:

* ``M == 1`` runs the weight-only decode GEMV over the raw fp8 weight (the
  activation is not quantized), for every recipe here;
* rowwise and dynamic per-tensor quantize the activation per token, then run the
  scaled GEMM; static per-tensor quantizes with the calibrated ``input_scale``;
* block-128 quantizes per (token, 128-K group), then runs the block-scaled GEMM.

One deliberate difference: for the W8A8 GEMMs the bias is added in fp32 inside the
GEMM epilogue (one rounding to the activation dtype) instead of a separate
activation-dtype add afterwards (two roundings). The GEMV paths add it afterwards,
as the reference does.
"""

from __future__ import annotations

import math

import torch

from ayaka.kernel.hip._common import require_fp8_dtype, validate_bias, validate_operand
from ayaka.kernel.hip._host import require_cuda, require_dtype, require_tensor
from ayaka.kernel.hip.gemm.fp8_gemm import fp8_blockwise_mm, fp8_scaled_mm
from ayaka.kernel.hip.gemm.fp8_gemv import fp8_weight_only_gemv
from ayaka.kernel.hip.gemm.fp8_w8a16_gemm import fp8_weight_only_gemm
from ayaka.kernel.hip.quant.fp8_quant import per_token_group_quant_fp8, per_token_quant_fp8, static_quant_fp8
from ayaka.utils.math_utils import div_ceil

__all__ = ["fp8_block_linear", "fp8_pertensor_linear", "fp8_rowwise_linear"]

_BLOCK128 = 128


def _validate_activation(x: torch.Tensor) -> None:
    require_tensor(x, "x")
    require_dtype(x, "x", (torch.float16, torch.bfloat16))
    require_cuda(x, "x")
    if x.ndim < 1:
        raise ValueError("x must have at least one dimension")


def _validate_dense_weight(weight: torch.Tensor, inner: int) -> None:
    validate_operand(weight, "weight", dtype=require_fp8_dtype(), allow_transposed=False)
    if weight.shape[1] != inner:
        raise ValueError(f"weight must be [N, K] with K={inner}, got {tuple(weight.shape)}")


def _flatten_activation(x: torch.Tensor) -> tuple[tuple[int, ...], int, int, torch.Tensor]:
    lead = tuple(x.shape[:-1])
    inner = int(x.shape[-1])
    rows = math.prod(lead) if lead else 1
    x2d = x.reshape(rows, inner)
    if not x2d.is_contiguous():
        x2d = x2d.contiguous()
    return lead, inner, rows, x2d


def _weight_only(x2d, weight, weight_scale, *, block_size_y: int, block_size_x: int, scale_dtype: str) -> torch.Tensor:
    """W8A16: split-K GEMV at one row, tiled GEMM above it."""
    inner = int(x2d.shape[1])
    stride = div_ceil(inner, block_size_x)
    if x2d.shape[0] == 1:
        return fp8_weight_only_gemv(x2d.reshape(inner), weight, weight_scale, scale_row_stride=stride,
                                    block_size_y=block_size_y, block_size_x=block_size_x, scale_dtype=scale_dtype)
    return fp8_weight_only_gemm(x2d, weight, weight_scale, scale_row_stride=stride,
                                block_size_y=block_size_y, block_size_x=block_size_x, scale_dtype=scale_dtype)


def _output(x2d: torch.Tensor, columns: int) -> torch.Tensor:
    return torch.empty((x2d.shape[0], columns), dtype=x2d.dtype, device=x2d.device)


def _finish(result: torch.Tensor, lead: tuple[int, ...], bias: torch.Tensor | None) -> torch.Tensor:
    if bias is not None:
        result = result + bias
    return result.reshape(*lead, result.shape[-1])


def fp8_pertensor_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None = None,
    input_scale: torch.Tensor | None = None,
    uniform_scale: bool = False,
) -> torch.Tensor:
    """``x @ (weight * weight_scale)^T`` for a scalar or per-row ``[N]`` fp32 weight scale.

    ``input_scale`` (static W8A8) runs static quant + scaled GEMM at ``M > 1``;
    without it ``M > 1`` runs weight-only. ``M == 1`` always runs the GEMV.
    ``uniform_scale`` lets a piecewise-constant ``[N]`` scale collapse to a scalar.
    """
    _validate_activation(x)
    lead, inner, rows, x2d = _flatten_activation(x)
    _validate_dense_weight(weight, inner)
    columns = int(weight.shape[0])
    validate_bias(bias, x2d, columns, reference_name="x")
    scale = weight_scale
    if uniform_scale and scale.numel() > 1:
        scale = scale.reshape(-1)[0]
    if rows == 1 or input_scale is None:
        result = _weight_only(x2d, weight, weight_scale, block_size_y=columns if weight_scale.numel() == 1 else 1,
                              block_size_x=inner, scale_dtype="float32")
        return _finish(result, lead, bias)
    quantized = static_quant_fp8(x2d, input_scale)
    result = fp8_scaled_mm(quantized, weight.t(), input_scale.reshape(()), scale, bias=bias,
                           out=_output(x2d, columns), backend="auto")
    return _finish(result, lead, None)


def fp8_rowwise_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """``x @ (weight * weight_scale)^T`` with dynamic per-token W8A8 at ``M > 1``."""
    _validate_activation(x)
    lead, inner, rows, x2d = _flatten_activation(x)
    _validate_dense_weight(weight, inner)
    columns = int(weight.shape[0])
    validate_bias(bias, x2d, columns, reference_name="x")
    if rows == 1:
        result = _weight_only(x2d, weight, weight_scale, block_size_y=columns if weight_scale.numel() == 1 else 1,
                              block_size_x=inner, scale_dtype="float32")
        return _finish(result, lead, bias)
    quantized, activation_scale = per_token_quant_fp8(x2d)
    result = fp8_scaled_mm(quantized, weight.t(), activation_scale, weight_scale, bias=bias,
                           out=_output(x2d, columns), backend="auto")
    return _finish(result, lead, None)


def fp8_block_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """``x @ dequant(weight)^T`` with ``[ceil(N/128), ceil(K/128)]`` block scales."""
    _validate_activation(x)
    lead, inner, rows, x2d = _flatten_activation(x)
    _validate_dense_weight(weight, inner)
    columns = int(weight.shape[0])
    validate_bias(bias, x2d, columns, reference_name="x")
    scale_dtype = "bfloat16" if weight_scale.dtype is torch.bfloat16 else "float32"
    if rows == 1:
        result = _weight_only(x2d, weight, weight_scale, block_size_y=_BLOCK128, block_size_x=_BLOCK128,
                              scale_dtype=scale_dtype)
        return _finish(result, lead, bias)
    if inner % _BLOCK128:
        raise ValueError(f"K={inner} must be divisible by 128 for the blockwise W8A8 path")
    quantized, activation_scale = per_token_group_quant_fp8(x2d, _BLOCK128)
    result = fp8_blockwise_mm(quantized, weight, activation_scale, weight_scale, bias=bias, out=_output(x2d, columns))
    return _finish(result, lead, None)
