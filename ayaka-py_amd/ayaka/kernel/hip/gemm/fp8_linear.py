"""Dense FP8 linear entry points used by the FP8 linear methods.

Public contract of ``python/ayaka/kernel/triton/gemm/fp8_linear.py:102-260``: the same
three functions, arguments, validations (order, exception types, messages) and recipe
routing. Routing by the flattened row count ``M``:

=================  ====================================  ==================================
recipe             M == 1                                 M > 1
=================  ====================================  ==================================
per-tensor         weight-only GEMV, scale rows 1 or N   static quant + scaled GEMM when an
                                                         ``input_scale`` is given, else the
                                                         weight-only GEMM
rowwise            weight-only GEMV, per-row scale       per-token quant + scaled GEMM
block-128          weight-only GEMV, 128 x 128 blocks    group-128 quant + block GEMM
=================  ====================================  ==================================

How the calls are assembled is this module's own: one ``_Activation`` record carries
the validated, flattened input and knows how to shape a result back; each recipe is a
short decision over it. For the W8A8 GEMMs the bias is added in fp32 inside the GEMM
epilogue (one rounding to the activation dtype) where the reference adds it afterwards
in the activation dtype (two roundings); the weight-only paths add it afterwards as the
reference does.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from ayaka.kernel.hip._common import require_fp8_dtype, validate_bias, validate_operand
from ayaka.kernel.hip._host import require_cuda, require_dtype, require_tensor
from ayaka.kernel.hip.gemm.fp8_gemm import (fp8_blockwise_mm, fp8_rowwise_linear_small, fp8_scaled_mm,
                                            rowwise_small_applies)
from ayaka.kernel.hip.gemm.fp8_gemv import fp8_weight_only_gemv
from ayaka.kernel.hip.gemm.fp8_w8a16_gemm import fp8_weight_only_gemm
from ayaka.kernel.hip.quant.fp8_quant import (per_token_group_quant_fp8, per_token_group_quant_fp8_colmajor,
                                              per_token_quant_fp8, static_quant_fp8)
from ayaka.utils.math_utils import div_ceil

__all__ = ["fp8_block_linear", "fp8_pertensor_linear", "fp8_rowwise_linear"]

#: K (and N) extent of one block scale in the block-128 checkpoint contract.
_SCALE_TILE = 128
# Row counts up to this run the decode-batch GEMM kernels, which read row-major
# activation scales in 16-byte chunks; larger ones the tiled kernels.
_DECODE_BATCH_ROWS = 64


@dataclass(frozen=True)
class _Activation:
    """A validated ``[..., K]`` activation viewed as a contiguous ``[M, K]`` matrix, and
    the ``[N, K]`` weight it is multiplied with."""

    lead: tuple[int, ...]
    matrix: torch.Tensor
    columns: int

    @property
    def rows(self) -> int:
        return int(self.matrix.shape[0])

    @property
    def inner(self) -> int:
        return int(self.matrix.shape[1])

    @classmethod
    def of(cls, x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> _Activation:
        # Validation order of the reference: activation, then weight against K, then bias.
        require_tensor(x, "x")
        require_dtype(x, "x", (torch.float16, torch.bfloat16))
        require_cuda(x, "x")
        if x.ndim < 1:
            raise ValueError("x must have at least one dimension")
        k = int(x.shape[-1])
        lead = tuple(int(d) for d in x.shape[:-1])
        matrix = x.reshape(math.prod(lead), k)  # prod(()) == 1: a [K] input is one row
        if not matrix.is_contiguous():
            matrix = matrix.contiguous()
        validate_operand(weight, "weight", dtype=require_fp8_dtype(), allow_transposed=False)
        if int(weight.shape[1]) != k:
            raise ValueError(f"weight must be [N, K] with K={k}, got {tuple(weight.shape)}")
        act = cls(lead, matrix, int(weight.shape[0]))
        validate_bias(bias, matrix, act.columns, reference_name="x")
        return act

    def empty_output(self) -> torch.Tensor:
        return torch.empty((self.rows, self.columns), dtype=self.matrix.dtype, device=self.matrix.device)

    def shaped(self, result: torch.Tensor, bias_after: torch.Tensor | None = None) -> torch.Tensor:
        """``result`` ([M, N] or [N]) back to ``[..., N]``, adding a not-yet-applied bias."""
        if bias_after is not None:
            result = result + bias_after
        return result.reshape(*self.lead, self.columns)

    def weight_only(self, weight: torch.Tensor, scale: torch.Tensor, scale_rows: int, scale_cols: int,
                    scale_dtype: str) -> torch.Tensor:
        """The activation is not quantized: decode GEMV at one row, W8A16 GEMM above.
        ``scale_rows x scale_cols`` is the weight-scale block (``block_size_y/x``)."""
        geometry = dict(scale_row_stride=div_ceil(self.inner, scale_cols), block_size_y=scale_rows,
                        block_size_x=scale_cols, scale_dtype=scale_dtype)
        if self.rows == 1:
            return fp8_weight_only_gemv(self.matrix.reshape(self.inner), weight, scale, **geometry)
        return fp8_weight_only_gemm(self.matrix, weight, scale, **geometry)

    def channel_scaled(self, weight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
        """Weight-only product for a scalar or per-row ``[N]`` fp32 weight scale."""
        rows_per_scale = self.columns if scale.numel() == 1 else 1
        return self.weight_only(weight, scale, rows_per_scale, self.inner, "float32")


def fp8_pertensor_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None = None,
    input_scale: torch.Tensor | None = None,
    uniform_scale: bool = False,
) -> torch.Tensor:
    """``x @ (weight * weight_scale)^T`` for a scalar or per-row ``[N]`` fp32 weight scale.

    With ``input_scale`` (static W8A8), ``M > 1`` quantizes the activation with it and
    runs the scaled GEMM; otherwise every ``M`` stays weight-only. ``uniform_scale``
    declares a piecewise-constant ``[N]`` scale, which the GEMM then takes as a scalar.
    """
    act = _Activation.of(x, weight, bias)
    if act.rows == 1 or input_scale is None:
        return act.shaped(act.channel_scaled(weight, weight_scale), bias)
    gemm_scale = weight_scale.reshape(-1)[0] if uniform_scale and weight_scale.numel() > 1 else weight_scale
    result = fp8_scaled_mm(static_quant_fp8(act.matrix, input_scale), weight.t(), input_scale.reshape(()),
                           gemm_scale, bias=bias, out=act.empty_output(), backend="auto")
    return act.shaped(result)


def fp8_rowwise_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """``x @ (weight * weight_scale)^T``; ``M > 1`` quantizes the activation per token."""
    act = _Activation.of(x, weight, bias)
    if act.rows == 1:
        return act.shaped(act.channel_scaled(weight, weight_scale), bias)
    if rowwise_small_applies(act.matrix, weight, weight_scale):
        # 2-8 rows against a small weight: quantizer and GEMM in one launch (same bits)
        return act.shaped(fp8_rowwise_linear_small(act.matrix, weight, weight_scale, bias))
    quantized, token_scale = per_token_quant_fp8(act.matrix)
    result = fp8_scaled_mm(quantized, weight.t(), token_scale, weight_scale, bias=bias, out=act.empty_output(),
                           backend="auto")
    return act.shaped(result)


def fp8_block_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """``x @ dequant(weight)^T`` with ``[ceil(N/128), ceil(K/128)]`` fp32/bf16 block scales;
    ``M > 1`` quantizes the activation per (token, 128-K group), so K must divide by 128."""
    act = _Activation.of(x, weight, bias)
    if act.rows == 1:
        scale_dtype = "bfloat16" if weight_scale.dtype is torch.bfloat16 else "float32"
        return act.shaped(act.weight_only(weight, weight_scale, _SCALE_TILE, _SCALE_TILE, scale_dtype), bias)
    if act.inner % _SCALE_TILE:
        raise ValueError(f"K={act.inner} must be divisible by 128 for the blockwise W8A8 path")
    if act.rows > _DECODE_BATCH_ROWS:
        # Prefill sizes: the quantizer writes the scales column-major, one cache line per
        # 32 rows for the GEMM's per-block scale reads (same values, same result bits).
        quantized, group_scale = per_token_group_quant_fp8_colmajor(act.matrix, _SCALE_TILE)
        result = fp8_blockwise_mm(quantized, weight, group_scale, weight_scale, bias=bias, out=act.empty_output(),
                                  a_scale_col_major=True)
        return act.shaped(result)
    quantized, group_scale = per_token_group_quant_fp8(act.matrix, _SCALE_TILE)
    result = fp8_blockwise_mm(quantized, weight, group_scale, weight_scale, bias=bias, out=act.empty_output())
    return act.shaped(result)
