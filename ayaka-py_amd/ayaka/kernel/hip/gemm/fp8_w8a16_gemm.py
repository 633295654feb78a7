"""W8A16 GEMM operator (M > 1): e4m3 weights dequantized onto 16-bit MFMA.

Reference ``python/ayaka/kernel/triton/gemm/fp8_w8a16_gemm.py:144`` (and the
``fp8_matmul_channelwise`` convenience wrapper, :238). Each dequantized weight
``w * scale`` is rounded to the activation dtype before the product, as the
reference does, then multiplied on ``v_mfma_f32_32x32x16_{bf16,f16}`` with fp32
accumulation; the output is rounded once to the activation dtype.
"""

import torch

from ayaka.kernel.hip import _lib
from ayaka.kernel.hip._common import validate_w8a16_scale, weight_bytes
from ayaka.kernel.hip._host import prepare_output, require_cuda, require_last_dim_stride1
from ayaka.kernel.ops import custom_op
from ayaka.utils.math_utils import div_ceil

__all__ = ["fp8_matmul_channelwise", "fp8_weight_only_gemm"]

_SCALE_FORMATS = ("e8m0", "float32", "bfloat16")
_SCALE_CODES = {"e8m0": _lib.AYK_U8, "float32": _lib.AYK_F32, "bfloat16": _lib.AYK_BF16}


def _fp8_weight_only_gemm_fake(input, weight, weight_scale, scale_row_stride=None, block_size_y=1,
                               block_size_x=128, scale_dtype="e8m0", out=None):
    return out if out is not None else torch.empty((input.shape[0], weight.shape[0]), dtype=input.dtype, device=input.device)


def _aligned_rows(t: torch.Tensor, elem_align: int) -> torch.Tensor:
    """``t`` if the kernel's 16-byte loads fit its layout, else a zero-padded copy."""
    rows, k = t.shape
    if k % elem_align == 0 and (rows <= 1 or t.stride(0) % elem_align == 0) and t.data_ptr() % 16 == 0:
        return t
    padded = torch.zeros((rows, div_ceil(k, 16) * 16), dtype=t.dtype, device=t.device)
    padded[:, :k] = t
    return padded


@custom_op(name="fp8_weight_only_gemm", fake_impl=_fp8_weight_only_gemm_fake, mutates_args=["out"])
def fp8_weight_only_gemm(
    input: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    scale_row_stride: int | None = None,
    block_size_y: int = 1,
    block_size_x: int = 128,
    scale_dtype: str = "e8m0",
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``input @ dequant(weight).T`` for ``[M, K]`` fp16/bf16 activations.

    Args:
        input: ``[M, K]`` fp16/bf16, ``stride(1) == 1``.
        weight: ``[N, K]`` e4m3 or raw ``uint8`` bytes.
        weight_scale: storage of ``scale[n // block_size_y, k // block_size_x]``.
        scale_row_stride: distance between scale rows (default ``ceil(K / block_size_x)``).
        scale_dtype: ``"e8m0"``, ``"float32"`` or ``"bfloat16"``.
        out: optional ``[M, N]`` buffer of ``input``'s dtype.
    """
    if not isinstance(input, torch.Tensor):
        raise TypeError("input must be a torch.Tensor")
    if input.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("input must have dtype float16 or bfloat16")
    require_cuda(input, "input")
    if input.ndim != 2:
        raise ValueError("input must be 2-D")
    if input.stride(1) != 1:
        raise ValueError("input must have stride(1) == 1")
    weight_view = weight_bytes(weight)
    if weight_view.shape[1] != input.shape[1]:
        raise ValueError("weight must be [N, K] with the same K as input")
    rows, inner, columns = int(input.shape[0]), int(input.shape[1]), int(weight_view.shape[0])
    if block_size_x <= 0 or block_size_y <= 0:
        raise ValueError("block sizes must be positive")
    if scale_dtype not in _SCALE_FORMATS:
        raise ValueError("scale_dtype must be 'e8m0', 'float32', or 'bfloat16'")
    if scale_row_stride is None:
        scale_row_stride = div_ceil(inner, block_size_x)
    if scale_row_stride <= 0:
        raise ValueError("scale_row_stride must be positive")
    validate_w8a16_scale(weight_scale, input, scale_dtype=scale_dtype, block_size_y=block_size_y,
                         scale_row_stride=scale_row_stride, columns=columns)
    result = prepare_output(input, out, shape=(rows, columns), like_name="input")
    require_last_dim_stride1(result, "out")
    if rows == 0 or columns == 0:
        return result
    x_k = _aligned_rows(input, 8)
    w_k = _aligned_rows(weight_view, 16)
    scale = weight_scale if weight_scale.is_contiguous() else weight_scale.contiguous()
    nbytes = _lib.query("ayk_fp8_weight_only_gemm_workspace_bytes", rows, columns, inner, block_size_x)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=input.device) if nbytes else None
    _lib.call(
        "ayk_fp8_weight_only_gemm", x_k.data_ptr(), _lib.dtype_code(input.dtype),
        int(x_k.stride(0)) if rows > 1 else int(x_k.shape[1]), rows,
        w_k.data_ptr(), int(w_k.stride(0)) if columns > 1 else int(w_k.shape[1]), columns, inner,
        scale.data_ptr(), _SCALE_CODES[scale_dtype], scale_row_stride, block_size_y, block_size_x,
        result.data_ptr(), int(result.stride(0)) if rows > 1 else columns,
        _lib.ptr(ws), nbytes, _lib.stream_of(input),
    )
    return result


def fp8_matmul_channelwise(input: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor) -> torch.Tensor:
    """Per-output-channel fp32 scales: ``weight_scale`` is ``[N]``."""
    if not isinstance(input, torch.Tensor):
        raise TypeError("input must be a torch.Tensor")
    if input.ndim != 2:
        raise ValueError("input must be 2-D")
    return fp8_weight_only_gemm(input, weight, weight_scale, scale_row_stride=1, block_size_y=1,
                                block_size_x=int(input.shape[1]), scale_dtype="float32")
