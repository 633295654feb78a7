"""Decode (M == 1) FP8 GEMV operators on the gfx950 split-K GEMV kernel.

Operators and contracts of the reference (``python/ayaka/kernel/triton/gemm/fp8_gemv.py``):

* ``fp8_weight_only_gemv`` (:323) -- W8A16: fp16/bf16 activation, e4m3 weight with
  ``scale[n // block_size_y, k // block_size_x]`` in UE8M0 / fp32 / bf16;
* ``fp8_blockwise_gemv`` (:433) -- W8A8: the M == 1 case of the 128-block contract.

The K split is chosen from shapes only (never tensor values), with a fixed-order
reduction, so results are deterministic and the launch is graph-capture safe.
"""

import torch

from ayaka.kernel.hip import _lib
from ayaka.kernel.hip._common import (
    FP8,
    OUTPUT_DTYPES,
    validate_bias,
    validate_block_scale,
    validate_operand,
    validate_scale,
    validate_w8a16_scale,
    weight_bytes,
)
from ayaka.kernel.hip._host import prepare_output, require_cuda, require_dtype, require_last_dim_stride1, require_tensor
from ayaka.kernel.ops import custom_op
from ayaka.utils.math_utils import div_ceil

__all__ = ["fp8_blockwise_gemv", "fp8_weight_only_gemv"]

_SCALE_FORMATS = ("e8m0", "float32", "bfloat16")
_SCALE_CODES = {"e8m0": _lib.AYK_U8, "float32": _lib.AYK_F32, "bfloat16": _lib.AYK_BF16}
_BLOCK_K = 128


def _flatten_vector(x: torch.Tensor, name: str, size: int) -> torch.Tensor:
    if not isinstance(x, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if x.numel() != size:
        raise ValueError(f"{name} must have exactly {size} elements (M == 1)")
    require_cuda(x, name)
    flat = x.reshape(-1)
    return flat if flat.is_contiguous() else flat.contiguous()


def _vector_output(reference: torch.Tensor, out: torch.Tensor | None, size: int, dtype: torch.dtype) -> torch.Tensor:
    result = prepare_output(reference, out, shape=(size,), dtype=dtype, like_name="input")
    require_last_dim_stride1(result, "out")
    return result


def _workspace(query: str, n: int, k: int, device: torch.device) -> tuple[torch.Tensor | None, int]:
    nbytes = _lib.query(query, n, k)
    if nbytes == 0:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes


# ------------------------------------------------------------------ W8A16
def _weight_only_gemv_fake(
    input: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    scale_row_stride: int | None = None,
    block_size_y: int = 1,
    block_size_x: int = 128,
    scale_dtype: str = "e8m0",
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    return out if out is not None else torch.empty((weight.shape[0],), dtype=input.dtype, device=input.device)


@custom_op(name="fp8_weight_only_gemv", fake_impl=_weight_only_gemv_fake, mutates_args=["out"])
def fp8_weight_only_gemv(
    input: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    scale_row_stride: int | None = None,
    block_size_y: int = 1,
    block_size_x: int = 128,
    scale_dtype: str = "e8m0",
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``input @ dequant(weight).T`` for one activation row.

    Args:
        input: ``[K]`` (any shape with K elements) fp16/bf16 CUDA tensor.
        weight: ``[N, K]`` e4m3 or raw ``uint8`` e4m3 bytes, ``stride(1) == 1``.
        weight_scale: storage of ``scale[n // block_size_y, k // block_size_x]``.
        scale_row_stride: distance between scale rows, default ``ceil(K / block_size_x)``.
        block_size_y / block_size_x: output rows / K columns sharing one scale.
        scale_dtype: ``"e8m0"``, ``"float32"`` or ``"bfloat16"``.
        out: optional ``[N]`` buffer of ``input``'s dtype.
    """
    if not isinstance(input, torch.Tensor):
        raise TypeError("input must be a torch.Tensor")
    if input.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("input must have dtype float16 or bfloat16")
    require_cuda(input, "input")
    weight_view = weight_bytes(weight)
    columns, inner = int(weight_view.shape[0]), int(weight_view.shape[1])
    a = _flatten_vector(input, "input", inner)
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
    result = _vector_output(input, out, columns, input.dtype)
    if columns == 0:
        return result
    scale = weight_scale if weight_scale.is_contiguous() else weight_scale.contiguous()
    ws, nbytes = _workspace("ayk_fp8_weight_only_gemv_workspace_bytes", columns, inner, input.device)
    _lib.call(
        "ayk_fp8_weight_only_gemv", a.data_ptr(), _lib.dtype_code(input.dtype), weight_view.data_ptr(),
        weight_view.stride(0), columns, inner, scale.data_ptr(), _SCALE_CODES[scale_dtype], scale_row_stride,
        block_size_y, block_size_x, result.data_ptr(), _lib.ptr(ws), nbytes, _lib.stream_of(input),
    )
    return result


# ------------------------------------------------------------------ W8A8 block-128
def _blockwise_gemv_fake(
    a: torch.Tensor,
    b: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    return out if out is not None else torch.empty((b.shape[0],), dtype=torch.float32, device=a.device)


@custom_op(name="fp8_blockwise_gemv", fake_impl=_blockwise_gemv_fake, mutates_args=["out"])
def fp8_blockwise_gemv(
    a: torch.Tensor,
    b: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """M == 1 case of ``fp8_blockwise_mm``.

    Args:
        a: ``[K]`` (any shape with K elements) e4m3.
        b: ``[N, K]`` e4m3, ``stride(1) == 1``.
        scale_a: ``[ceil(K / 128)]`` activation scales.
        scale_b: ``[ceil(N / 128), ceil(K / 128)]`` weight scales.
        bias: optional ``[N]``.
        out: optional ``[N]`` buffer (fp32, fp16 or bf16); fp32 when omitted.
    """
    require_tensor(a, "a")
    require_dtype(a, "a", (FP8,))
    require_cuda(a, "a")
    validate_operand(b, "b", dtype=FP8, allow_transposed=False)
    columns, inner = int(b.shape[0]), int(b.shape[1])
    a_vec = _flatten_vector(a, "a", inner)
    scale_k = div_ceil(inner, _BLOCK_K)
    validate_scale(scale_a, "scale_a", a, scale_k)
    validate_block_scale(scale_b, "scale_b", a, (div_ceil(columns, _BLOCK_K), scale_k))
    validate_bias(bias, a, columns)
    dtype = out.dtype if out is not None else torch.float32
    if dtype not in OUTPUT_DTYPES:
        raise TypeError("out must be float16, bfloat16, or float32")
    result = _vector_output(a, out, columns, dtype)
    if columns == 0:
        return result
    sa = scale_a.reshape(-1).expand(scale_k).contiguous() if scale_a.ndim == 0 else scale_a
    ws, nbytes = _workspace("ayk_fp8_blockwise_gemv_workspace_bytes", columns, inner, a.device)
    _lib.call(
        "ayk_fp8_blockwise_gemv", a_vec.data_ptr(), b.data_ptr(), b.stride(0), columns, inner,
        sa.data_ptr(), _lib.dtype_code(sa.dtype), scale_b.data_ptr(), _lib.dtype_code(scale_b.dtype),
        _lib.ptr(bias), _lib.dtype_code(bias.dtype) if bias is not None else 0,
        result.data_ptr(), _lib.dtype_code(result.dtype), _lib.ptr(ws), nbytes, _lib.stream_of(a),
    )
    return result
