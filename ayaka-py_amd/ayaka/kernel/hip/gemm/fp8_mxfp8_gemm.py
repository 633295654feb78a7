"""MXFP8 GEMM operator: e4m3 operands with UE8M0 scales per 32-wide K group.

Reference ``python/ayaka/kernel/triton/gemm/fp8_mxfp8_gemm.py:163``. For M > 1 the
per-group scales are applied inside gfx950's scaled MFMA
(``v_mfma_scale_f32_32x32x64_f8f6f4``), which takes exactly one UE8M0 code per 32
K elements of each row; M == 1 runs the decode GEMV. Bias is added in fp32 before
the single rounding to the output dtype, as in the reference.

One hardware difference is documented and tested: the MFMA decodes a *weight*
scale code 0 as 2^-127 where the reference decodes it as 0; the difference is below
any output rounding unless the weights themselves are huge.
"""

import torch

from ayaka.kernel.hip import _lib
from ayaka.kernel.hip._common import FP8, OUTPUT_DTYPES, validate_bias, validate_operand
from ayaka.kernel.hip._host import prepare_output, require_last_dim_stride1, require_tensor
from ayaka.kernel.hip.gemm.fp8_gemm import kernel_operand
from ayaka.kernel.ops import custom_op

__all__ = ["mxfp8_scaled_mm"]

MX_BLOCK = 32


def _validate_mx_scale(scale: torch.Tensor, name: str, reference: torch.Tensor, shape: tuple[int, int]) -> None:
    require_tensor(scale, name)
    if scale.device != reference.device:
        raise ValueError(f"{name} and a must be on the same CUDA device")
    if scale.dtype is not torch.uint8:
        raise TypeError("scale must have dtype uint8 (UE8M0)")
    if tuple(scale.shape) != shape:
        raise ValueError(f"{name} must have shape {shape}")
    if not scale.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _mxfp8_scaled_mm_fake(a, a_scale, weight, weight_scale, bias=None, out=None):
    return out if out is not None else torch.empty((a.shape[0], weight.shape[0]), dtype=torch.float32, device=a.device)


@custom_op(name="mxfp8_scaled_mm", fake_impl=_mxfp8_scaled_mm_fake, mutates_args=["out"])
def mxfp8_scaled_mm(
    a: torch.Tensor,
    a_scale: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``(a @ weight^T)`` with per-32 UE8M0 scales on both operands.

    Args:
        a: ``[M, K]`` e4m3; a_scale: ``[M, K // 32]`` uint8.
        weight: ``[N, K]`` e4m3; weight_scale: ``[N, K // 32]`` uint8.
        bias: optional ``[N]`` (added in fp32); out: optional ``[M, N]`` (fp32 default).
    """
    validate_operand(a, "a", dtype=FP8, allow_transposed=False)
    validate_operand(weight, "weight", dtype=FP8, allow_transposed=False)
    if a.shape[1] != weight.shape[1]:
        raise ValueError(f"inner dimensions do not match: a is {tuple(a.shape)}, weight is {tuple(weight.shape)}")
    rows, inner, columns = int(a.shape[0]), int(a.shape[1]), int(weight.shape[0])
    if inner % MX_BLOCK:
        raise ValueError(f"K={inner} must be a multiple of the MXFP8 group size 32")
    scale_k = inner // MX_BLOCK
    _validate_mx_scale(a_scale, "a_scale", a, (rows, scale_k))
    _validate_mx_scale(weight_scale, "weight_scale", a, (columns, scale_k))
    validate_bias(bias, a, columns)
    result = prepare_output(a, out, shape=(rows, columns), dtype=torch.float32, dtypes=OUTPUT_DTYPES, like_name="a")
    require_last_dim_stride1(result, "out")
    if rows == 0 or columns == 0:
        return result
    a_k = kernel_operand(a)
    w_k = kernel_operand(weight)
    ldo = int(result.stride(0)) if rows > 1 else columns
    # split-K partials for launches short of one round of tiles (torch's allocator: the
    # graph pool under capture)
    nbytes = _lib.query("ayk_mxfp8_scaled_mm_workspace_bytes", rows, columns, inner)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=a.device) if nbytes else None
    _lib.call(
        "ayk_mxfp8_scaled_mm", a_k.data_ptr(), int(a_k.stride(0)) if rows > 1 else inner,
        a_scale.data_ptr(), scale_k, w_k.data_ptr(), int(w_k.stride(0)) if columns > 1 else inner,
        weight_scale.data_ptr(), scale_k, rows, columns, inner,
        _lib.ptr(bias), _lib.dtype_code(bias.dtype) if bias is not None else 0,
        result.data_ptr(), _lib.dtype_code(result.dtype), ldo, _lib.ptr(ws), nbytes, _lib.stream_of(a),
    )
    return result
