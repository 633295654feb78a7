"""INT8 scaled GEMM on the gfx950 int8 MFMA kernels.

``int8_scaled_mm`` -- ``(a @ b) * scale_a * scale_b + bias`` for int8 operands with
int32 accumulation (``v_mfma_i32_32x32x32_i8``) and an fp32 epilogue, reference
``python/ayaka/kernel/triton/gemm/int8_gemm.py:134`` (oracle
``kernel/triton/reference/gemm.py:192-211``). The kernels are the fp8 GEMM's tiles with
the int8 matrix instruction; the per-row / per-column scales, the bias and the output
cast are fused into their epilogue.
"""

import torch

from ayaka.kernel.hip import _lib
from ayaka.kernel.hip._common import OUTPUT_DTYPES, validate_bias, validate_operand, validate_scale
from ayaka.kernel.hip._host import fake_tensor, prepare_output, require_last_dim_stride1
from ayaka.kernel.hip.gemm.fp8_gemm import kernel_operand
from ayaka.kernel.ops import custom_op
from ayaka.utils.math_utils import validate_output_dtype

__all__ = ["int8_scaled_mm"]


def _row_stride(t: torch.Tensor) -> int:
    return int(t.stride(0)) if t.shape[0] > 1 else int(t.shape[1])


def _int8_scaled_mm_fake(a, b, scale_a, scale_b, bias=None, out=None, out_dtype=torch.bfloat16):
    return out if out is not None else fake_tensor(a, shape=(a.shape[0], b.shape[1]), dtype=out_dtype)


@custom_op(name="int8_scaled_mm", fake_impl=_int8_scaled_mm_fake, mutates_args=["out"])
def int8_scaled_mm(
    a: torch.Tensor,
    b: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    out_dtype: torch.dtype = torch.bfloat16,
) -> torch.Tensor:
    """``(a @ b) * scale_a * scale_b + bias`` for INT8 operands.

    Args:
        a: ``[M, K]`` ``torch.int8`` with ``stride(1) == 1`` and ``K`` a multiple of 16.
        b: ``[K, N]`` ``torch.int8``, or the transposed view of an ``[N, K]`` weight
            (``stride(0) == 1``).
        scale_a: ``[M]`` float32 scale applied to the int32 accumulator.
        scale_b: ``[N]`` float32 scale.
        bias: optional ``[N]`` (fp32, fp16 or bf16), added in fp32.
        out: optional ``[M, N]`` fp32 / fp16 / bf16 buffer; ``out_dtype`` is used only when
            it is omitted.

    Raises:
        TypeError: non-int8 operands, non-float32 scales, an unsupported bias dtype.
        ValueError: mismatched shapes, K not a multiple of 16, a bad ``out`` or ``out_dtype``.
    """
    validate_operand(a, "a", dtype=torch.int8, allow_transposed=False)
    validate_operand(b, "b", dtype=torch.int8, allow_transposed=True)
    if a.shape[1] != b.shape[0]:
        raise ValueError(f"inner dimensions do not match: a is {tuple(a.shape)}, b is {tuple(b.shape)}")
    rows, inner, columns = int(a.shape[0]), int(a.shape[1]), int(b.shape[1])
    if inner % 16:
        raise ValueError("K must be a multiple of 16, matching the CUDA API")
    validate_scale(scale_a, "scale_a", a, rows, dtypes=(torch.float32,), scalar_ok=False)
    validate_scale(scale_b, "scale_b", a, columns, dtypes=(torch.float32,), scalar_ok=False)
    validate_bias(bias, a, columns)
    if out is None:
        validate_output_dtype(out_dtype)
    result = prepare_output(a, out, shape=(rows, columns), dtype=out_dtype, dtypes=OUTPUT_DTYPES, like_name="a")
    require_last_dim_stride1(result, "out")
    if rows == 0 or columns == 0:
        return result
    a_k = kernel_operand(a)
    w_k = kernel_operand(b.t())
    inner = int(a_k.shape[1])
    # split-K partials for launches short of one round of tiles
    nbytes = _lib.query("ayk_int8_scaled_mm_workspace_bytes", rows, columns, inner)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=a.device) if nbytes else None
    _lib.call(
        "ayk_int8_scaled_mm", a_k.data_ptr(), _row_stride(a_k), w_k.data_ptr(), _row_stride(w_k),
        rows, columns, inner, scale_a.data_ptr(), scale_b.data_ptr(),
        _lib.ptr(bias), _lib.dtype_code(bias.dtype) if bias is not None else 0,
        result.data_ptr(), _lib.dtype_code(result.dtype), _row_stride(result),
        _lib.ptr(ws), nbytes, _lib.stream_of(a),
    )
    return result
