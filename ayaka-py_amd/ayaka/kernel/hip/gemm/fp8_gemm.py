"""W8A8 FP8 GEMM operators on the gfx950 fp8 MFMA kernel.

* ``fp8_scaled_mm`` -- ``(a @ b) * scale_a * scale_b + bias`` (per-tensor / rowwise),
  reference ``python/ayaka/kernel/triton/gemm/fp8_gemm.py:246``;
* ``fp8_blockwise_mm`` -- 128x128 block-scaled product, reference ``fp8_gemm.py:370``.

Both accumulate in fp32 on ``v_mfma_scale_f32_32x32x64_f8f6f4`` and round once to the
output dtype (fp32 by default, as in the reference). ``backend`` is accepted for
signature compatibility; there is one implementation, so ``"triton"``, ``"auto"``
and ``"cublaslt"`` all run the HIP kernel.
"""

import torch

from ayaka.kernel.hip import _lib
from ayaka.kernel.hip._common import (
    FP8,
    OUTPUT_DTYPES,
    SCALE_BLOCK_K,
    validate_bias,
    validate_block_scale,
    validate_operand,
    validate_scale,
)
from ayaka.kernel.hip._host import prepare_output, require_last_dim_stride1
from ayaka.kernel.ops import custom_op
from ayaka.utils.math_utils import div_ceil

__all__ = ["fp8_blockwise_mm", "fp8_rowwise_linear_small", "fp8_scaled_mm"]

_BACKENDS = ("triton", "auto", "cublaslt")


def _mm_output(a: torch.Tensor, out: torch.Tensor | None, rows: int, columns: int) -> torch.Tensor:
    result = prepare_output(a, out, shape=(rows, columns), dtype=torch.float32, dtypes=OUTPUT_DTYPES, like_name="a")
    require_last_dim_stride1(result, "out")
    return result


def kernel_operand(t: torch.Tensor) -> torch.Tensor:
    """A ``[rows, K]`` e4m3 operand in the layout the MFMA kernels load.

    The kernels read 16-byte vectors, so K, the row stride and the base address
    must be multiples of 16 bytes. Anything else is copied into a zero-padded
    ``[rows, ceil(K/16)*16]`` buffer (zeros contribute nothing to the dot).
    """
    rows, k = t.shape
    if t.stride(1) == 1 and k % 16 == 0 and (rows <= 1 or t.stride(0) % 16 == 0) and t.data_ptr() % 16 == 0:
        return t
    padded = torch.zeros((rows, div_ceil(k, 16) * 16), dtype=t.dtype, device=t.device)
    padded[:, :k] = t
    return padded


def _row_stride(t: torch.Tensor) -> int:
    return int(t.stride(0)) if t.shape[0] > 1 else int(t.shape[1])


# ------------------------------------------------------------------ per-tensor / rowwise
def _fp8_scaled_mm_fake(a, b, scale_a, scale_b, bias=None, out=None, backend="triton"):
    return out if out is not None else torch.empty((a.shape[0], b.shape[1]), dtype=torch.float32, device=a.device)


@custom_op(name="fp8_scaled_mm", fake_impl=_fp8_scaled_mm_fake, mutates_args=["out"])
def fp8_scaled_mm(
    a: torch.Tensor,
    b: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    backend: str = "triton",
) -> torch.Tensor:
    """``(a @ b) * scale_a * scale_b + bias`` for e4m3 operands.

    Args:
        a: ``[M, K]`` e4m3, ``stride(1) == 1``.
        b: ``[K, N]`` e4m3, or the ``[N, K]`` weight viewed transposed (``stride(0) == 1``).
        scale_a: scalar or ``[M]``; scale_b: scalar or ``[N]`` (fp32/fp16/bf16).
        bias: optional ``[N]``, added in fp32.
        out: optional ``[M, N]`` fp32/fp16/bf16 buffer; fp32 is allocated when omitted.
        backend: accepted for compatibility, see module docstring.
    """
    validate_operand(a, "a", dtype=FP8, allow_transposed=False)
    validate_operand(b, "b", dtype=FP8, allow_transposed=True)
    if a.shape[1] != b.shape[0]:
        raise ValueError(f"inner dimensions do not match: a is {tuple(a.shape)}, b is {tuple(b.shape)}")
    rows, inner, columns = int(a.shape[0]), int(a.shape[1]), int(b.shape[1])
    validate_scale(scale_a, "scale_a", a, rows)
    validate_scale(scale_b, "scale_b", a, columns)
    validate_bias(bias, a, columns)
    if backend not in _BACKENDS:
        raise ValueError(f"backend must be one of {_BACKENDS}, got {backend!r}")
    result = _mm_output(a, out, rows, columns)
    if rows == 0 or columns == 0:
        return result
    a_k = kernel_operand(a)
    w_k = kernel_operand(b.t())
    inner = int(a_k.shape[1])
    # split-K partials for launches short of one round of tiles (torch's allocator: the
    # graph pool under capture)
    nbytes = _lib.query("ayk_fp8_scaled_mm_workspace_bytes", rows, columns, inner)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=a.device) if nbytes else None
    _lib.call(
        "ayk_fp8_scaled_mm", a_k.data_ptr(), _row_stride(a_k), w_k.data_ptr(), _row_stride(w_k),
        rows, columns, inner,
        scale_a.data_ptr(), _lib.dtype_code(scale_a.dtype), int(scale_a.ndim != 0),
        scale_b.data_ptr(), _lib.dtype_code(scale_b.dtype), int(scale_b.ndim != 0),
        _lib.ptr(bias), _lib.dtype_code(bias.dtype) if bias is not None else 0,
        result.data_ptr(), _lib.dtype_code(result.dtype), _row_stride(result),
        _lib.ptr(ws), nbytes, _lib.stream_of(a),
    )
    return result


# ------------------------------------------------------------------ fused small batch
_SMALL_ROWS = (2, 8)
_SMALL_WEIGHT_BYTES = 1 << 24


def rowwise_small_applies(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor) -> bool:
    """Whether ``fp8_rowwise_linear_small`` takes this product: 2 to 8 rows, a weight of at
    most 2^24 bytes with 16-byte rows, an fp32 scalar or ``[N]`` weight scale, and rows of
    x that the kernel can stage in LDS (``M * K <= 64 KiB``) with 16-byte loads. Shapes,
    dtypes and strides only (traceable); base addresses are checked by the op."""
    rows, k = int(x.shape[0]), int(x.shape[1])
    n = int(weight.shape[0])
    return (_SMALL_ROWS[0] <= rows <= _SMALL_ROWS[1] and n * k <= _SMALL_WEIGHT_BYTES and k % 16 == 0
            and rows * k <= 64 * 1024 and x.dtype in (torch.bfloat16, torch.float16, torch.float32)
            and x.stride(1) == 1 and (x.stride(0) * x.element_size()) % 16 == 0
            and weight.dtype == FP8 and weight.stride(1) == 1 and weight.stride(0) % 16 == 0
            and weight_scale.dtype == torch.float32 and weight_scale.numel() in (1, n) and weight_scale.is_contiguous())


def _fp8_rowwise_linear_small_fake(x, weight, weight_scale, bias=None):
    return torch.empty((x.shape[0], weight.shape[0]), dtype=x.dtype, device=x.device)


@custom_op(name="fp8_rowwise_linear_small", fake_impl=_fp8_rowwise_linear_small_fake)
def fp8_rowwise_linear_small(
    x: torch.Tensor,
    weight: torch.Tensor,
    weight_scale: torch.Tensor,
    bias: torch.Tensor | None = None,
) -> torch.Tensor:
    """Per-token quantization of ``x`` and the rowwise product in one launch, for 2 to 8 rows.

    The result equals ``fp8_scaled_mm(*per_token_quant_fp8(x), weight.t(), ...)`` (the
    reference's ``fp8_rowwise_linear`` at ``fp8_linear.py:168``) bit for bit; the two
    launches become one. Not part of the reference's operator set; ``fp8_rowwise_linear``
    uses it where ``rowwise_small_applies`` holds.

    Args:
        x: ``[M, K]`` bf16 / fp16 / fp32; weight: ``[N, K]`` e4m3; weight_scale: fp32
        scalar or ``[N]``; bias: optional ``[N]``. Returns ``[M, N]`` in ``x``'s dtype.
    """
    if not rowwise_small_applies(x, weight, weight_scale):
        raise ValueError("fp8_rowwise_linear_small: shape, dtype or layout outside its contract")
    validate_bias(bias, x, int(weight.shape[0]))
    rows, k, n = int(x.shape[0]), int(x.shape[1]), int(weight.shape[0])
    if x.data_ptr() % 16 or weight.data_ptr() % 16:  # views at odd offsets: the two launches
        from ayaka.kernel.hip.quant.fp8_quant import per_token_quant_fp8

        q, s = per_token_quant_fp8(x)
        return fp8_scaled_mm(q, weight.t(), s, weight_scale, bias, out=torch.empty((rows, n), dtype=x.dtype, device=x.device))
    out = torch.empty((rows, n), dtype=x.dtype, device=x.device)
    _lib.call(
        "ayk_fp8_rowwise_linear_small", x.data_ptr(), _lib.dtype_code(x.dtype), int(x.stride(0)), rows,
        weight.data_ptr(), int(weight.stride(0)), n, k, weight_scale.data_ptr(), int(weight_scale.numel() != 1),
        _lib.ptr(bias), _lib.dtype_code(bias.dtype) if bias is not None else 0,
        out.data_ptr(), _lib.dtype_code(out.dtype), n, _lib.stream_of(x),
    )
    return out


# ------------------------------------------------------------------ block-128
def _fp8_blockwise_mm_fake(a, b, scale_a, scale_b, bias=None, out=None, a_scale_col_major=False):
    return out if out is not None else torch.empty((a.shape[0], b.shape[0]), dtype=torch.float32, device=a.device)


@custom_op(name="fp8_blockwise_mm", fake_impl=_fp8_blockwise_mm_fake, mutates_args=["out"])
def fp8_blockwise_mm(
    a: torch.Tensor,
    b: torch.Tensor,
    scale_a: torch.Tensor,
    scale_b: torch.Tensor,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    a_scale_col_major: bool = False,
) -> torch.Tensor:
    """``sum_kb (a[:, kb] @ b[:, kb]^T) * scale_a[m, kb] * scale_b[n // 128, kb] + bias``.

    Args:
        a: ``[M, K]`` e4m3; b: ``[N, K]`` e4m3 weight, both ``stride(1) == 1``.
        scale_a: ``[M, ceil(K/128)]`` (or ``[ceil(K/128), M]`` with ``a_scale_col_major``).
        scale_b: ``[ceil(N/128), ceil(K/128)]``.
        bias: optional ``[N]``; out: optional ``[M, N]`` fp32/fp16/bf16 (fp32 default).
    """
    validate_operand(a, "a", dtype=FP8, allow_transposed=False)
    validate_operand(b, "b", dtype=FP8, allow_transposed=False)
    if a.shape[1] != b.shape[1]:
        raise ValueError(f"inner dimensions do not match: a is {tuple(a.shape)}, b is {tuple(b.shape)}")
    rows, inner, columns = int(a.shape[0]), int(a.shape[1]), int(b.shape[0])
    scale_k = div_ceil(inner, SCALE_BLOCK_K)
    validate_block_scale(scale_a, "scale_a", a, (scale_k, rows) if a_scale_col_major else (rows, scale_k))
    validate_block_scale(scale_b, "scale_b", a, (div_ceil(columns, SCALE_BLOCK_K), scale_k))
    validate_bias(bias, a, columns)
    result = _mm_output(a, out, rows, columns)
    if rows == 0 or columns == 0:
        return result
    a_k = kernel_operand(a)
    w_k = kernel_operand(b)
    inner = int(a_k.shape[1])
    # split-K partials for launches with too few tiles (torch's allocator: the graph pool
    # under capture)
    nbytes = _lib.query("ayk_fp8_blockwise_mm_workspace_bytes", rows, columns, inner)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=a.device) if nbytes else None
    _lib.call(
        "ayk_fp8_blockwise_mm", a_k.data_ptr(), _row_stride(a_k), w_k.data_ptr(), _row_stride(w_k),
        rows, columns, inner,
        scale_a.data_ptr(), _lib.dtype_code(scale_a.dtype), int(bool(a_scale_col_major)),
        scale_b.data_ptr(), _lib.dtype_code(scale_b.dtype),
        _lib.ptr(bias), _lib.dtype_code(bias.dtype) if bias is not None else 0,
        result.data_ptr(), _lib.dtype_code(result.dtype), _row_stride(result),
        _lib.ptr(ws), nbytes, _lib.stream_of(a),
    )
    return result
