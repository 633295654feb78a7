"""Dynamic and static activation quantizers to OCP e4m3fn, on gfx950 HIP kernels.

Operator set and contracts of the reference
(``python/ayaka/kernel/triton/quant/fp8_quant.py:297-560``):

* ``per_token_quant_fp8(x)`` -- one fp32 scale per token over the whole row;
* ``per_token_group_quant_fp8(x, group_size=128)`` -- one fp32 scale per
  (token, K group); the ``scale_a`` producer of ``fp8_blockwise_mm``;
* ``per_token_group_quant_mxfp8(x, group_size=32)`` -- one UE8M0 code per
  (token, K group), code 0 for an all-zero group;
* ``static_quant_fp8(x, scale, out=None)`` -- one device-resident per-tensor scale.

Every quantizer is bit-exact against the reference's plain-torch formulas: fp32
amax, IEEE division ``x / s``, clamp to +-448, round-to-nearest-even encode. (The
reference's static *kernel* multiplies by ``1/s``; its oracle divides, and the
oracle is the contract followed here.)
"""

import math

import torch

from ayaka.kernel.hip import _lib
from ayaka.kernel.hip._host import fake_tensor, prepare_output, require_cuda, require_dtype, require_tensor
from ayaka.kernel.ops import custom_op

__all__ = [
    "per_token_group_quant_fp8",
    "per_token_group_quant_mxfp8",
    "per_token_quant_fp8",
    "static_quant_fp8",
]

FP8 = torch.float8_e4m3fn
_FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_GROUP = 128
_MX_GROUP = 32


def _validate_input(x: torch.Tensor, name: str) -> None:
    require_tensor(x, name)
    require_dtype(x, name, _FLOAT_DTYPES)
    require_cuda(x, name)
    if x.ndim < 1:
        raise ValueError(f"{name} must have at least one dimension")


def _rows_2d(x: torch.Tensor) -> torch.Tensor:
    k = int(x.shape[-1])
    x2d = x.reshape(-1, k)
    if x2d.stride(-1) != 1 or (x2d.shape[0] > 1 and x2d.stride(0) < k):
        x2d = x2d.contiguous()
    return x2d


def _check_group_size(group_size: int, *, pow2: bool) -> None:
    if isinstance(group_size, bool) or not isinstance(group_size, int):
        raise TypeError("group_size must be an integer")
    if group_size < 1 or (pow2 and group_size & (group_size - 1)):
        raise ValueError("group_size must be a positive power of two" if pow2 else "group_size must be positive")


# ---------------------------------------------------------------- per-token group
def _per_token_group_quant_fake(x: torch.Tensor, group_size: int = _GROUP) -> tuple[torch.Tensor, torch.Tensor]:
    k = x.shape[-1]
    rows = math.prod(x.shape[:-1]) if x.ndim > 1 else 1
    return fake_tensor(x, shape=(rows, k), dtype=FP8), fake_tensor(x, shape=(rows, k // group_size), dtype=torch.float32)


@custom_op(name="per_token_group_quant_fp8", fake_impl=_per_token_group_quant_fake)
def per_token_group_quant_fp8(x: torch.Tensor, group_size: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize ``x`` to e4m3 with one fp32 scale per token per K group.

    Args:
        x: ``[..., K]`` fp16/bf16/fp32 CUDA tensor.
        group_size: K elements per scale; a power of two dividing ``K``.

    Returns:
        ``(x_fp8 [M, K], x_scale [M, K // group_size] fp32)``, ``M = numel // K``.
    """
    _validate_input(x, "x")
    _check_group_size(group_size, pow2=True)
    k = int(x.shape[-1])
    if k % group_size:
        raise ValueError(f"K={k} must be divisible by group_size={group_size}")
    x2d = _rows_2d(x)
    rows = int(x2d.shape[0])
    y = torch.empty((rows, k), dtype=FP8, device=x.device)
    scale = torch.empty((rows, k // group_size), dtype=torch.float32, device=x.device)
    if rows:
        _lib.call("ayk_per_token_group_quant_fp8", x2d.data_ptr(), _lib.dtype_code(x.dtype), rows, k,
                  x2d.stride(0) if rows > 1 else k, group_size, y.data_ptr(), k, scale.data_ptr(), _lib.stream_of(x))
    return y, scale


def _per_token_group_quant_colmajor_fake(x: torch.Tensor, group_size: int = _GROUP) -> tuple[torch.Tensor, torch.Tensor]:
    k = x.shape[-1]
    rows = math.prod(x.shape[:-1]) if x.ndim > 1 else 1
    return fake_tensor(x, shape=(rows, k), dtype=FP8), fake_tensor(x, shape=(k // group_size, rows), dtype=torch.float32)


@custom_op(name="per_token_group_quant_fp8_colmajor", fake_impl=_per_token_group_quant_colmajor_fake)
def per_token_group_quant_fp8_colmajor(x: torch.Tensor, group_size: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """``per_token_group_quant_fp8`` with the scales stored ``[K // group_size, M]``.

    The same codes and scale values, bit for bit; only the scale table is transposed,
    the layout ``fp8_blockwise_mm(..., a_scale_col_major=True)`` reads at one cache line
    per 32 rows. Not part of the reference's operator set (its quantizer writes
    ``[M, K // group_size]`` only); the block-128 linear uses it at prefill sizes.
    """
    _validate_input(x, "x")
    _check_group_size(group_size, pow2=True)
    k = int(x.shape[-1])
    if k % group_size:
        raise ValueError(f"K={k} must be divisible by group_size={group_size}")
    x2d = _rows_2d(x)
    rows = int(x2d.shape[0])
    y = torch.empty((rows, k), dtype=FP8, device=x.device)
    scale = torch.empty((k // group_size, rows), dtype=torch.float32, device=x.device)
    if rows:
        _lib.call("ayk_per_token_group_quant_fp8_strided", x2d.data_ptr(), _lib.dtype_code(x.dtype), rows, k,
                  x2d.stride(0) if rows > 1 else k, group_size, y.data_ptr(), k, scale.data_ptr(), 1, rows,
                  _lib.stream_of(x))
    return y, scale


# ---------------------------------------------------------------- MXFP8
def _per_token_group_quant_mxfp8_fake(x: torch.Tensor, group_size: int = _MX_GROUP) -> tuple[torch.Tensor, torch.Tensor]:
    k = x.shape[-1]
    rows = math.prod(x.shape[:-1]) if x.ndim > 1 else 1
    return fake_tensor(x, shape=(rows, k), dtype=FP8), fake_tensor(x, shape=(rows, k // group_size), dtype=torch.uint8)


@custom_op(name="per_token_group_quant_mxfp8", fake_impl=_per_token_group_quant_mxfp8_fake)
def per_token_group_quant_mxfp8(x: torch.Tensor, group_size: int = 32) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize ``x`` to e4m3 with one UE8M0 scale code per token per K group.

    Returns:
        ``(x_fp8 [M, K], x_scale [M, K // group_size] uint8)``. Code 0 marks an
        all-zero group (decodes to +0.0); codes 1..254 decode to ``2 ** (code - 127)``.
    """
    _validate_input(x, "x")
    _check_group_size(group_size, pow2=False)
    k = int(x.shape[-1])
    if k % group_size:
        raise ValueError(f"K={k} must be divisible by group_size={group_size}")
    x2d = _rows_2d(x)
    rows = int(x2d.shape[0])
    y = torch.empty((rows, k), dtype=FP8, device=x.device)
    scale = torch.empty((rows, k // group_size), dtype=torch.uint8, device=x.device)
    if rows:
        _lib.call("ayk_per_token_group_quant_mxfp8", x2d.data_ptr(), _lib.dtype_code(x.dtype), rows, k,
                  x2d.stride(0) if rows > 1 else k, group_size, y.data_ptr(), k, scale.data_ptr(), _lib.stream_of(x))
    return y, scale


# ---------------------------------------------------------------- rowwise
def _per_token_quant_fake(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    k = x.shape[-1]
    rows = math.prod(x.shape[:-1]) if x.ndim > 1 else 1
    return fake_tensor(x, shape=(rows, k), dtype=FP8), fake_tensor(x, shape=(rows,), dtype=torch.float32)


@custom_op(name="per_token_quant_fp8", fake_impl=_per_token_quant_fake)
def per_token_quant_fp8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize ``x`` to e4m3 with one fp32 scale per token (any ``K >= 1``).

    Returns:
        ``(x_fp8 [M, K], x_scale [M] fp32)``.
    """
    _validate_input(x, "x")
    k = int(x.shape[-1])
    if k < 1:
        raise ValueError("x must have a positive last dimension")
    x2d = _rows_2d(x)
    rows = int(x2d.shape[0])
    y = torch.empty((rows, k), dtype=FP8, device=x.device)
    scale = torch.empty((rows,), dtype=torch.float32, device=x.device)
    if rows:
        _lib.call("ayk_per_token_quant_fp8", x2d.data_ptr(), _lib.dtype_code(x.dtype), rows, k,
                  x2d.stride(0) if rows > 1 else k, y.data_ptr(), k, scale.data_ptr(), _lib.stream_of(x))
    return y, scale


# ---------------------------------------------------------------- static
def _static_quant_fake(x: torch.Tensor, scale: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    return out if out is not None else fake_tensor(x, dtype=FP8)


@custom_op(name="static_quant_fp8", fake_impl=_static_quant_fake, mutates_args=["out"])
def static_quant_fp8(x: torch.Tensor, scale: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """Quantize ``x`` to e4m3 under one device-resident per-tensor ``scale``.

    The scale is read by the kernel, never on the host, so the op is graph-capture
    safe. Returns ``out`` when given (same shape as ``x``, e4m3).
    """
    _validate_input(x, "x")
    if not isinstance(scale, torch.Tensor):
        raise TypeError("scale must be a torch.Tensor")
    require_cuda(scale, "scale")
    if scale.numel() != 1:
        raise ValueError("scale must contain exactly one element")
    if scale.dtype not in _FLOAT_DTYPES:
        raise TypeError("scale must have dtype float16, bfloat16, or float32")
    result = prepare_output(x, out, dtype=FP8, name="out", like_name="x")
    if x.numel() == 0:
        return result
    x_flat = x.reshape(-1)
    if not x_flat.is_contiguous():
        x_flat = x_flat.contiguous()
    target = result if result.is_contiguous() else torch.empty_like(result)
    _lib.call("ayk_static_quant_fp8", x_flat.data_ptr(), _lib.dtype_code(x.dtype), x_flat.numel(),
              scale.data_ptr(), _lib.dtype_code(scale.dtype), target.data_ptr(), _lib.stream_of(x))
    if target is not result:
        result.copy_(target)
    return result
