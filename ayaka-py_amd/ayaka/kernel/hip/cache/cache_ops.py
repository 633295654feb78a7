"""KV-cache writes and gathers on the gfx950 kernels of ``csrc/kvcache.hip``.

Same operator names, signatures, checks and messages as the reference's
``python/ayaka/kernel/triton/cache/cache_ops.py``:

* ``scatter_cache`` (``ayaka::cache_scatter``, reference :65) -- one plane;
* ``write_kv`` (``ayaka::cache_write_kv``, reference :160) -- the fused K/V write;
* ``gather_cache`` (``ayaka::cache_gather``, reference :230) -- gather, optionally
  dequantizing.

An fp8 cache (``float8_e4m3fn`` / ``float8_e5m2``) stores
``round_to_nearest_even(clamp(x * inverse_scale, -max, max))`` -- the per-tensor static
quantization of ``kvcache/storage/quantization.py:127-212`` -- and a float cache ``x``
cast to its dtype. Caches are ``[pages, page_size, heads, head_dim]``; a slot is
``page * page_size + offset``. Negative slots are skipped (masked padding); the caller
validates the others, as the reference requires. There is no CPU path: the operators
are registered for CUDA (HIP) tensors only, so the dispatcher rejects CPU tensors.
"""

from __future__ import annotations

import math

import torch

from ayaka.kernel.hip import _lib
from ayaka.kernel.ops import custom_op

__all__ = ["gather_cache", "scatter_cache", "write_kv"]

_COMPUTE_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
_FP8_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)


def _require_cuda(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise ValueError("KV cache operands must be on the GPU (this package has no CPU path)")


def _check_scale(*scales: float) -> None:
    if any(not math.isfinite(s) or s <= 0 for s in scales):
        raise ValueError("KV inverse scales must be finite and positive")


def _check_plane(source: torch.Tensor, cache: torch.Tensor, slots: torch.Tensor) -> int:
    """Validate one plane against its cache; returns the row width (heads * head_dim)."""
    if slots.ndim != 1 or slots.dtype != torch.int64 or slots.device != cache.device:
        raise ValueError("KV write slots must be a rank-1 int64 tensor on the cache device")
    if cache.ndim != 4 or tuple(source.shape) != (slots.numel(), *cache.shape[2:]):
        raise ValueError("KV write payload must match the slot count and cache head geometry")
    if not cache.is_contiguous():
        raise ValueError("KV cache pages must flatten without copying")
    if source.dtype not in _COMPUTE_DTYPES or cache.dtype not in (*_COMPUTE_DTYPES, *_FP8_DTYPES):
        raise ValueError("unsupported KV write dtype")
    return math.prod(cache.shape[2:])


def _source_rows(source: torch.Tensor, width: int) -> tuple[torch.Tensor, int]:
    """``source`` as rows of ``width`` contiguous elements and the row stride. Any
    alignment is accepted: the library takes 8-element vector kernels when rows are
    16-byte aligned, per-element kernels otherwise."""
    rows = source.reshape(source.shape[0], width)
    if rows.stride(-1) != 1 or (rows.shape[0] > 1 and rows.stride(0) < width):
        rows = rows.contiguous()
    stride = int(rows.stride(0)) if rows.shape[0] > 1 else width
    return rows, stride


def _launch_write(key, value, key_cache, value_cache, slots, k_inverse, v_inverse, width) -> None:
    k_rows, stride = _source_rows(key, width)
    v_rows = None
    if value is not None:
        v_rows, v_stride = _source_rows(value, width)
        if v_stride != stride:
            k_rows, v_rows, stride = k_rows.contiguous(), v_rows.contiguous(), width
    slots_c = slots.contiguous()
    _lib.call(
        "ayk_kv_cache_write", k_rows.data_ptr(), None if v_rows is None else v_rows.data_ptr(),
        _lib.dtype_code(key.dtype), int(slots_c.numel()), width, stride, key_cache.data_ptr(),
        None if value_cache is None else value_cache.data_ptr(), _lib.dtype_code(key_cache.dtype),
        int(key_cache.shape[0] * key_cache.shape[1]), slots_c.data_ptr(), float(k_inverse), float(v_inverse),
        _lib.stream_of(key_cache),
    )


def _scatter_cache_fake(source, destination, slots, inverse_scale) -> None:
    return None


@custom_op(name="cache_scatter", fake_impl=_scatter_cache_fake, mutates_args=["destination"])
def scatter_cache(source: torch.Tensor, destination: torch.Tensor, slots: torch.Tensor, inverse_scale: float) -> None:
    """Write one plane through validated slots, with static inverse FP8 scale."""
    _require_cuda(source, destination, slots)
    _check_scale(inverse_scale)
    width = _check_plane(source, destination, slots)
    if slots.numel():
        _launch_write(source, None, destination, None, slots, inverse_scale, inverse_scale, width)


def _write_kv_fake(key, value, key_cache, value_cache, slots, k_inverse, v_inverse) -> None:
    return None


@custom_op(name="cache_write_kv", fake_impl=_write_kv_fake, mutates_args=["key_cache", "value_cache"])
def write_kv(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slots: torch.Tensor,
    k_inverse: float,
    v_inverse: float,
) -> None:
    """Fused NHD MHA/GQA write; called once before attention reads the cache."""
    _require_cuda(key, value, key_cache, value_cache, slots)
    _check_scale(k_inverse, v_inverse)
    width = _check_plane(key, key_cache, slots)
    _check_plane(value, value_cache, slots)
    if key_cache.shape != value_cache.shape or key_cache.dtype != value_cache.dtype:
        raise ValueError("KV cache planes must share geometry and dtype")
    if key_cache.device != value_cache.device or key.dtype != value.dtype:
        raise ValueError("KV planes must share cache device and payload dtype")
    if slots.numel():
        _launch_write(key, value, key_cache, value_cache, slots, k_inverse, v_inverse, width)


def _gather_cache_fake(source, slots, destination, scale, dequantize) -> None:
    return None


@custom_op(name="cache_gather", fake_impl=_gather_cache_fake, mutates_args=["destination"])
def gather_cache(source: torch.Tensor, slots: torch.Tensor, destination: torch.Tensor, scale: float, dequantize: bool) -> None:
    """Gather slots (including repeats), optionally dequantizing into the output."""
    _require_cuda(source, slots, destination)
    if source.ndim < 3:
        raise ValueError("KV cache source must be [pages, page_size, ...]")
    width = math.prod(source.shape[2:])
    if slots.ndim != 1 or slots.dtype != torch.int64:
        raise ValueError("gather slots must be a rank-1 int64 tensor")
    if destination.numel() != slots.numel() * width:
        raise ValueError("gather destination must hold one cache row per slot")
    if dequantize and (source.dtype not in _FP8_DTYPES or destination.dtype not in _COMPUTE_DTYPES):
        raise ValueError("dequantize needs an fp8 cache and a float destination")
    if not source.is_contiguous() or not destination.is_contiguous():
        raise ValueError("gather needs a contiguous cache and destination")
    if slots.numel() == 0:
        return
    slots_c = slots.contiguous()
    _lib.call(
        "ayk_kv_cache_gather", source.data_ptr(), _lib.dtype_code(source.dtype), int(source.shape[0] * source.shape[1]),
        width, slots_c.data_ptr(), int(slots_c.numel()), destination.data_ptr(), _lib.dtype_code(destination.dtype),
        float(scale), int(bool(dequantize)), _lib.stream_of(source),
    )
