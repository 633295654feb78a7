"""ctypes binding of ``libayaka_fp8.so`` (declared in ``include/ayaka_fp8.h``).

The library is built in-tree by ``ayaka-py_amd/build_ext.py``. Loading fails loudly:
there is no CPU or Python fallback for any operator of this package, so a missing
or stale library raises :class:`~ayaka.utils.import_utils.CapabilityError`.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
import threading
from typing import Any

import torch

from ayaka.utils.import_utils import CapabilityError

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libayaka_fp8.so"

# ayk_dtype values (include/ayaka_fp8.h)
AYK_F32 = 0
AYK_F16 = 1
AYK_BF16 = 2
AYK_E4M3 = 3
AYK_U8 = 4
AYK_E5M2 = 5

# ayk_status values
AYK_OK = 0
AYK_EINVAL = 1
AYK_EARCH = 2
AYK_ELAUNCH = 3
AYK_EWORKSPACE = 4

_DTYPE_CODES: dict[torch.dtype, int] = {
    torch.float32: AYK_F32,
    torch.float16: AYK_F16,
    torch.bfloat16: AYK_BF16,
    torch.float8_e4m3fn: AYK_E4M3,
    torch.uint8: AYK_U8,
    torch.float8_e5m2: AYK_E5M2,
}

_p = ctypes.c_void_p
_i = ctypes.c_int
_l = ctypes.c_int64
_z = ctypes.c_size_t
_f = ctypes.c_float

#: name -> argtypes (restype int unless listed in _RESTYPES)
SIGNATURES: dict[str, list[Any]] = {
    "ayk_last_error": [],
    "ayk_last_plan": [],
    "ayk_abi_version": [],
    "ayk_device_supported": [_i],
    "ayk_per_token_quant_fp8": [_p, _i, _l, _l, _l, _p, _l, _p, _p],
    "ayk_per_token_group_quant_fp8": [_p, _i, _l, _l, _l, _l, _p, _l, _p, _p],
    "ayk_fp8_rowwise_linear_small": [_p, _i, _l, _l, _p, _l, _l, _l, _p, _i, _p, _i, _p, _i, _l, _p],
    "ayk_per_token_group_quant_fp8_strided": [_p, _i, _l, _l, _l, _l, _p, _l, _p, _l, _l, _p],
    "ayk_per_token_group_quant_mxfp8": [_p, _i, _l, _l, _l, _l, _p, _l, _p, _p],
    "ayk_static_quant_fp8": [_p, _i, _l, _p, _i, _p, _p],
    "ayk_fp8_scaled_mm": [_p, _l, _p, _l, _l, _l, _l, _p, _i, _i, _p, _i, _i, _p, _i, _p, _i, _l, _p, _z, _p],
    "ayk_fp8_scaled_mm_workspace_bytes": [_l, _l, _l],
    "ayk_fp8_blockwise_mm": [_p, _l, _p, _l, _l, _l, _l, _p, _i, _i, _p, _i, _p, _i, _p, _i, _l, _p, _z, _p],
    "ayk_fp8_blockwise_mm_workspace_bytes": [_l, _l, _l],
    "ayk_fp8_grouped_blockwise_mm": [_p, _p, _p, _p, _p, _p, _p, _l, _l, _l, _l, _p, _i, _p],
    "ayk_int8_scaled_mm": [_p, _l, _p, _l, _l, _l, _l, _p, _p, _p, _i, _p, _i, _l, _p, _z, _p],
    "ayk_int8_scaled_mm_workspace_bytes": [_l, _l, _l],
    "ayk_kv_cache_write": [_p, _p, _i, _l, _l, _l, _p, _p, _i, _l, _p, _f, _f, _p],
    "ayk_kv_cache_gather": [_p, _i, _l, _l, _p, _l, _p, _i, _f, _i, _p],
    "ayk_mxfp8_scaled_mm": [_p, _l, _p, _l, _p, _l, _p, _l, _l, _l, _l, _p, _i, _p, _i, _l, _p, _z, _p],
    "ayk_mxfp8_scaled_mm_workspace_bytes": [_l, _l, _l],
    "ayk_fp8_weight_only_gemv": [_p, _i, _p, _l, _l, _l, _p, _i, _l, _l, _l, _p, _p, _z, _p],
    "ayk_fp8_weight_only_gemv_workspace_bytes": [_l, _l],
    "ayk_fp8_weight_only_gemv_static": [_p, _i, _p, _l, _l, _l, _p, _i, _l, _l, _l, _p, _p],
    "ayk_fp8_weight_only_gemv_static_max_bytes": [],
    "ayk_fp8_weight_only_gemm": [_p, _i, _l, _l, _p, _l, _l, _l, _p, _i, _l, _l, _l, _p, _l, _p, _z, _p],
    "ayk_fp8_weight_only_gemm_workspace_bytes": [_l, _l, _l, _l],
    "ayk_fp8_blockwise_gemv": [_p, _p, _l, _l, _l, _p, _i, _p, _i, _p, _i, _p, _i, _p, _z, _p],
    "ayk_fp8_blockwise_gemv_workspace_bytes": [_l, _l],
}
_RESTYPES: dict[str, Any] = {
    "ayk_last_error": ctypes.c_char_p,
    "ayk_last_plan": ctypes.c_char_p,
    "ayk_fp8_weight_only_gemv_workspace_bytes": _z,
    "ayk_fp8_blockwise_gemv_workspace_bytes": _z,
    "ayk_fp8_blockwise_mm_workspace_bytes": _z,
    "ayk_fp8_scaled_mm_workspace_bytes": _z,
    "ayk_int8_scaled_mm_workspace_bytes": _z,
    "ayk_mxfp8_scaled_mm_workspace_bytes": _z,
    "ayk_fp8_weight_only_gemm_workspace_bytes": _z,
    "ayk_fp8_weight_only_gemv_static_max_bytes": _z,
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load_library(path: str | os.PathLike[str] | None = None) -> ctypes.CDLL:
    """Load (once) and return the C-ABI library with typed prototypes."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        target = pathlib.Path(path) if path is not None else LIB_PATH
        if not target.exists():
            raise CapabilityError(
                "ayaka.kernel.hip",
                detail=f"{target} is not built",
                remedy="run `python ayaka-py_amd/build_ext.py` (hipcc --offload-arch=gfx950)",
            )
        lib = ctypes.CDLL(str(target))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, ctypes.c_int)
        if path is None:
            _lib = lib
        return lib


def dtype_code(dtype: torch.dtype) -> int:
    """ayk_dtype code of a torch dtype."""
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"dtype {dtype} has no ayk_dtype code") from None


def ptr(t: torch.Tensor | None) -> int | None:
    """Raw device pointer of a tensor (None passes NULL)."""
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    """Handle of the current torch stream on ``t``'s device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def call(name: str, *args: Any) -> None:
    """Call a status-returning entry point, mapping failures to Python errors.

    ``AYK_EARCH`` becomes :class:`CapabilityError`; ``AYK_EINVAL`` becomes
    ``ValueError``; every other failure ``RuntimeError``.
    """
    lib = load_library()
    status = getattr(lib, name)(*args)
    if status == AYK_OK:
        return
    message = (lib.ayk_last_error() or b"").decode("utf-8", "replace")
    if status == AYK_EARCH:
        raise CapabilityError(
            name.removeprefix("ayk_"),
            detail=message,
            remedy="run on an MI355X (gfx950) GPU",
        )
    if status == AYK_EINVAL:
        raise ValueError(message)
    raise RuntimeError(f"{name} failed ({status}): {message}")


def last_plan() -> str:
    """The kernels (and K split) of the last GEMM launch on this thread."""
    return (load_library().ayk_last_plan() or b"").decode("utf-8", "replace")


def query(name: str, *args: Any) -> int:
    """Call a size-returning entry point."""
    return int(getattr(load_library(), name)(*args))
