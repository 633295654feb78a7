"""gfx950 HIP implementation of the ``torch.ops.ayaka`` FP8 linear operators.

Importing this package loads ``libayaka_fp8.so`` lazily (first call) and registers
every operator under the reference's names and schemas.
"""

from ayaka.kernel.hip.cache.cache_ops import gather_cache, scatter_cache, write_kv
from ayaka.kernel.hip.gemm.fp8_gemm import fp8_blockwise_mm, fp8_scaled_mm
from ayaka.kernel.hip.gemm.fp8_gemv import fp8_blockwise_gemv, fp8_weight_only_gemv
from ayaka.kernel.hip.gemm.fp8_linear import fp8_block_linear, fp8_pertensor_linear, fp8_rowwise_linear
from ayaka.kernel.hip.gemm.fp8_mxfp8_gemm import mxfp8_scaled_mm
from ayaka.kernel.hip.gemm.fp8_w8a16_gemm import fp8_matmul_channelwise, fp8_weight_only_gemm
from ayaka.kernel.hip.gemm.int8_gemm import int8_scaled_mm
from ayaka.kernel.hip.moe.moe_grouped_gemm import fp8_blockwise_scaled_grouped_mm
from ayaka.kernel.hip.quant.fp8_quant import (
    per_token_group_quant_fp8,
    per_token_group_quant_mxfp8,
    per_token_quant_fp8,
    static_quant_fp8,
)

__all__ = [
    "fp8_block_linear",
    "fp8_blockwise_gemv",
    "fp8_blockwise_mm",
    "fp8_blockwise_scaled_grouped_mm",
    "fp8_matmul_channelwise",
    "fp8_pertensor_linear",
    "fp8_rowwise_linear",
    "fp8_scaled_mm",
    "fp8_weight_only_gemm",
    "fp8_weight_only_gemv",
    "gather_cache",
    "int8_scaled_mm",
    "mxfp8_scaled_mm",
    "per_token_group_quant_fp8",
    "per_token_group_quant_mxfp8",
    "per_token_quant_fp8",
    "scatter_cache",
    "static_quant_fp8",
    "write_kv",
]
