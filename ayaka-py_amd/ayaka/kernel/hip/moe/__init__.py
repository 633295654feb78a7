"""MoE FP8 operators on the gfx950 kernels."""

from ayaka.kernel.hip.moe.moe_grouped_gemm import fp8_blockwise_scaled_grouped_mm, get_group_gemm_starts

__all__ = ["fp8_blockwise_scaled_grouped_mm", "get_group_gemm_starts"]
