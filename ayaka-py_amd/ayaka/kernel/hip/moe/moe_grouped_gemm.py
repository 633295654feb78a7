"""MoE FP8 block-128 grouped GEMM on the gfx950 kernel ``fp8_grouped_block_kernel``.

Same function, argument order, checks and messages as the reference's
``kernel/triton/moe/moe_grouped_gemm.py:599`` ``fp8_blockwise_scaled_grouped_mm``
(a signature-compatible stand-in for the CUTLASS MoE op):

    out[m, n] = sum_kb scales_a[m, kb] * scales_b[e][n / 128][kb] * (a[m, kb-block] . b[e][n, kb-block])

for each expert ``e`` over its rows ``[expert_offsets[e], + problem_sizes[e][0])``, each
128-wide K block's partial scaled and added into an fp32 sum that is rounded to the
output dtype once; rows of no expert are left untouched.

The pointer tables (``a_ptrs`` .. ``b_scales_ptrs``) and scale-layout descriptors
(``layout_sfa`` / ``layout_sfb``) are workspaces the reference fills as a side effect
(``get_group_gemm_starts``, :61-135, in its normal and swap-AB flavours); they are
filled here with the same values by device tensor arithmetic, without a host sync.
The kernel itself reads ``problem_sizes`` and ``expert_offsets`` on the device and
derives every operand address from them, so one kernel serves both flavours: swap-AB
is a tiling choice of the CUTLASS kernels that changes the summation order only, and
``swap_ab`` picks the flavour of the tables. ``stride_a/b/c`` must hold the dense
leading dimensions (K, K, N) that the layout checks below already imply; ``workspace``
is accepted for signature compatibility only.
"""

from __future__ import annotations

import torch

from ayaka.kernel.hip import _lib

__all__ = ["fp8_blockwise_scaled_grouped_mm", "get_group_gemm_starts"]

SCALE_BLOCK = 128
# Row count from which the activation scales are handed to the kernel column-major.
COLUMN_MAJOR_SCALES_MIN_ROWS = 4096
_OUT_DTYPES = (torch.bfloat16, torch.float16)


def _check(condition: object, message: str) -> None:
    if not condition:
        raise ValueError(message)


def _same_device(*tensors: torch.Tensor) -> None:
    first = tensors[0].device
    for t in tensors[1:]:
        if t.device != first:
            raise ValueError(f"tensor on {t.device} does not share the device {first} of the other operands")


def _mem_layout_ok(t: torch.Tensor, e: int, rows: int, cols: int) -> bool:
    """``t`` is [e, rows, cols] contiguous, or the [e, cols, rows] transposed view of one."""
    if tuple(t.shape) == (e, rows, cols):
        return t.is_contiguous()
    if tuple(t.shape) == (e, cols, rows):
        return tuple(t.stride()) == (rows * cols, 1, cols)
    return False


def get_group_gemm_starts(expert_offsets, a_ptrs, b_ptrs, out_ptrs, a_scales_ptrs, b_scales_ptrs, a_tensors,
                          b_tensors, out_tensors, a_scales, b_scales, layout_sfa, layout_sfb, problem_sizes,
                          problem_sizes_transpose, transpose: bool = False) -> None:
    """Fill the per-expert device address tables and scale descriptors (reference
    ``moe_grouped_gemm.py:61-135``): normal flavour ``a`` = tokens at ``off * K`` and
    ``b`` = weights at ``e * N * K``; ``transpose`` swaps the two roles (weights become
    the ``a`` operand) and writes the transposed problem sizes. Descriptors are
    ``[rows, k_blocks, 1, k_blocks, rows * k_blocks]`` per expert, rows = tokens (per-row
    scales) or 128-row weight blocks."""
    e_count = expert_offsets.numel()
    if e_count == 0:
        return
    ps = problem_sizes.reshape(-1, 3)[:e_count].to(torch.int64)
    m, n, k = ps[:, 0], ps[:, 1], ps[:, 2]
    e = torch.arange(e_count, device=expert_offsets.device, dtype=torch.int64)
    off = expert_offsets[:e_count].to(torch.int64)
    if transpose:
        problem_sizes_transpose.reshape(-1, 3)[:e_count].copy_(torch.stack([n, m, k], dim=1).to(torch.int32))
        a_stride, b_stride = e * k * n, off * k
        a_scale_stride, b_scale_stride = e * k * n // 128 // 128, off * k // 128
    else:
        a_stride, b_stride = off * k, e * k * n
        a_scale_stride, b_scale_stride = off * k // 128, e * k * n // 128 // 128
    out_bytes = out_tensors.element_size()
    a_ptrs[:e_count].copy_(a_stride + a_tensors.data_ptr())
    b_ptrs[:e_count].copy_(b_stride + b_tensors.data_ptr())
    out_ptrs[:e_count].copy_(off * n * out_bytes + out_tensors.data_ptr())
    a_scales_ptrs[:e_count].copy_(a_scale_stride * 4 + a_scales.data_ptr())
    b_scales_ptrs[:e_count].copy_(b_scale_stride * 4 + b_scales.data_ptr())
    kb, nb = (k + 127) // 128, (n + 127) // 128
    sfa_rows, sfb_rows = (nb, m) if transpose else (m, nb)
    for layout, rows in ((layout_sfa, sfa_rows), (layout_sfb, sfb_rows)):
        desc = torch.stack([rows, kb, torch.ones_like(kb), kb, rows * kb], dim=1).to(torch.int32)
        layout[:e_count, :5].copy_(desc)


def fp8_blockwise_scaled_grouped_mm(
    output: torch.Tensor,
    a_ptrs: torch.Tensor,
    b_ptrs: torch.Tensor,
    out_ptrs: torch.Tensor,
    a_scales_ptrs: torch.Tensor,
    b_scales_ptrs: torch.Tensor,
    a: torch.Tensor,
    b: torch.Tensor,
    scales_a: torch.Tensor,
    scales_b: torch.Tensor,
    stride_a: torch.Tensor,
    stride_b: torch.Tensor,
    stride_c: torch.Tensor,
    layout_sfa: torch.Tensor,
    layout_sfb: torch.Tensor,
    problem_sizes: torch.Tensor,
    expert_offsets: torch.Tensor,
    workspace: torch.Tensor,
    *,
    swap_ab: bool | None = None,
) -> None:
    """Grouped block-128 FP8 GEMM into ``output`` (see the module docstring)."""
    _check(problem_sizes.dim() == 2, "problem_sizes must be 2D tensor")
    _check(problem_sizes.size(1) == 3, "problem_sizes must have shape (num_experts, 3)")
    _check(problem_sizes.size(0) == expert_offsets.size(0), "Number of experts in problem_sizes must match expert_offsets")
    _check(problem_sizes.dtype == torch.int32, "problem_sizes must be int32")
    _check(a.dtype == torch.float8_e4m3fn, "a must be kFloat8_e4m3fn")
    _check(b.dtype == torch.float8_e4m3fn, "b must be kFloat8_e4m3fn")
    _check(output.dtype in _OUT_DTYPES, "output must be bfloat16 or half")
    _check(scales_a.dtype == torch.float32, "scales_a must be float32")
    _check(scales_b.dtype == torch.float32, "scales_b must be float32")
    for name, t in (("stride_a", stride_a), ("stride_b", stride_b), ("stride_c", stride_c)):
        _check(t.dtype == torch.int64, f"{name} must be int64")
        _check(t.dim() == 1, f"{name} must be 1D tensor")
    _check(layout_sfa.dtype == torch.int32, "layout_sfa must be int32")
    _check(layout_sfb.dtype == torch.int32, "layout_sfb must be int32")
    _check(expert_offsets.dtype == torch.int32, "expert_offsets must be int32")
    _check(output.dim() == 2, "output must be 2D tensor")
    _check(a.dim() == 2, "a must be 2D tensor")
    _check(b.dim() == 3, "b must be 3D tensor")
    _check(scales_a.dim() == 2, "scales_a must be 2D tensor")
    _check(scales_b.dim() == 3, "scales_b must be 3D tensor")
    _check(layout_sfa.dim() == 2, "layout_sfa must be 2D tensor")
    _check(layout_sfb.dim() == 2, "layout_sfb must be 2D tensor")
    for name, t in (("a_ptrs", a_ptrs), ("b_ptrs", b_ptrs), ("out_ptrs", out_ptrs), ("a_scales_ptrs", a_scales_ptrs),
                    ("b_scales_ptrs", b_scales_ptrs), ("workspace", workspace)):
        _check(t.dim() == 1, f"{name} must be 1D tensor")
    for t in (output, a, b, scales_a, scales_b, problem_sizes, expert_offsets):
        _check(t.is_cuda, "all tensors must be CUDA tensors")
    _same_device(output, a, b, scales_a, scales_b, problem_sizes, expert_offsets, a_ptrs, b_ptrs, out_ptrs,
                 a_scales_ptrs, b_scales_ptrs, stride_a, stride_b, stride_c, layout_sfa, layout_sfb, workspace)

    num_experts = expert_offsets.size(0)
    m_total, k = a.shape
    n = output.size(1)
    for name, t in (("a_ptrs", a_ptrs), ("b_ptrs", b_ptrs), ("out_ptrs", out_ptrs), ("a_scales_ptrs", a_scales_ptrs),
                    ("b_scales_ptrs", b_scales_ptrs)):
        _check(t.dtype == torch.int64, f"{name} must be int64")
        _check(t.is_contiguous(), f"{name} must be contiguous")
        _check(t.numel() >= num_experts, f"{name} needs num_experts entries")
    for name, t in (("stride_a", stride_a), ("stride_b", stride_b), ("stride_c", stride_c)):
        _check(t.is_contiguous(), f"{name} must be contiguous")
        _check(t.numel() >= num_experts, f"{name} needs num_experts entries")
    _check(problem_sizes.is_contiguous(), "problem_sizes must be contiguous")
    _check(expert_offsets.is_contiguous(), "expert_offsets must be contiguous")
    _check(layout_sfa.is_contiguous() and layout_sfb.is_contiguous(), "layouts must be contiguous")
    _check(output.size(0) == m_total, "output and a must have the same number of rows")
    _check(n % SCALE_BLOCK == 0 and k % SCALE_BLOCK == 0, "N and K must be multiples of 128")
    _check(a.is_contiguous() and output.is_contiguous(), "a and output must be contiguous")
    _check(b.size(0) == num_experts and _mem_layout_ok(b, num_experts, n, k), "b must have memory layout [E][N][K]")
    _check(scales_b.size(0) == num_experts and _mem_layout_ok(scales_b, num_experts, n // 128, k // 128),
           "scales_b must have memory layout [E][N/128][K/128]")
    _check(tuple(scales_a.shape) == (m_total, k // 128) and scales_a.is_contiguous(),
           "scales_a must be a contiguous [M_total, K/128] tensor")
    if num_experts == 0 or m_total == 0:
        return

    swap = (m_total <= 2048) if swap_ab is None else bool(swap_ab)
    with torch.cuda.device(a.device):
        if swap:
            transposed = torch.empty((num_experts, 3), dtype=torch.int32, device=a.device)
            get_group_gemm_starts(expert_offsets, a_ptrs, b_ptrs, out_ptrs, a_scales_ptrs, b_scales_ptrs, b, a,
                                  output, scales_b, scales_a, layout_sfa, layout_sfb, problem_sizes, transposed, True)
        else:
            get_group_gemm_starts(expert_offsets, a_ptrs, b_ptrs, out_ptrs, a_scales_ptrs, b_scales_ptrs, a, b,
                                  output, scales_a, scales_b, layout_sfa, layout_sfb, problem_sizes, problem_sizes,
                                  False)
        # Large batches: experts over the whole K read the activation scales transposed
        # ([K/128, M_total], 32 rows per cache line), copied once here; the same values.
        sa_t = scales_a.t().contiguous() if m_total >= COLUMN_MAJOR_SCALES_MIN_ROWS else None
        _lib.call("ayk_fp8_grouped_blockwise_mm", a.data_ptr(), b.data_ptr(), scales_a.data_ptr(), _lib.ptr(sa_t),
                  scales_b.data_ptr(), problem_sizes.data_ptr(), expert_offsets.data_ptr(), num_experts, m_total, n,
                  k, output.data_ptr(), _lib.dtype_code(output.dtype), _lib.stream_of(output))
