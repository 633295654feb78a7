"""CPU oracle for the FP8 linear path -- TEST INFRASTRUCTURE ONLY.

A plain-torch (CPU, fp32/fp64) restatement of the reference's oracle functions and
dispatch order. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker: the product
(``ayaka-py_amd/``) never imports or calls it and has no CPU fallback.

Each function cites the reference lines it restates. The reference cannot be
imported in this environment (it requires Python >= 3.13 and Triton >= 3.8), so the
restatement is pinned by the checks in ``tests/test_oracle.py``: exhaustive codec
tables, closed-form known answers, brute-force fp64 sums on tiny shapes, and the
invariants listed there. No function here is "parity unpinned".

Conventions: e4m3 = ``torch.float8_e4m3fn`` (OCP, max 448); UE8M0 code c decodes to
``2 ** (c - 127)`` via the bit pattern ``c << 23`` (0 -> +0.0, 0xFF -> NaN).
"""

from __future__ import annotations

import torch

E4M3 = torch.float8_e4m3fn
E4M3_MAX = 448.0  # reference quant.py:10 (DType.FP8_E4M3.max_finite)
GROUP_FLOOR = 1e-10  # reference quant.py:16
MX_MIN_EXP = -126.0  # reference quant.py:36
MX_MAX_EXP = 127.0  # reference quant.py:37
SCALE_BLOCK = 128  # reference gemm/_common.py:292


# ------------------------------------------------------------------ codecs
def e8m0_values(codes: torch.Tensor) -> torch.Tensor:
    """UE8M0 codes -> fp32 (reference gemm.py:11-14)."""
    bits = (codes.to(torch.int32) << 23).view(torch.float32)
    return torch.where(codes == 0xFF, torch.full_like(bits, float("nan")), bits)


def e4m3_values(codes: torch.Tensor) -> torch.Tensor:
    """Raw e4m3 bytes (uint8) -> fp32 through torch's own decoder."""
    return codes.view(E4M3).float()


# ------------------------------------------------------------------ quantizers
def per_token_group_quant(x: torch.Tensor, group_size: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """Per (token, K group) e4m3 quant with fp32 scales (reference quant.py:19-29)."""
    k = x.shape[-1]
    g = x.reshape(-1, k).float().reshape(-1, k // group_size, group_size)
    scale = g.abs().amax(dim=-1).clamp_min(GROUP_FLOOR) / E4M3_MAX
    q = (g / scale[..., None]).clamp(-E4M3_MAX, E4M3_MAX)
    return q.reshape(-1, k).to(E4M3), scale


def per_token_group_quant_mxfp8(x: torch.Tensor, group_size: int = 32) -> tuple[torch.Tensor, torch.Tensor]:
    """Per (token, K group) e4m3 quant with UE8M0 scales (reference quant.py:40-56).

    The exponent is ``ceil(log2(max(amax / 448, 1e-38)))`` evaluated with torch's
    fp32 ``log2`` exactly as the reference does; ``tests/test_oracle.py`` pins that
    torch's fp32 ``log2`` equals the correctly rounded value on every input where the
    ceiling depends on the rounding.
    """
    k = x.shape[-1]
    g = x.reshape(-1, k).float().reshape(-1, k // group_size, group_size)
    amax = g.abs().amax(dim=-1)
    e = torch.ceil(torch.log2((amax / E4M3_MAX).clamp_min(1e-38))).clamp(MX_MIN_EXP, MX_MAX_EXP)
    zero = amax == 0
    code = torch.where(zero, torch.zeros_like(e), e + 127.0).to(torch.uint8)
    scale = torch.where(zero, torch.ones_like(amax), torch.exp2(e))
    q = (g / scale[..., None]).clamp(-E4M3_MAX, E4M3_MAX)
    q = torch.where(zero[..., None], torch.zeros_like(q), q)
    return q.reshape(-1, k).to(E4M3), code


def per_token_quant(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Rowwise e4m3 quant, one fp32 scale per token (reference quant.py:59-66)."""
    k = x.shape[-1]
    x2 = x.reshape(-1, k).float()
    scale = x2.abs().amax(dim=-1).clamp_min(GROUP_FLOOR) / E4M3_MAX
    return (x2 / scale[:, None]).clamp(-E4M3_MAX, E4M3_MAX).to(E4M3), scale


def static_quant(x: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """Per-tensor static quant, ``x / s`` (reference quant.py:69-79)."""
    return (x.float() / scale.float().reshape(())).clamp(-E4M3_MAX, E4M3_MAX).to(E4M3)


# ------------------------------------------------------------------ GEMM / GEMV
def fp8_scaled_mm(a, b_nk, scale_a, scale_b, bias=None) -> torch.Tensor:
    """``(a @ b) * sa * sb + bias`` in fp32 (reference gemm.py:17-37).

    ``b_nk`` is the ``[N, K]`` weight (the layer passes ``weight.t()`` as ``b``).
    """
    y = a.float() @ b_nk.float().t()
    sa = scale_a.float()
    y = y * (sa.reshape(-1, 1) if sa.ndim != 0 else sa)
    y = y * scale_b.float()
    if bias is not None:
        y = y + bias.float()
    return y


def int8_matmul_exact(a, b_nk) -> torch.Tensor:
    """``a @ b_nk^T`` of int8 operands as the exact integer sum (int64).

    The reference's int8 kernel accumulates in int32 (gemm/int8_gemm.py:70-81,
    ``tl.dot(..., out_dtype=tl.int32)``), which is exact for any K below 2^17 at int8
    magnitudes. fp64 represents every such sum exactly, so a fp64 product rounded back
    to int64 is that sum.
    """
    return (a.double() @ b_nk.double().t()).round().to(torch.int64)


def int8_scaled_mm(a, b_nk, scale_a, scale_b, bias=None) -> torch.Tensor:
    """``float(a @ b) * sa * sb + bias`` in fp32 (reference gemm.py:192-211).

    The accumulator is the exact int32 sum (as the reference kernel, int8_gemm.py:81;
    the reference's own fp32 restatement rounds sums above 2^24, the kernel does not),
    converted to fp32 once; then the reference's operation order: times ``scale_a``
    per row, times ``scale_b`` per column, plus ``bias``.
    """
    y = int8_matmul_exact(a, b_nk).to(torch.float32)
    y = y * scale_a.float().reshape(-1, 1)
    y = y * scale_b.float().reshape(1, -1)
    if bias is not None:
        y = y + bias.float()
    return y


def fp8_blockwise_mm(a, b, scale_a, scale_b, bias=None, a_scale_col_major: bool = False) -> torch.Tensor:
    """Per-128-K partials rescaled then summed, fp32 (reference gemm.py:40-70)."""
    m, k = a.shape
    n = b.shape[0]
    af, bf = a.float(), b.float()
    saf, sbf = scale_a.float(), scale_b.float()
    y = torch.zeros((m, n), dtype=torch.float32, device=a.device)
    for kb in range(-(-k // SCALE_BLOCK)):
        lo, hi = kb * SCALE_BLOCK, min((kb + 1) * SCALE_BLOCK, k)
        part = af[:, lo:hi] @ bf[:, lo:hi].t()
        sa = saf[kb, :] if a_scale_col_major else saf[:, kb]
        sb = sbf[:, kb].repeat_interleave(SCALE_BLOCK)[:n]
        y = y + part * sa.reshape(-1, 1) * sb.reshape(1, -1)
    if bias is not None:
        y = y + bias.float()
    return y


def grouped_blockwise_mm(a, b, scales_a, scales_b, problem_sizes, expert_offsets, out) -> torch.Tensor:
    """MoE grouped block-128 GEMM (reference kernel/triton/moe/moe_grouped_gemm.py:472-585,
    the non-swapped operand convention): for expert e with rows [off_e, off_e + M_e),
    ``out[rows, :N_e] = fp8_blockwise_mm(a[rows, :K_e], b[e, :N_e, :K_e], sa_e, sb_e)``
    rounded once to ``out``'s dtype, rows of no expert keeping ``out``'s values. ``b`` is
    [E, N, K]. The scale operands are addressed as the reference's pointer tables do
    (:85-101, :564-573): ``sa_e`` starts at element ``off_e * (K / 128)`` of ``scales_a``
    and ``sb_e`` at ``e * (N / 128) * (K / 128)`` of ``scales_b``, both with row stride
    ``K_e // 128`` (the same as slicing when K_e == K). Returns the updated copy of ``out``."""
    res = out.clone()
    k_all, n_all = a.shape[1], b.shape[1]
    sa_flat, sb_flat = scales_a.reshape(-1), scales_b.reshape(-1)
    for e in range(expert_offsets.numel()):
        m_e, n_e, k_e = (int(v) for v in problem_sizes[e])
        off = int(expert_offsets[e])
        if m_e <= 0 or n_e <= 0:
            continue
        kb, nb = k_e // SCALE_BLOCK, -(-n_e // SCALE_BLOCK)
        sa0, sb0 = off * (k_all // SCALE_BLOCK), e * (n_all // SCALE_BLOCK) * (k_all // SCALE_BLOCK)
        sa_e = sa_flat[sa0:sa0 + m_e * kb].reshape(m_e, kb)
        sb_e = sb_flat[sb0:sb0 + nb * kb].reshape(nb, kb)
        y = fp8_blockwise_mm(a[off:off + m_e, :k_e], b[e, :n_e, :k_e], sa_e, sb_e)
        res[off:off + m_e, :n_e] = y.to(res.dtype)
    return res


def mxfp8_scaled_mm(a, a_scale, b, b_scale, bias=None) -> torch.Tensor:
    """e4m3 operands with UE8M0 1x32 scales folded in, fp32 (reference gemm.py:73-92)."""
    k = a.shape[1]
    sa = e8m0_values(a_scale).repeat_interleave(32, dim=1)[:, :k]
    sb = e8m0_values(b_scale).repeat_interleave(32, dim=1)[:, :k]
    y = (a.float() * sa) @ (b.float() * sb).t()
    if bias is not None:
        y = y + bias.float()
    return y


def _w8a16_scale_matrix(weight_scale, n, k, scale_row_stride, by, bx, scale_dtype, dtype):
    stride = -(-k // bx) if scale_row_stride is None else int(scale_row_stride)
    vals = e8m0_values(weight_scale) if scale_dtype == "e8m0" else weight_scale
    vals = vals.to(dtype).reshape(-1)
    rows = torch.arange(n, device=vals.device) // by
    cols = torch.arange(k, device=vals.device) // bx
    return vals[rows[:, None] * stride + cols[None, :]]


def fp8_weight_only_gemm(x, weight, weight_scale, scale_row_stride=None, block_size_y=1,
                         block_size_x=128, scale_dtype="e8m0") -> torch.Tensor:
    """W8A16 at M > 1: dequantized weight rounded to x.dtype, fp32 dot, out x.dtype
    (reference gemm.py:95-126)."""
    n, k = weight.shape
    w = weight.view(E4M3).float() if weight.dtype == torch.uint8 else weight.float()
    s = _w8a16_scale_matrix(weight_scale, n, k, scale_row_stride, block_size_y, block_size_x, scale_dtype, torch.float32)
    deq = (w * s).to(x.dtype)
    return (x.float() @ deq.float().t()).to(x.dtype)


def fp8_weight_only_gemv(x, weight, weight_scale, scale_row_stride=None, block_size_y=1,
                         block_size_x=128, scale_dtype="e8m0") -> torch.Tensor:
    """W8A16 at M == 1 in fp64, rounded once to x.dtype (reference gemm.py:129-157)."""
    n, k = weight.shape
    w = weight.view(E4M3).double() if weight.dtype == torch.uint8 else weight.double()
    s = _w8a16_scale_matrix(weight_scale, n, k, scale_row_stride, block_size_y, block_size_x, scale_dtype, torch.float64)
    return ((w * s) @ x.reshape(-1).double()).float().to(x.dtype)


def fp8_blockwise_gemv(a, b, scale_a, scale_b, bias=None) -> torch.Tensor:
    """M == 1 block-128 product in fp64, returned fp32 (reference gemm.py:160-189)."""
    k = a.numel()
    n = b.shape[0]
    av, bv = a.reshape(-1).double(), b.double()
    sa, sb = scale_a.reshape(-1).double(), scale_b.double()
    y = torch.zeros(n, dtype=torch.float64, device=av.device)
    for kb in range(-(-k // SCALE_BLOCK)):
        lo, hi = kb * SCALE_BLOCK, min((kb + 1) * SCALE_BLOCK, k)
        part = av[lo:hi] @ bv[:, lo:hi].t()
        y = y + part * sa[kb] * sb[:, kb].repeat_interleave(SCALE_BLOCK)[:n]
    if bias is not None:
        y = y + bias.double()
    return y.float()


# ------------------------------------------------------------------ linear composition
def fp8_linear(recipe: str, x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
               bias: torch.Tensor | None = None, *, weight_block=None, scale_dtype: str = "float32",
               input_scale: torch.Tensor | None = None, bias_in_fp32: bool = False) -> torch.Tensor:
    """The reference's per-recipe dispatch on CPU (its "PyTorch CPU path").

    Order of ``gemm/fp8_linear.py:102-260`` and ``layers/linear/fp8.py:296-547``:
    M == 1 -> weight-only GEMV (all recipes but MXFP8); rowwise / dynamic
    per-tensor -> per-token quant + scaled mm; block-128 -> group-128 quant +
    blockwise mm; MXFP8 -> MX quant + MX mm (bias fused); W8A16 M > 1 -> weight-only
    GEMM; static per-tensor M > 1 -> static quant + scaled mm. Bias is added in the
    activation dtype afterwards except for MXFP8.

    ``bias_in_fp32`` instead adds the bias to the fp32 GEMM result before the single
    rounding for the W8A8 GEMM paths (the fused-epilogue form the HIP path uses there).
    """
    lead, k = x.shape[:-1], x.shape[-1]
    x2 = x.reshape(-1, k)
    m, n = x2.shape[0], weight.shape[0]
    fused = bias if bias_in_fp32 else None
    if recipe == "mxfp8":
        q, code = per_token_group_quant_mxfp8(x2, 32)
        return mxfp8_scaled_mm(q, code, weight, weight_scale, bias).to(x.dtype).reshape(*lead, n)
    if recipe in ("w8a8_rowwise", "w8a8_dynamic_per_tensor", "w8a8_static_per_tensor"):
        by = n if weight_scale.numel() == 1 else 1
        if m == 1:
            y = fp8_weight_only_gemv(x2.reshape(k), weight, weight_scale.float(), -(-k // k), by, k, "float32").reshape(1, n)
        elif recipe == "w8a8_static_per_tensor":
            y = fp8_scaled_mm(static_quant(x2, input_scale), weight, input_scale, weight_scale, fused)
        else:
            q, s = per_token_quant(x2)
            y = fp8_scaled_mm(q, weight, s, weight_scale, fused)
    elif recipe == "w8a8_block128":
        sdt = "bfloat16" if weight_scale.dtype == torch.bfloat16 else "float32"
        if m == 1:
            y = fp8_weight_only_gemv(x2.reshape(k), weight, weight_scale, -(-k // 128), 128, 128, sdt).reshape(1, n)
        else:
            q, s = per_token_group_quant(x2, 128)
            y = fp8_blockwise_mm(q, weight, s, weight_scale, fused)
    elif recipe == "w8a16":
        by, bx = weight_block if weight_block is not None else (1, k)
        if m == 1:
            y = fp8_weight_only_gemv(x2.reshape(k), weight, weight_scale, -(-k // bx), by, bx, scale_dtype).reshape(1, n)
        else:
            y = fp8_weight_only_gemm(x2, weight, weight_scale, -(-k // bx), by, bx, scale_dtype)
    else:
        raise ValueError(f"unknown recipe {recipe!r}")
    y = y.to(x.dtype)
    if bias is not None and not (fused is not None and m > 1 and recipe != "w8a16"):
        y = y + bias
    return y.reshape(*lead, n)


# ------------------------------------------------------------------ KV cache
def kv_write(source, cache, slots, inverse_scale: float) -> None:
    """Write rows of ``source`` [n, heads, head_dim] to ``cache`` [pages, page_size, heads,
    head_dim] at flattened slots (reference cache_ops.py:40-62 ``_write_reference``, with
    the negative-slot filter of ``_write_kv_reference`` :109-111): fp8 caches take
    ``x.float() * inverse_scale`` clamped to the dtype's finite range, then torch's
    round-to-nearest-even cast; float caches a plain cast.
    """
    valid = slots >= 0
    source, slots = source[valid], slots[valid]
    payload = source
    if cache.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        limit = torch.finfo(cache.dtype).max
        payload = payload.float().mul(inverse_scale).clamp(-limit, limit)
    payload = payload.to(cache.dtype)
    target = cache.flatten(0, 1)
    if cache.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        target.view(torch.uint8).index_copy_(0, slots, payload.contiguous().view(torch.uint8))
    else:
        target.index_copy_(0, slots, payload)


def kv_gather(cache, slots, dtype, scale: float, dequantize: bool) -> torch.Tensor:
    """Rows of ``cache`` at ``slots`` (reference cache_ops.py:206-227 ``_gather_reference``):
    ``float(x) * scale`` when dequantizing, then cast to ``dtype``."""
    flat = cache.flatten(0, 1)
    if cache.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        result = flat.view(torch.uint8).index_select(0, slots).view(cache.dtype)
    else:
        result = flat.index_select(0, slots)
    if dequantize:
        result = result.float().mul(scale)
    return result.to(dtype)
