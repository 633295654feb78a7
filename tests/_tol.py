"""Tolerance rule for floating-point GEMM/GEMV parity.

A kernel output ``y`` matches the oracle ``ref`` when every element satisfies

    |y - ref| <= 1e-2 * |ref| + 1e-3 * max|ref|

i.e. a 1e-2 relative error (the bar stated for this path: fp32 accumulation, bf16
out, max relative error <= 1e-2 against a dequant-matmul oracle), with an absolute
floor of 1e-3 of the output's scale for outputs that cancel to near zero.
"""

import torch

REL = 1e-2
FLOOR = 1e-3


def rounding_allowance(gemm: torch.Tensor, out: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Elementwise gap between the fused-bias order (one rounding of ``gemm + bias`` to
    ``dtype``) and the reference's order (``gemm`` rounded to ``dtype``, then the bias added
    in ``dtype``): at most one ``dtype`` ulp of ``|gemm|`` plus one of ``|out|``."""
    bits, min_exp = {torch.bfloat16: (7, -126), torch.float16: (10, -14), torch.float32: (23, -126)}[dtype]

    def ulp(v: torch.Tensor) -> torch.Tensor:
        a = v.detach().float().cpu().abs()
        _, e = torch.frexp(a)  # |v| = f * 2^e, f in [0.5, 1); e = 0 for v = 0
        e = torch.where(a == 0, torch.full_like(e, min_exp + 1), e)
        return torch.exp2((torch.clamp(e - 1, min=min_exp) - bits).float())
    return ulp(gemm) + ulp(out)


def assert_linear_close(y: torch.Tensor, ref: torch.Tensor, label: str = "", extra: torch.Tensor | None = None) -> float:
    """``extra`` (optional, elementwise) widens the bound by a known, separately justified
    allowance, e.g. ``rounding_allowance`` when ``ref`` follows another bias order."""
    y = y.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert y.shape == ref.shape, f"{label}: shape {tuple(y.shape)} != {tuple(ref.shape)}"
    assert torch.isfinite(y).all(), f"{label}: non-finite output"
    scale = ref.abs().max().item() if ref.numel() else 0.0
    err = (y - ref).abs()
    bound = REL * ref.abs() + FLOOR * scale
    if extra is not None:
        bound = bound + extra.detach().float().cpu()
    bad = err > bound
    if bad.any():
        i = int((err - bound).argmax())
        raise AssertionError(
            f"{label}: {int(bad.sum())}/{err.numel()} elements out of tolerance; worst flat index {i}: "
            f"kernel {y.flatten()[i].item():.6g} vs oracle {ref.flatten()[i].item():.6g}"
        )
    return float(err.max().item() / scale) if scale else 0.0
