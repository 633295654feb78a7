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


def assert_linear_close(y: torch.Tensor, ref: torch.Tensor, label: str = "") -> float:
    y = y.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert y.shape == ref.shape, f"{label}: shape {tuple(y.shape)} != {tuple(ref.shape)}"
    assert torch.isfinite(y).all(), f"{label}: non-finite output"
    scale = ref.abs().max().item() if ref.numel() else 0.0
    err = (y - ref).abs()
    bound = REL * ref.abs() + FLOOR * scale
    bad = err > bound
    if bad.any():
        i = int((err - bound).argmax())
        raise AssertionError(
            f"{label}: {int(bad.sum())}/{err.numel()} elements out of tolerance; worst flat index {i}: "
            f"kernel {y.flatten()[i].item():.6g} vs oracle {ref.flatten()[i].item():.6g}"
        )
    return float(err.max().item() / scale) if scale else 0.0
