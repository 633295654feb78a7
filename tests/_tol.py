"""Tolerance rule for floating-point GEMM/GEMV parity.

A kernel output ``y`` matches the oracle ``ref`` when every element of every output row
(the last dimension; a vector is one row) satisfies

    |y - ref| <= 1e-2 * |ref| + 1e-3 * max|ref_row|

i.e. a 1e-2 relative error (the bar stated for this path: fp32 accumulation, bf16
out, max relative error <= 1e-2 against a dequant-matmul oracle), with an absolute
floor of 1e-3 of *that row's* scale for outputs that cancel to near zero. The floor is
per row, so a row whose magnitude is far below the largest row's is held to its own
scale (heavy-tailed activation rows, log-uniform block scales).

``assert_linear_close`` returns the measured max relative error ``|y - ref| / |ref|``
over the elements above their row's floor, the figure reported beside the throughput.
"""

import json
import os

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


def row_floor(ref: torch.Tensor) -> torch.Tensor:
    """``FLOOR * max|ref_row|`` broadcast to ``ref``'s shape (rows along the last dim)."""
    if ref.numel() == 0:
        return torch.zeros_like(ref)
    a = ref.abs()
    if a.dim() == 0:
        return FLOOR * a
    return FLOOR * a.amax(dim=-1, keepdim=True).expand_as(a)


def assert_linear_close(y: torch.Tensor, ref: torch.Tensor, label: str = "", extra: torch.Tensor | None = None) -> float:
    """``extra`` (optional, elementwise) widens the bound by a known, separately justified
    allowance, e.g. ``rounding_allowance`` when ``ref`` follows another bias order.
    Returns the max relative error over the elements above their row's floor."""
    y = y.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert y.shape == ref.shape, f"{label}: shape {tuple(y.shape)} != {tuple(ref.shape)}"
    assert torch.isfinite(y).all(), f"{label}: non-finite output"
    err = (y - ref).abs()
    floor = row_floor(ref)
    bound = REL * ref.abs() + floor
    if extra is not None:
        bound = bound + extra.detach().float().cpu()
    bad = err > bound
    if bad.any():
        i = int((err - bound).argmax())
        raise AssertionError(
            f"{label}: {int(bad.sum())}/{err.numel()} elements out of tolerance; worst flat index {i}: "
            f"kernel {y.flatten()[i].item():.6g} vs oracle {ref.flatten()[i].item():.6g}"
        )
    above = ref.abs() > floor
    return float((err[above] / ref.abs()[above]).max().item()) if above.any() else 0.0


def error_stats(y: torch.Tensor, ref: torch.Tensor) -> dict:
    """Error figures of one output against the oracle (rows along the last dim):

    * ``max_err_over_row_max``: max |y - ref| / max|ref_row| (the error in units of each
      row's scale);
    * ``max_rel_err_significant``: max |y - ref| / |ref| over elements with
      |ref| >= 0.1 max|ref_row|;
    * ``max_rel_err_above_floor``: the same over every element above the 1e-3 row floor
      (near the floor this is fp32 summation-order noise under cancellation, not a
      relative error of the product);
    * ``max_row_normwise_err``: max over rows of ||y - ref||_2 / ||ref||_2.
    """
    y = y.detach().float().cpu()
    ref = ref.detach().float().cpu()
    if ref.dim() == 0:
        y, ref = y.reshape(1), ref.reshape(1)
    y2, r2 = y.reshape(-1, ref.shape[-1]), ref.reshape(-1, ref.shape[-1])
    err = (y2 - r2).abs()
    a = r2.abs()
    rowmax = a.amax(dim=-1, keepdim=True)
    safe = torch.where(rowmax > 0, rowmax, torch.ones_like(rowmax))

    def rel_over(mask: torch.Tensor) -> float:
        return float((err[mask] / a[mask]).max().item()) if mask.any() else 0.0

    norm = torch.linalg.vector_norm(r2, dim=-1)
    dnorm = torch.linalg.vector_norm(y2 - r2, dim=-1)
    normwise = torch.where(norm > 0, dnorm / torch.where(norm > 0, norm, torch.ones_like(norm)), dnorm)
    return {
        "max_err_over_row_max": float((err / safe).max().item()) if err.numel() else 0.0,
        "max_rel_err_significant": rel_over(a >= 0.1 * rowmax),
        "max_rel_err_above_floor": rel_over(a > FLOOR * rowmax),
        "max_row_normwise_err": float(normwise.max().item()) if normwise.numel() else 0.0,
    }


def record_parity(label: str, **fields) -> None:
    """Append one JSON record to the file ``AYAKA_PARITY_LOG`` names (no-op when unset)."""
    path = os.environ.get("AYAKA_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps({"label": label, **fields}) + "\n")
