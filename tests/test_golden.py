"""The CPU oracle against the committed golden fixtures.

The fixtures are computed by ``tests/golden/make_golden.py`` with numpy code written
independently of the oracle (table-driven e4m3 rounding, fp64 products), so these
tests pin the oracle; the GPU suite checks the HIP kernels against the same files.
"""

import numpy as np
import torch

from oracle import fp8_oracle as ora
from tests import _golden as G


def _codes(q: torch.Tensor) -> np.ndarray:
    return q.view(torch.uint8).numpy()


def test_quantizers_match_golden_bit_for_bit():
    fx = G.load()
    x = G.bf16(fx["quant_x_bf16"])
    q, s = ora.per_token_quant(x)
    assert np.array_equal(_codes(q), fx["pt_q"]) and np.array_equal(s.numpy(), fx["pt_s"])
    q, s = ora.per_token_group_quant(x, 128)
    assert np.array_equal(_codes(q), fx["g128_q"]) and np.array_equal(s.numpy(), fx["g128_s"])
    q, c = ora.per_token_group_quant_mxfp8(x, 32)
    assert np.array_equal(_codes(q), fx["mx_q"]) and np.array_equal(c.numpy(), fx["mx_code"])


def test_mx_exponent_boundaries_match_golden():
    fx = G.load()
    q, c = ora.per_token_group_quant_mxfp8(G.t(fx["mxb_x_f32"]), 32)
    assert np.array_equal(c.numpy(), fx["mxb_code"])
    assert np.array_equal(_codes(q), fx["mxb_q"])


def _close(y: torch.Tensor, ref: np.ndarray, rel: float) -> None:
    y = y.double().numpy()
    assert np.all(np.abs(y - ref) <= rel * np.abs(ref) + 1e-6 * np.abs(ref).max()), np.abs(y - ref).max()


def test_products_match_golden():
    fx = G.load()
    # fp32 accumulation, fp32 out: only summation-order rounding separates it from fp64
    y = ora.fp8_scaled_mm(G.e4m3(fx["smm_a"]), G.e4m3(fx["smm_b"]), G.t(fx["smm_sa"]), G.t(fx["smm_sb"]), G.t(fx["smm_bias"]))
    _close(y, fx["smm_out"], 1e-5)
    y = ora.fp8_blockwise_mm(G.e4m3(fx["bmm_a"]), G.e4m3(fx["bmm_b"]), G.t(fx["bmm_sa"]), G.t(fx["bmm_sb"]))
    _close(y, fx["bmm_out"], 1e-5)
    y = ora.mxfp8_scaled_mm(G.e4m3(fx["mxm_a"]), G.t(fx["mxm_ca"]), G.e4m3(fx["mxm_w"]), G.t(fx["mxm_cw"]), G.t(fx["mxm_bias"]))
    _close(y, fx["mxm_out"], 1e-5)


def test_weight_only_matches_golden():
    fx = G.load()
    w, x = G.e4m3(fx["w16_w"]), G.bf16(fx["w16_x_bf16"])
    k = x.shape[1]
    for name, by, bx, sdt in (("row", 1, k, "float32"), ("b128", 128, 128, "float32"), ("e8m0", 1, 32, "e8m0")):
        sc = G.t(fx[f"w16_{name}_scale"])
        stride = -(-k // bx)
        # outputs are bf16: one rounding (2^-9 relative) on top of fp32 summation
        y = ora.fp8_weight_only_gemv(x[0], w, sc, stride, by, bx, sdt)
        _close(y.float(), fx[f"w16_{name}_gemv"], 2**-8)
        y = ora.fp8_weight_only_gemm(x, w, sc, stride, by, bx, sdt)
        _close(y.float(), fx[f"w16_{name}_gemm"], 2**-8)
