"""GPU: the HIP kernels against the committed golden fixtures (no oracle involved).

Quantizers must match bit for bit; products must lie within the north-star tolerance
(|y - ref| <= 1e-2 |ref| + 1e-3 max|ref|) of the fp64 expected values.
"""

import numpy as np
import pytest
import torch

from tests import _golden as G
from tests._tol import assert_linear_close

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)


def _codes(q: torch.Tensor) -> np.ndarray:
    return q.view(torch.uint8).cpu().numpy()


def test_quantizers_match_golden(gpu):
    import ayaka.kernel.hip as H

    _say("golden quantizers")
    fx = G.load()
    x = G.bf16(fx["quant_x_bf16"]).to(gpu)
    q, s = H.per_token_quant_fp8(x)
    assert np.array_equal(_codes(q), fx["pt_q"])
    assert np.array_equal(s.reshape(-1).cpu().numpy(), fx["pt_s"])
    q, s = H.per_token_group_quant_fp8(x, 128)
    assert np.array_equal(_codes(q), fx["g128_q"])
    assert np.array_equal(s.cpu().numpy(), fx["g128_s"])
    q, c = H.per_token_group_quant_mxfp8(x, 32)
    assert np.array_equal(_codes(q), fx["mx_q"])
    assert np.array_equal(c.cpu().numpy(), fx["mx_code"])
    q, c = H.per_token_group_quant_mxfp8(G.t(fx["mxb_x_f32"]).to(gpu), 32)
    assert np.array_equal(c.cpu().numpy(), fx["mxb_code"])
    assert np.array_equal(_codes(q), fx["mxb_q"])


def test_products_match_golden(gpu):
    import ayaka.kernel.hip as H

    _say("golden products")
    fx = G.load()
    d = lambda a: a.to(gpu)  # noqa: E731
    out = torch.empty(5, 24, dtype=torch.float32, device=gpu)
    H.fp8_scaled_mm(d(G.e4m3(fx["smm_a"])), d(G.e4m3(fx["smm_b"])).t(), d(G.t(fx["smm_sa"])), d(G.t(fx["smm_sb"])),
                    d(G.t(fx["smm_bias"])), out=out)
    assert_linear_close(out, torch.from_numpy(fx["smm_out"]).float(), "fp8_scaled_mm golden")
    out = torch.empty(3, 130, dtype=torch.float32, device=gpu)
    H.fp8_blockwise_mm(d(G.e4m3(fx["bmm_a"])), d(G.e4m3(fx["bmm_b"])), d(G.t(fx["bmm_sa"])), d(G.t(fx["bmm_sb"])), out=out)
    assert_linear_close(out, torch.from_numpy(fx["bmm_out"]).float(), "fp8_blockwise_mm golden")
    out = torch.empty(3, 20, dtype=torch.float32, device=gpu)
    H.mxfp8_scaled_mm(d(G.e4m3(fx["mxm_a"])), d(G.t(fx["mxm_ca"])), d(G.e4m3(fx["mxm_w"])), d(G.t(fx["mxm_cw"])),
                      d(G.t(fx["mxm_bias"])), out=out)
    assert_linear_close(out, torch.from_numpy(fx["mxm_out"]).float(), "mxfp8_scaled_mm golden")


@pytest.mark.parametrize("name,by,bx,sdt", [("row", 1, 256, "float32"), ("b128", 128, 128, "float32"), ("e8m0", 1, 32, "e8m0")])
def test_weight_only_matches_golden(gpu, name, by, bx, sdt):
    import ayaka.kernel.hip as H

    _say(f"golden weight-only {name}")
    fx = G.load()
    w, x = G.e4m3(fx["w16_w"]).to(gpu), G.bf16(fx["w16_x_bf16"]).to(gpu)
    sc = G.t(fx[f"w16_{name}_scale"]).to(gpu)
    stride = -(-256 // bx)
    y = H.fp8_weight_only_gemv(x[0].contiguous(), w, sc, stride, by, bx, sdt)
    assert_linear_close(y.reshape(-1), torch.from_numpy(fx[f"w16_{name}_gemv"]).float(), f"gemv {name} golden")
    y = H.fp8_weight_only_gemm(x, w, sc, stride, by, bx, sdt)
    assert_linear_close(y, torch.from_numpy(fx[f"w16_{name}_gemm"]).float(), f"gemm {name} golden")
