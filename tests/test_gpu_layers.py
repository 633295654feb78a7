"""GPU: the FP8 LinearMethod lifecycle end to end, for every recipe.

``FP8Config.from_config(quantization_config)`` -> ``create_weights`` on the GPU ->
checkpoint tensors through the parameters' ``weight_loader`` ->
``process_weights_after_loading`` -> ``apply`` at decode and prefill M, compared with
the CPU oracle's composition of the same recipe (``oracle.fp8_linear``).
"""

import sys

import pytest
import torch
from torch import nn

from oracle import fp8_oracle as ora
from tests._tol import assert_linear_close, rounding_allowance

pytestmark = pytest.mark.gpu
FP8 = torch.float8_e4m3fn
N, K = 384, 1024


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _checkpoint(recipe, g):
    """Synthetic checkpoint tensors: (weight e4m3, scale, oracle kwargs, config)."""
    wf = torch.randn(N, K, generator=g) * 0.02
    if recipe in ("w8a8_rowwise", "w8a16"):
        s = wf.abs().amax(dim=1) / 448
        return (wf / s[:, None]).to(FP8), s, {}
    if recipe in ("w8a8_dynamic_per_tensor", "w8a8_static_per_tensor"):
        s = wf.abs().amax() / 448
        return (wf / s).to(FP8), s.reshape(()), {}
    if recipe == "w8a8_block128":
        s = wf.reshape(N // 128, 128, K // 128, 128).abs().amax(dim=(1, 3)) / 448
        w = (wf / s.repeat_interleave(128, 0).repeat_interleave(128, 1)).to(FP8)
        return w, s, {}
    if recipe == "mxfp8":
        q, c = ora.per_token_group_quant_mxfp8(wf, 32)
        return q, c, {}
    raise AssertionError(recipe)


CONFIGS = {
    "w8a8_rowwise": {"fp8_recipe": "w8a8_rowwise"},
    "w8a8_dynamic_per_tensor": {"quant_method": "fp8", "activation_scheme": "dynamic"},
    "w8a8_static_per_tensor": {"quant_method": "fp8", "activation_scheme": "static"},
    "w8a8_block128": {"weight_block_size": [128, 128], "scale_format": "float32"},
    "mxfp8": {"quant_algo": "mxfp8"},
    "w8a16": {"quant_algo": "w8a16"},
}


@pytest.mark.parametrize("m", [1, 7, 64])
@pytest.mark.parametrize("recipe", list(CONFIGS))
def test_linear_method_lifecycle(gpu, recipe, m):
    from ayaka.layers.linear.fp8 import FP8Config

    _say(f"layer lifecycle recipe={recipe} m={m}")
    g = torch.Generator().manual_seed(sum(map(ord, recipe)) + m)
    w, s, _ = _checkpoint(recipe, g)
    method = FP8Config.from_config(CONFIGS[recipe]).get_quant_method(None, "model.layers.0.mlp.down_proj")
    layer = nn.Module()
    method.create_weights(layer, output_partition_sizes=[N], input_size_per_partition=K, device=gpu)
    layer.weight.data.copy_(w.to(gpu))
    scale_name = "weight_scale_inv" if recipe == "w8a8_block128" else "weight_scale"
    param = getattr(layer, scale_name)
    param.weight_loader(layer, param, s.to(gpu))
    input_scale = None
    if recipe == "w8a8_static_per_tensor":
        input_scale = torch.tensor(0.05)
        layer.input_scale.weight_loader(layer, layer.input_scale, input_scale.to(gpu))
    method.process_weights_after_loading(layer)

    x = torch.randn(m, K, generator=g).to(torch.bfloat16)
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    y = method.apply(layer, x.to(gpu), bias.to(gpu))
    oracle_recipe = recipe
    kw = {}
    if recipe == "w8a16":
        kw = dict(weight_block=None, scale_dtype="float32")
        s_ref = s.reshape(N, 1)
    elif recipe in ("w8a8_dynamic_per_tensor", "w8a8_static_per_tensor"):
        s_ref = torch.full((N,), float(s))  # the loader broadcasts the scalar into [N]
    else:
        s_ref = s
    ref = ora.fp8_linear(oracle_recipe, x, w, s_ref, bias, input_scale=input_scale, bias_in_fp32=True, **kw)
    # the reference's W8A16 method returns [N] for a one-token input (no lead dims)
    expected_shape = (N,) if (recipe == "w8a16" and m == 1) else (m, N)
    assert y.shape == expected_shape and y.dtype == torch.bfloat16
    assert_linear_close(y.reshape(m, N), ref, f"{recipe} m={m}")
    # The reference's own bias order (a separate add in x.dtype after the GEMM's
    # rounding, gemm/fp8_linear.py:92-99) is within the same tolerance.
    # Up to the two orders' own rounding gap (test_fused_bias_against_reference_order).
    ref_order = ora.fp8_linear(oracle_recipe, x, w, s_ref, bias, input_scale=input_scale, bias_in_fp32=False, **kw)
    gemm = ora.fp8_linear(oracle_recipe, x, w, s_ref, None, input_scale=input_scale, **kw)
    assert_linear_close(y.reshape(m, N), ref_order, f"{recipe} m={m} (reference bias order)",
                        extra=rounding_allowance(gemm, ref_order, torch.bfloat16).reshape(m, N))


@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("recipe", ["w8a8_rowwise", "w8a8_static_per_tensor", "w8a8_block128"])
def test_fused_bias_against_reference_order(gpu, recipe, xdt):
    """The W8A8 GEMMs add the bias in fp32 before the one rounding to x.dtype; the
    reference rounds the GEMM result to x.dtype and adds the bias in x.dtype
    (gemm/fp8_linear.py:92-99). With a bias as large as the products, the two orders
    differ by at most one rounding of the GEMM result plus one of the sum:
    |fused - reference| <= ulp(|gemm|) + ulp(|out|) in x.dtype, on top of the
    kernel's accumulation error (checked against the fused-order oracle)."""
    from ayaka.layers.linear.fp8 import FP8Config

    m = 64
    _say(f"fused bias vs reference order recipe={recipe} x={xdt}")
    g = torch.Generator().manual_seed(99 + len(recipe))
    w, s, _ = _checkpoint(recipe, g)
    method = FP8Config.from_config(CONFIGS[recipe]).get_quant_method(None, "model.layers.0.mlp.up_proj")
    layer = nn.Module()
    method.create_weights(layer, output_partition_sizes=[N], input_size_per_partition=K, params_dtype=xdt, device=gpu)
    layer.weight.data.copy_(w.to(gpu))
    param = getattr(layer, "weight_scale_inv" if recipe == "w8a8_block128" else "weight_scale")
    param.weight_loader(layer, param, s.to(gpu))
    input_scale = None
    if recipe == "w8a8_static_per_tensor":
        input_scale = torch.tensor(0.05)
        layer.input_scale.weight_loader(layer, layer.input_scale, input_scale.to(gpu))
    method.process_weights_after_loading(layer)
    s_ref = torch.full((N,), float(s)) if recipe == "w8a8_static_per_tensor" else s
    x = torch.randn(m, K, generator=g).to(xdt)
    gemm = ora.fp8_linear(recipe, x.float().to(xdt), w, s_ref, None, input_scale=input_scale).float()
    bias = (-gemm[0] + torch.randn(N, generator=g) * gemm.abs().mean()).to(xdt)  # cancels row 0
    y = method.apply(layer, x.to(gpu), bias.to(gpu)).float().cpu()
    fused = ora.fp8_linear(recipe, x, w, s_ref, bias, input_scale=input_scale, bias_in_fp32=True).float()
    ref_order = ora.fp8_linear(recipe, x, w, s_ref, bias, input_scale=input_scale, bias_in_fp32=False).float()
    assert_linear_close(y, fused, f"{recipe} fused order")
    gap = (fused - ref_order).abs()
    bound = rounding_allowance(gemm, torch.maximum(fused.abs(), ref_order.abs()), xdt)
    assert (gap <= bound).all(), f"order gap {gap.max().item()} beyond one rounding each"
    _say(f"  max |fused - reference order| = {gap.max().item():.4g}; "
         f"max |kernel - reference order| / max|ref| = {((y - ref_order).abs().max() / ref_order.abs().max()).item():.3g}")
