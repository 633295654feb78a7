"""GPU: a seeded sweep of shapes through the drop-in layer API, every recipe.

The config-point and kernel tests pin the shapes the benchmarks use and the edges each
kernel's plan names. This sweep draws (M, N, K) at random, from 1-row decode up to
K-split and 256 x 256 prefill launches, with ragged N and K where the recipe allows,
and checks ``LinearMethod.apply`` (activation quant + kernel choice + epilogue) against
the CPU oracle's composition of the same recipe under the stated tolerance. The kernel
routes differ by M, N, K and alignment, so a shape that falls between the planned
cases is where a dispatch mistake would show.
"""

import random
import sys

import pytest
import torch
from torch import nn

from oracle import fp8_oracle as ora
from tests._tol import assert_linear_close, rounding_allowance

pytestmark = pytest.mark.gpu
FP8 = torch.float8_e4m3fn

CONFIGS = {
    "w8a8_rowwise": {"fp8_recipe": "w8a8_rowwise"},
    "w8a8_dynamic_per_tensor": {"quant_method": "fp8", "activation_scheme": "dynamic"},
    "w8a8_static_per_tensor": {"quant_method": "fp8", "activation_scheme": "static"},
    "w8a8_block128": {"weight_block_size": [128, 128], "scale_format": "float32"},
    "mxfp8": {"quant_algo": "mxfp8"},
    "w8a16": {"quant_algo": "w8a16"},
}
K_UNIT = {"w8a8_block128": 128, "mxfp8": 32}  # the dynamic quantizers' group widths; else 16


def _cases(per_recipe=24, seed=2024):
    rng = random.Random(seed)
    cases = []
    for recipe in CONFIGS:
        unit = K_UNIT.get(recipe, 16)
        for i in range(per_recipe):
            m = [1, rng.randint(2, 8), rng.randint(9, 64), rng.randint(65, 255), rng.randint(256, 640),
                 rng.randint(2, 640)][i % 6]
            n = rng.choice([rng.randint(8, 700), rng.randint(256, 2600), 4 * rng.randint(64, 650)])
            k = unit * rng.randint(max(1, 128 // unit), 4096 // unit)
            xdt = rng.choice(["bfloat16", "bfloat16", "float16"])
            cases.append((recipe, m, n, k, xdt))
    return cases


def _checkpoint(recipe, n, k, g):
    """Checkpoint tensors of one recipe for an [n, k] weight: (e4m3 weight, scale)."""
    wf = torch.randn(n, k, generator=g) * 0.02
    if recipe in ("w8a8_rowwise", "w8a16"):
        s = wf.abs().amax(dim=1).clamp_min(1e-6) / 448
        return (wf / s[:, None]).to(FP8), s
    if recipe in ("w8a8_dynamic_per_tensor", "w8a8_static_per_tensor"):
        s = wf.abs().amax() / 448
        return (wf / s).to(FP8), s.reshape(())
    if recipe == "w8a8_block128":
        nb, kb = -(-n // 128), k // 128
        pad = torch.zeros(nb * 128, k)
        pad[:n] = wf
        s = pad.reshape(nb, 128, kb, 128).abs().amax(dim=(1, 3)).clamp_min(1e-6) / 448
        w = (pad / s.repeat_interleave(128, 0).repeat_interleave(128, 1))[:n].to(FP8)
        return w, s
    if recipe == "mxfp8":
        return ora.per_token_group_quant_mxfp8(wf, 32)
    raise AssertionError(recipe)


@pytest.mark.parametrize("recipe,m,n,k,xdt", _cases())
def test_linear_shape_sweep(gpu, recipe, m, n, k, xdt):
    from ayaka.layers.linear.fp8 import FP8Config

    print(f"shape sweep recipe={recipe} m={m} n={n} k={k} x={xdt}", flush=True)
    xdt = getattr(torch, xdt)
    sys.stdout.flush()
    g = torch.Generator().manual_seed(m * 7919 + n * 31 + k)
    w, s = _checkpoint(recipe, n, k, g)
    method = FP8Config.from_config(CONFIGS[recipe]).get_quant_method(None, "model.layers.0.mlp.down_proj")
    layer = nn.Module()
    method.create_weights(layer, output_partition_sizes=[n], input_size_per_partition=k, params_dtype=xdt, device=gpu)
    layer.weight.data.copy_(w.to(gpu))
    param = getattr(layer, "weight_scale_inv" if recipe == "w8a8_block128" else "weight_scale")
    param.weight_loader(layer, param, s.to(gpu))
    input_scale = None
    if recipe == "w8a8_static_per_tensor":
        input_scale = torch.tensor(0.05)
        layer.input_scale.weight_loader(layer, layer.input_scale, input_scale.to(gpu))
    method.process_weights_after_loading(layer)

    x = torch.randn(m, k, generator=g).to(xdt)
    bias = torch.randn(n, generator=g).to(xdt)
    y = method.apply(layer, x.to(gpu), bias.to(gpu))
    kw = {}
    if recipe == "w8a16":
        kw = dict(weight_block=None, scale_dtype="float32")
        s_ref = s.reshape(n, 1)
    elif recipe in ("w8a8_dynamic_per_tensor", "w8a8_static_per_tensor"):
        s_ref = torch.full((n,), float(s))  # the loader broadcasts the scalar into [N]
    else:
        s_ref = s
    # The bias order of the path taken: the W8A8 GEMMs add it in fp32 before their one
    # rounding; the weight-only paths (W8A16 at every M, the M = 1 GEMV of the W8A8
    # recipes) round first and add it in bf16, as the reference does. MXFP8 fuses it.
    # Rounding before the add can move a result that cancels against the bias by one
    # ulp of the product on either side of a rounding boundary: that ulp (and one
    # of the sum) is allowed on top of the tolerance there, as in the lifecycle test.
    fused_bias = recipe != "w8a16" and m > 1
    ref = ora.fp8_linear(recipe, x, w, s_ref, bias, input_scale=input_scale, bias_in_fp32=fused_bias, **kw)
    extra = None
    if not fused_bias:
        gemm = ora.fp8_linear(recipe, x, w, s_ref, None, input_scale=input_scale, **kw)
        extra = rounding_allowance(gemm, ref, xdt).reshape(m, n)
    assert_linear_close(y.reshape(m, n), ref, f"{recipe} m={m} n={n} k={k}", extra=extra)


def _quant_cases(n=48, seed=99):
    rng = random.Random(seed)
    kinds = ["per_token", "group128", "group_col", "mx32", "static"]
    cases = []
    for i in range(n):
        kind = kinds[i % len(kinds)]
        m = rng.choice([1, rng.randint(2, 16), rng.randint(17, 700)])
        unit = {"group128": 128, "group_col": 128, "mx32": 32}.get(kind, 1)
        k = unit * rng.randint(1, 20000 // unit) if rng.random() < 0.7 else unit * rng.randint(1, 256 // unit + 1)
        cases.append((kind, m, k, rng.choice(["bfloat16", "float16", "float32"])))
    return cases


def _bits(t):
    t = t.cpu().contiguous()
    return t.view(torch.uint8) if t.dtype == FP8 else (t.view(torch.int32) if t.dtype == torch.float32 else t)


@pytest.mark.parametrize("kind,m,k,xdt", _quant_cases())
def test_quant_shape_sweep(gpu, kind, m, k, xdt):
    """The activation quantizers on random shapes: e4m3 bytes and scales bit-exact."""
    from ayaka.kernel.hip import (per_token_group_quant_fp8, per_token_group_quant_mxfp8, per_token_quant_fp8,
                                  static_quant_fp8)
    from ayaka.kernel.hip.quant.fp8_quant import per_token_group_quant_fp8_colmajor

    print(f"quant sweep {kind} m={m} k={k} x={xdt}", flush=True)
    g = torch.Generator().manual_seed(m * 131 + k)
    x = (torch.randn(m, k, generator=g) * torch.exp(torch.randn(m, 1, generator=g) * 3)).to(getattr(torch, xdt))
    xg = x.to(gpu)
    if kind == "per_token":
        (q, s), (rq, rs) = per_token_quant_fp8(xg), ora.per_token_quant(x)
    elif kind == "group128":
        (q, s), (rq, rs) = per_token_group_quant_fp8(xg, 128), ora.per_token_group_quant(x, 128)
    elif kind == "group_col":
        (q, s_t), (rq, rs) = per_token_group_quant_fp8_colmajor(xg, 128), ora.per_token_group_quant(x, 128)
        s = s_t.t()  # [K / 128, M] column-major scales
    elif kind == "mx32":
        (q, s), (rq, rs) = per_token_group_quant_mxfp8(xg, 32), ora.per_token_group_quant_mxfp8(x, 32)
    else:
        scale = torch.tensor(0.03)
        q, s = static_quant_fp8(xg, scale.to(gpu)), scale
        rq, rs = ora.static_quant(x, scale), scale
    torch.cuda.synchronize()
    assert torch.equal(_bits(s.reshape(rs.shape)), _bits(rs)), "scales differ"
    assert torch.equal(_bits(q), _bits(rq)), "codes differ"


def _w8a16_cases(n=30, seed=31):
    rng = random.Random(seed)
    layouts = [(1, 0, "float32"), (128, 128, "bfloat16"), (128, 128, "float32"), (1, 32, "e8m0"), (64, 64, "float32")]
    cases = []
    for i in range(n):
        by, bx, sdt = layouts[i % len(layouts)]
        m = rng.choice([1, rng.randint(2, 8), rng.randint(9, 32), rng.randint(33, 300)])
        nn_ = rng.randint(16, 3000)
        k = rng.choice([256 * rng.randint(1, 24), 16 * rng.randint(1, 400)])
        if bx:
            k = max(bx, k // bx * bx)
        cases.append((m, nn_, k, by, bx, sdt, rng.choice(["bfloat16", "float16"])))
    return cases


@pytest.mark.parametrize("m,n,k,by,bx,sdt,xdt", _w8a16_cases())
def test_weight_only_shape_sweep(gpu, m, n, k, by, bx, sdt, xdt):
    """W8A16 GEMV / GEMM on random shapes and every scale layout (per channel, 128 x 128
    bf16 / fp32 blocks, per-32 UE8M0, 64 x 64) against the oracle."""
    from ayaka.kernel.hip import fp8_weight_only_gemm, fp8_weight_only_gemv

    print(f"w8a16 sweep m={m} n={n} k={k} block={by}x{bx} scale={sdt} x={xdt}", flush=True)
    bx = bx or k  # 0: one scale per row
    g = torch.Generator().manual_seed(m * 17 + n * 3 + k)
    w = (torch.randn(n, k, generator=g) * 40).clamp(-448, 448).to(FP8)
    rows, cols = -(-n // by), -(-k // bx)
    if sdt == "e8m0":
        scale = torch.randint(115, 125, (rows, cols), generator=g, dtype=torch.uint8)
    else:
        scale = (torch.rand(rows, cols, generator=g) * 0.01 + 1e-3).to(getattr(torch, sdt))
    x = torch.randn(m, k, generator=g).to(getattr(torch, xdt))
    if m == 1:
        y = fp8_weight_only_gemv(x.reshape(k).to(gpu), w.to(gpu), scale.to(gpu), cols, by, bx, sdt).reshape(1, n)
        ref = ora.fp8_weight_only_gemv(x.reshape(k), w, scale, cols, by, bx, sdt).reshape(1, n)
    else:
        y = fp8_weight_only_gemm(x.to(gpu), w.to(gpu), scale.to(gpu), cols, by, bx, sdt)
        ref = ora.fp8_weight_only_gemm(x, w, scale, cols, by, bx, sdt)
    assert_linear_close(y, ref, f"w8a16 m={m} n={n} k={k} {by}x{bx} {sdt}")
