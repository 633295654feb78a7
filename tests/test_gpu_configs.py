"""GPU parity at every BASELINE.json configuration, at full size, through the layer API.

Every (configuration, projection, M) point of ``BASELINE.json:configs`` runs the drop-in
path exactly as a model would: ``FP8Config.from_config`` -> ``create_weights`` on the
GPU -> checkpoint tensors through the parameters' ``weight_loader`` ->
``process_weights_after_loading`` -> ``apply``. Inputs follow the configurations'
distributions (``workloads.py``). Each point is checked twice:

* against the CPU oracle (``oracle.fp8_linear``, the reference's dispatch) on sampled
  rows -- every row up to M = 64, else the first and last 8 rows and two seeded rows of
  every 128-row tile -- and all N columns (M = 1: the whole output, fp64 GEMV);
* over the whole output, against the oracle's torch restatement evaluated on the device.
  For the W8A8 recipes the path's own activation quantizer runs first and its output is
  checked bit for bit against the CPU oracle's quantizer over *all* rows; the device
  restatement of the GEMM then takes those operands. (torch's own device quantizer is
  not a valid stand-in: its fp32 division and log2 differ from the CPU oracle's in the
  last bit on a few thousand elements per configuration, measured.)

Tolerance (``tests/_tol.py``): ``|y - ref| <= 1e-2 |ref| + 1e-3 max|ref_row|``, the floor
taken per output row. Each point's measured max relative error (over the elements above
their row's floor) is printed and, when ``AYAKA_PARITY_LOG`` names a file, appended to it
as one JSON record. The W8A8 GEMMs
fuse the bias in fp32 (oracle ``bias_in_fp32=True``); the reference's own order (bias
added in bf16 after the GEMM's rounding) is checked within the same tolerance.

"""

import sys

import pytest
import torch
from torch import nn

import workloads as wl
from oracle import fp8_oracle as ora
from tests._tol import assert_linear_close, error_stats, record_parity, rounding_allowance

pytestmark = pytest.mark.gpu

# (config, recipe for the oracle, FP8Config quantization_config)
RECIPES = {
    "cfg1_per_tensor": ("w8a8_dynamic_per_tensor", {"quant_method": "fp8", "activation_scheme": "dynamic"}),
    "cfg2_w8a16": ("w8a16", {"quant_algo": "w8a16"}),
    "cfg3_rowwise": ("w8a8_rowwise", {"fp8_recipe": "w8a8_rowwise"}),
    "cfg4_block128": ("w8a8_block128", {"weight_block_size": [128, 128], "scale_format": "float32"}),
    "cfg5_mxfp8": ("mxfp8", {"quant_algo": "mxfp8"}),
}

CASES = [(cfg["name"], proj, n, k, m) for cfg in wl.CONFIGS for proj, n, k in cfg["shapes"] for m in cfg["ms"]]

_cache: dict = {}


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _weights(cfg: str, proj: str, n: int, k: int, device):
    """(weight e4m3 on device, scale as loaded on device, CPU copies) for one projection;
    only the most recent projection is kept, so memory stays bounded."""
    key = (cfg, proj)
    if key not in _cache:
        _cache.clear()
        torch.cuda.empty_cache()
        if cfg == "cfg1_per_tensor":
            w, s = wl.cfg1_weights(n, k, device)
        elif cfg in ("cfg2_w8a16", "cfg3_rowwise"):
            w, s = wl.cfg23_weights(n, k, device)
            if cfg == "cfg2_w8a16":
                s = s.reshape(n, 1)
        elif cfg == "cfg4_block128":
            w, s = wl.cfg4_weights(n, k, device)
        else:
            w, s = wl.cfg5_weights(n, k, device)
        torch.cuda.synchronize()
        _cache[key] = (w, s, w.cpu(), s.cpu())
    return _cache[key]


def _activations(cfg: str, m: int, k: int, device):
    if cfg in ("cfg2_w8a16", "cfg3_rowwise"):
        return wl.outlier_activations(m, k, device)
    if cfg == "cfg5_mxfp8":
        return wl.student_t_activations(m, k, device)
    return wl.normal_activations(m, k, device)


def _layer(config: dict, w: torch.Tensor, s: torch.Tensor, device):
    from ayaka.layers.linear.fp8 import FP8Config

    method = FP8Config.from_config(config).get_quant_method(None, "model.layers.0.mlp.proj")
    layer = nn.Module()
    method.create_weights(layer, output_partition_sizes=[int(w.shape[0])], input_size_per_partition=int(w.shape[1]),
                          device=device)
    layer.weight.data.copy_(w)
    name = "weight_scale_inv" if "weight_scale_inv" in dict(layer.named_parameters()) else "weight_scale"
    param = getattr(layer, name)
    param.weight_loader(layer, param, s)
    method.process_weights_after_loading(layer)
    return method, layer


def _oracle_kwargs(recipe: str) -> dict:
    return {"weight_block": None, "scale_dtype": "float32"} if recipe == "w8a16" else {}


def _assert_quant_exact(q, scale, ref_q, ref_scale, label):
    assert torch.equal(q.cpu().view(torch.uint8), ref_q.view(torch.uint8)), f"{label}: quantized values differ"
    got, want = scale.cpu().reshape(ref_scale.shape), ref_scale
    if want.dtype == torch.uint8:
        assert torch.equal(got, want), f"{label}: UE8M0 codes differ"
    else:
        assert torch.equal(got.float().view(torch.int32), want.float().view(torch.int32)), f"{label}: scales differ"


def _device_reference(recipe, x, w, s, bias, kw):
    """The oracle on the device over every row. W8A8 at M > 1: the path's quantizer, pinned
    bit for bit to the CPU oracle's over all rows, feeds the oracle's GEMM restatement."""
    from ayaka.kernel.hip import per_token_group_quant_fp8, per_token_group_quant_mxfp8, per_token_quant_fp8

    m = x.shape[0]
    if recipe == "w8a16" or m == 1 and recipe != "mxfp8":
        return ora.fp8_linear(recipe, x, w, s, bias, bias_in_fp32=True, **kw)
    x_cpu = x.cpu()
    if recipe == "mxfp8":
        q, codes = per_token_group_quant_mxfp8(x, 32)
        _assert_quant_exact(q, codes, *ora.per_token_group_quant_mxfp8(x_cpu, 32), "MX quant")
        y = ora.mxfp8_scaled_mm(q, codes, w, s, bias)
    elif recipe == "w8a8_block128":
        q, sa = per_token_group_quant_fp8(x, 128)
        _assert_quant_exact(q, sa, *ora.per_token_group_quant(x_cpu, 128), "group-128 quant")
        y = ora.fp8_blockwise_mm(q, w, sa, s, bias)
    else:
        q, sa = per_token_quant_fp8(x)
        _assert_quant_exact(q, sa, *ora.per_token_quant(x_cpu), "per-token quant")
        y = ora.fp8_scaled_mm(q, w, sa, s, bias)
    return y.to(x.dtype)


@pytest.mark.parametrize("cfg,proj,n,k,m", CASES, ids=[f"{c}-{p}-M{m}" for c, p, n, k, m in CASES])
def test_config_point(gpu, cfg, proj, n, k, m):
    recipe, config = RECIPES[cfg]
    _say(f"config parity {cfg} {proj} N={n} K={k} M={m}")
    w, s, w_cpu, s_cpu = _weights(cfg, proj, n, k, gpu)
    x = _activations(cfg, m, k, gpu)
    bias = wl.bias_vector(n, gpu) if cfg == "cfg3_rowwise" else None
    method, layer = _layer(config, w, s, gpu)
    y = method.apply(layer, x, bias).reshape(m, n)
    assert y.dtype == torch.bfloat16
    kw = _oracle_kwargs(recipe)

    # Whole output against the oracle's torch restatement on the device.
    ref_dev = _device_reference(recipe, x, w, s, bias, kw)
    assert_linear_close(y, ref_dev.reshape(m, n), f"{cfg} {proj} M={m} (device oracle, all rows)")
    stats_all = error_stats(y, ref_dev.reshape(m, n))
    del ref_dev

    # Sampled rows, all columns, against the CPU oracle.
    rows = wl.sample_rows(m)
    x_s = x.cpu()[rows]
    b_cpu = bias.cpu() if bias is not None else None
    ref = ora.fp8_linear(recipe, x_s, w_cpu, s_cpu, b_cpu, bias_in_fp32=True, **kw).reshape(len(rows), n)
    y_s = y.cpu()[rows]
    assert_linear_close(y_s, ref, f"{cfg} {proj} M={m} (CPU oracle, {len(rows)} rows)")
    stats_cpu = error_stats(y_s, ref)
    if bias is not None:
        ref_order = ora.fp8_linear(recipe, x_s, w_cpu, s_cpu, b_cpu, bias_in_fp32=False, **kw).reshape(len(rows), n)
        gemm = ora.fp8_linear(recipe, x_s, w_cpu, s_cpu, None, **kw).reshape(len(rows), n)
        assert_linear_close(y_s, ref_order, f"{cfg} {proj} M={m} (reference bias order)",
                            extra=rounding_allowance(gemm, ref_order, torch.bfloat16))
    # On elements of at least a tenth of their row's maximum the bf16 output is within one
    # bf16 ulp (2^-7 relative) of the bf16-rounded oracle: max relative error <= 1e-2.
    for label, st in (("device oracle", stats_all), ("CPU oracle", stats_cpu)):
        assert st["max_rel_err_significant"] <= 1e-2, f"{cfg} {proj} M={m} ({label}): {st}"
        assert st["max_err_over_row_max"] <= 1e-2, f"{cfg} {proj} M={m} ({label}): {st}"
    _say(f"  all rows vs device oracle: {stats_all}; {len(rows)} rows vs CPU oracle: {stats_cpu}")
    record_parity(f"{cfg}/{proj}/M{m}", recipe=recipe, n=n, k=k, m=m, all_rows=stats_all,
                  cpu_rows=stats_cpu, cpu_row_count=len(rows),
                  quant_checked_bit_exact=recipe != "w8a16" and (m > 1 or recipe == "mxfp8"))
