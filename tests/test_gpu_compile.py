"""GPU: ``torch.compile(fullgraph=True)`` over ``FP8*LinearMethod.apply`` for every recipe.

The reference registers a fake (meta) kernel for every ``ayaka::*`` operator so that
compiled graphs can hold them (``kernel/ops.py:155-203``). Here the whole ``apply`` --
host validation, routing, activation quant and GEMM/GEMV operators -- is traced by
dynamo without a graph break, run through AOT autograd (fake-tensor propagation through
the registered fakes, functionalization of the ``_out`` variants), and the compiled
call must return the eager result bit for bit: both run the same HIP kernels.
"""

import sys

import pytest
import torch
from torch import nn

from tests.test_gpu_layers import CONFIGS, K, N, _checkpoint

pytestmark = pytest.mark.gpu


def _layer(recipe, gpu, g):
    from ayaka.layers.linear.fp8 import FP8Config

    w, s, _ = _checkpoint(recipe, g)
    method = FP8Config.from_config(CONFIGS[recipe]).get_quant_method(None, "model.layers.0.mlp.down_proj")
    layer = nn.Module()
    method.create_weights(layer, output_partition_sizes=[N], input_size_per_partition=K, device=gpu)
    layer.weight.data.copy_(w.to(gpu))
    param = getattr(layer, "weight_scale_inv" if recipe == "w8a8_block128" else "weight_scale")
    param.weight_loader(layer, param, s.to(gpu))
    if recipe == "w8a8_static_per_tensor":
        layer.input_scale.weight_loader(layer, layer.input_scale, torch.tensor(0.05, device=gpu))
    method.process_weights_after_loading(layer)
    return method, layer


@pytest.mark.parametrize("m", [1, 7, 64, 100])  # 100: the tiled GEMMs (block-128: column-major scales)
@pytest.mark.parametrize("recipe", list(CONFIGS))
def test_compiled_apply_matches_eager(gpu, recipe, m):
    print(f"torch.compile fullgraph recipe={recipe} m={m}", flush=True)
    sys.stdout.flush()
    torch._dynamo.reset()
    g = torch.Generator().manual_seed(7 * m + len(recipe))
    method, layer = _layer(recipe, gpu, g)
    x = torch.randn(m, K, generator=g).to(torch.bfloat16).to(gpu)
    bias = torch.randn(N, generator=g).to(torch.bfloat16).to(gpu)

    graphs = []

    def counting_backend(gm, example_inputs):
        graphs.append(gm)
        from torch._dynamo.backends.common import aot_autograd

        return aot_autograd(fw_compiler=lambda g_, _: g_)(gm, example_inputs)

    def fn(inp):
        return method.apply(layer, inp, bias)

    eager = fn(x)
    compiled = torch.compile(fn, fullgraph=True, backend=counting_backend)
    got = compiled(x)
    torch.cuda.synchronize()
    assert len(graphs) == 1, f"expected one graph, dynamo produced {len(graphs)}"
    targets = {str(n.target) for n in graphs[0].graph.nodes if n.op == "call_function"}
    assert any("ayaka" in t for t in targets), f"no ayaka operator in the traced graph: {sorted(targets)}"
    assert got.shape == eager.shape and got.dtype == eager.dtype
    assert torch.equal(got.view(torch.int16), eager.view(torch.int16)), f"{recipe} m={m}: compiled != eager"
    # A second call with new data reuses the compiled graph.
    x2 = torch.randn(m, K, generator=g).to(torch.bfloat16).to(gpu)
    assert torch.equal(compiled(x2).view(torch.int16), fn(x2).view(torch.int16))
    assert len(graphs) == 1
