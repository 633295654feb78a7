"""GPU: FP8 checkpoint ingestion end to end. A packed q/k/v FP8 checkpoint on disk
(written with the ``safetensors`` library) -> ``load_fp8_linear`` streaming the
weights through pinned staging into HBM (a small staging size forces several
chunks per tensor) -> ``quant_method.apply`` at decode and prefill M, against the
CPU oracle's composition of the same recipe on the concatenated checkpoint tensors."""

import sys

import pytest
import torch

from oracle import fp8_oracle as ora
from tests._tol import assert_linear_close
from tests.test_checkpoint_ingest import CONFIGS, K, PARTS, QKV, write_fp8_checkpoint

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.mark.parametrize("m", [1, 40])
@pytest.mark.parametrize("recipe", list(CONFIGS))
def test_checkpoint_to_hbm_to_apply(gpu, tmp_path, recipe, m):
    from ayaka.model_loader.fp8_checkpoint import load_fp8_linear
    from ayaka.model_loader.reader import CheckpointReader

    _say(f"checkpoint ingestion recipe={recipe} m={m}")
    weights, scales, inputs = write_fp8_checkpoint(tmp_path, recipe, seed=m)
    with CheckpointReader(tmp_path, staging_bytes=1 << 20) as reader:
        layer = load_fp8_linear(reader, QKV, [p for p, _ in PARTS], device=gpu)
    assert layer.weight.device.type == "cuda"
    assert torch.equal(layer.weight.data.cpu().view(torch.uint8), torch.cat(weights).view(torch.uint8))
    n = sum(rows for _, rows in PARTS)
    w = torch.cat(weights)
    kw, input_scale = {}, None
    if recipe in ("w8a8_dynamic_per_tensor", "w8a8_static_per_tensor"):
        s_ref = torch.cat([s.expand(rows) for s, (_, rows) in zip(scales, PARTS)])
        input_scale = inputs[-1] if inputs else None
    elif recipe == "w8a16":
        s_ref = torch.cat(scales).reshape(n, 1)
        kw = dict(weight_block=None, scale_dtype="float32")
    else:
        s_ref = torch.cat(scales)
    g = torch.Generator().manual_seed(7 + m)
    x = torch.randn(m, K, generator=g).to(torch.bfloat16)
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    y = layer.quant_method.apply(layer, x.to(gpu), bias.to(gpu))
    ref = ora.fp8_linear(recipe, x, w, s_ref, bias, input_scale=input_scale, bias_in_fp32=True, **kw)
    assert_linear_close(y.reshape(m, n), ref, f"{recipe} m={m}")


def test_multi_chunk_stream_into_hbm(gpu, tmp_path):
    """A 5 MiB + 3 B tensor through 1 MiB staging buffers (6 chunks, the last short)
    lands in HBM byte for byte."""
    from safetensors.torch import save_file

    from ayaka.model_loader.reader import CheckpointReader

    _say("multi-chunk stream")
    g = torch.Generator().manual_seed(3)
    data = torch.randint(0, 256, ((5 << 20) + 3,), generator=g, dtype=torch.uint8)
    save_file({"pad": torch.ones(5, dtype=torch.uint8), "blob": data}, str(tmp_path / "model.safetensors"))
    with CheckpointReader(tmp_path, staging_bytes=1 << 20) as reader:
        out = reader.read("blob", gpu)
        torch.cuda.synchronize()
    assert torch.equal(out.cpu(), data)
