"""FP8 checkpoint ingestion on the CPU: safetensors header validation, payload reads,
sharded indexes, and packed FP8 linear layers loaded from a checkpoint directory.

Checkpoints are written with the ``safetensors`` library itself, an independent
implementation of the format: every tensor our reader returns must equal the one
``safetensors`` reads back, byte for byte. Corrupt headers are bytes literals, one
per refusal the reference's parser makes (``model_loader/st.py:100-331``)."""

import json
import struct

import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from ayaka.exceptions import CheckpointCorruptError, UnsupportedWeightFormatError
from ayaka.model_loader.fp8_checkpoint import load_fp8_linear
from ayaka.model_loader.reader import CheckpointReader
from ayaka.model_loader.st import parse_safetensors_header, read_safetensors_header
from ayaka.types import DType

FP8 = torch.float8_e4m3fn


def _tensors(g):
    return {
        "w8": (torch.randn(16, 32, generator=g) * 50).clamp(-448, 448).to(FP8),
        "codes": torch.randint(0, 255, (16, 1), generator=g, dtype=torch.uint8),
        "bf": torch.randn(3, 5, generator=g).to(torch.bfloat16),
        "f16": torch.randn(7, generator=g).to(torch.float16),
        "f32": torch.randn(2, 2, 2, generator=g),
        "i64": torch.arange(5, dtype=torch.int64),
        "e5": torch.randn(9, generator=g).to(torch.float8_e5m2),
        "scalar": torch.tensor(0.125),
        "empty": torch.empty(0, 4),
        "flags": torch.tensor([True, False, True]),
    }


def _bits(t):
    return t.contiguous().view(-1).view(torch.uint8) if t.numel() else torch.empty(0, dtype=torch.uint8)


def test_reader_matches_the_safetensors_library(tmp_path):
    tensors = _tensors(torch.Generator().manual_seed(0))
    path = tmp_path / "model.safetensors"
    save_file(tensors, str(path), metadata={"format": "pt", "producer": "test"})
    header = read_safetensors_header(path)
    assert dict(header.metadata) == {"format": "pt", "producer": "test"}
    assert header.tensor_keys == set(tensors)
    assert header.payload_bytes == sum(t.numel() * t.element_size() for t in tensors.values())
    by_key = {e.tensor_key: e for e in header.entries}
    assert by_key["w8"].dtype is DType.FP8_E4M3 and by_key["codes"].dtype is DType.UINT8
    assert by_key["scalar"].shape == () and by_key["scalar"].numel == 1
    with CheckpointReader(tmp_path) as reader, safe_open(str(path), "pt") as lib:
        for key in tensors:
            ours, theirs = reader.read(key), lib.get_tensor(key)
            assert ours.dtype == theirs.dtype and ours.shape == theirs.shape, key
            assert torch.equal(_bits(ours), _bits(theirs)), key
        # read_into a row slice of a larger tensor, and a same-size reinterpretation
        big = torch.zeros(20, 32, dtype=FP8)
        reader.read_into("w8", big[2:18])
        assert torch.equal(_bits(big[2:18]), _bits(tensors["w8"]))
        assert torch.equal(_bits(big[:2]), torch.zeros(64, dtype=torch.uint8))
        raw = torch.empty(16, 32, dtype=torch.uint8)
        reader.read_into("w8", raw)
        assert torch.equal(raw.view(-1), _bits(tensors["w8"]))
        with pytest.raises(ValueError, match="destination holds"):
            reader.read_into("w8", torch.empty(15, 32, dtype=FP8))
        with pytest.raises(ValueError, match="contiguous"):
            reader.read_into("w8", torch.empty(32, 16, dtype=FP8).t())
        with pytest.raises(KeyError, match="no tensor"):
            reader.entry("missing")


def _header(obj, *, payload=64, raw=None):
    text = raw if raw is not None else json.dumps(obj).encode()
    return dict(raw_header=text, file_uri="f", data_start=8 + len(text), file_size=8 + len(text) + payload)


def _entry(dtype="F32", shape=(2,), begin=0, end=8):
    return {"dtype": dtype, "shape": list(shape), "data_offsets": [begin, end]}


@pytest.mark.parametrize("case,error,match", [
    (dict(raw=b"\xff\xfe"), CheckpointCorruptError, "UTF-8"),
    (dict(raw=b"{not json"), CheckpointCorruptError, "not valid JSON"),
    (dict(raw=b"[1, 2]"), CheckpointCorruptError, "not an object"),
    (dict(raw=b'{"a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]},'
               b' "a": {"dtype": "F32", "shape": [1], "data_offsets": [4, 8]}}'), CheckpointCorruptError, "duplicate"),
    (dict(obj={"a": 3}), CheckpointCorruptError, "not an object"),
    (dict(obj={"a": _entry(dtype="Q7")}), CheckpointCorruptError, "unknown safetensors dtype"),
    (dict(obj={"a": _entry(dtype=4)}), CheckpointCorruptError, "not a string"),
    (dict(obj={"a": _entry(dtype="I4", shape=(4,), end=2)}), UnsupportedWeightFormatError, "sub-byte"),
    (dict(obj={"a": _entry(dtype="F4", shape=(4,), end=2)}), UnsupportedWeightFormatError, "sub-byte"),
    (dict(obj={"a": {"dtype": "F32", "shape": [True], "data_offsets": [0, 4]}}), CheckpointCorruptError, "list of ints"),
    (dict(obj={"a": {"dtype": "F32", "shape": "2", "data_offsets": [0, 8]}}), CheckpointCorruptError, "list of ints"),
    (dict(obj={"a": _entry(shape=(-2,))}), CheckpointCorruptError, "negative dim"),
    (dict(obj={"a": {"dtype": "F32", "shape": [2], "data_offsets": [0]}}), CheckpointCorruptError, r"\[begin, end\]"),
    (dict(obj={"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8.0]}}), CheckpointCorruptError, "integers"),
    (dict(obj={"a": _entry(begin=-8, end=0)}), CheckpointCorruptError, "negative data_offset"),
    (dict(obj={"a": _entry(begin=8, end=0)}), CheckpointCorruptError, "backwards"),
    (dict(obj={"a": _entry(end=12)}), CheckpointCorruptError, "require 8"),
    (dict(obj={"a": _entry(shape=(16,), end=64), "b": _entry(shape=(2,), begin=64, end=72)}),
     CheckpointCorruptError, "beyond the file size"),
    (dict(obj={"a": _entry(shape=(4,), begin=0, end=16), "b": _entry(shape=(2,), begin=8, end=16)}),
     CheckpointCorruptError, "overlaps"),
])
def test_header_refusals(case, error, match):
    with pytest.raises(error, match=match):
        parse_safetensors_header(**_header(case.get("obj"), raw=case.get("raw")))


def test_header_accepts_empty_tensors_and_metadata():
    h = parse_safetensors_header(**_header({
        "__metadata__": {"format": "pt"}, "z": _entry(shape=(0, 3), begin=0, end=0), "a": _entry(begin=0, end=8),
        "c": _entry(dtype="U8", shape=(3,), begin=8, end=11)}))
    assert [e.tensor_key for e in h.entries] == ["z", "a", "c"]
    assert h.metadata == (("format", "pt"),)
    assert h.entries[1].byte_offset == h.data_start and h.entries[2].end_offset == h.data_start + 11


def test_header_file_refusals(tmp_path):
    p = tmp_path / "x.safetensors"
    p.write_bytes(b"\x01\x02")
    with pytest.raises(CheckpointCorruptError, match="too small"):
        read_safetensors_header(p)
    p.write_bytes(struct.pack("<Q", 0))
    with pytest.raises(CheckpointCorruptError, match="length is 0"):
        read_safetensors_header(p)
    p.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(CheckpointCorruptError, match="refusing"):
        read_safetensors_header(p)
    p.write_bytes(struct.pack("<Q", 100) + b"{}")
    with pytest.raises(CheckpointCorruptError, match="but the file is"):
        read_safetensors_header(p)
    # a payload cut short after the header was written
    save_file({"w": torch.ones(64)}, str(p))
    data = p.read_bytes()
    p.write_bytes(data[:-8])
    with pytest.raises(CheckpointCorruptError, match="beyond the file size"):
        read_safetensors_header(p)


def test_sharded_index_and_conflicts(tmp_path):
    g = torch.Generator().manual_seed(1)
    a, b = torch.randn(4, generator=g), torch.randn(3, generator=g)
    save_file({"a": a}, str(tmp_path / "model-00001-of-00002.safetensors"))
    save_file({"b": b}, str(tmp_path / "model-00002-of-00002.safetensors"))
    index = {"metadata": {}, "weight_map": {"a": "model-00001-of-00002.safetensors", "b": "model-00002-of-00002.safetensors"}}
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(index))
    with CheckpointReader(tmp_path) as r:
        assert set(r.keys()) == {"a", "b"} and torch.equal(r.read("a"), a) and torch.equal(r.read("b"), b)
    # the same name in two shards
    save_file({"a": a}, str(tmp_path / "model-00002-of-00002.safetensors"))
    with pytest.raises(CheckpointCorruptError, match="stored in both"):
        CheckpointReader(tmp_path)
    index["weight_map"]["c"] = "../elsewhere.safetensors"
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(index))
    with pytest.raises(CheckpointCorruptError, match="not a file in the checkpoint directory"):
        CheckpointReader(tmp_path)
    index["weight_map"]["c"] = "model-00003-of-00003.safetensors"
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps(index))
    with pytest.raises(CheckpointCorruptError, match="missing"):
        CheckpointReader(tmp_path)
    with pytest.raises(CheckpointCorruptError, match="no such checkpoint"):
        CheckpointReader(tmp_path / "nowhere")
    (tmp_path / "empty").mkdir()
    with pytest.raises(CheckpointCorruptError, match="no safetensors checkpoint"):
        CheckpointReader(tmp_path / "empty")


# ------------------------------------------------------------------ FP8 ingestion
PARTS = (("q_proj", 256), ("k_proj", 128), ("v_proj", 128))
K = 256
QKV = "model.layers.0.self_attn.qkv_proj"
PARENT = "model.layers.0.self_attn"

CONFIGS = {
    "w8a8_rowwise": {"fp8_recipe": "w8a8_rowwise"},
    "w8a8_dynamic_per_tensor": {"quant_method": "fp8", "activation_scheme": "dynamic"},
    "w8a8_static_per_tensor": {"quant_method": "fp8", "activation_scheme": "static"},
    "w8a8_block128": {"quant_method": "fp8", "weight_block_size": [128, 128], "scale_format": "float32"},
    "mxfp8": {"quant_algo": "mxfp8"},
    "w8a16": {"quant_algo": "w8a16"},
}


def write_fp8_checkpoint(root, recipe, seed=0, inverse=False):
    """A packed-QKV FP8 checkpoint: returns (per-part weights, per-part scales as
    written, per-part input scales). ``inverse`` stores 1/scale with
    ``scale_direction: inverse`` in the config."""
    g = torch.Generator().manual_seed(seed)
    tensors, weights, scales, inputs = {}, [], [], []
    for name, rows in PARTS:
        w = (torch.randn(rows, K, generator=g) * 60).clamp(-448, 448).to(FP8)
        if recipe in ("w8a8_rowwise", "w8a16"):
            s = torch.rand(rows, generator=g) * 1e-3 + 1e-4
        elif recipe in ("w8a8_dynamic_per_tensor", "w8a8_static_per_tensor"):
            s = torch.rand((), generator=g) * 1e-3 + 1e-4
        elif recipe == "w8a8_block128":
            s = torch.rand(rows // 128, K // 128, generator=g) * 1e-3 + 1e-4
        else:
            s = torch.randint(110, 125, (rows, K // 32), generator=g, dtype=torch.uint8)
        stored = (1.0 / s) if inverse and s.dtype != torch.uint8 else s
        scale_name = "weight_scale_inv" if recipe == "w8a8_block128" else "weight_scale"
        tensors[f"{PARENT}.{name}.weight"] = w
        tensors[f"{PARENT}.{name}.{scale_name}"] = stored
        if recipe == "w8a8_static_per_tensor":
            x_s = torch.rand((), generator=g) * 0.01 + 0.01
            tensors[f"{PARENT}.{name}.input_scale"] = x_s
            inputs.append(x_s)
        weights.append(w)
        scales.append(s)
    tensors["model.layers.0.mlp.down_proj.weight"] = torch.randn(8, 8, generator=g).to(torch.bfloat16)
    save_file(tensors, str(root / "model.safetensors"))
    qc = dict(CONFIGS[recipe], ignored_layers=["model.layers.0.mlp"])
    if inverse:
        qc["scale_direction"] = "inverse"
    (root / "config.json").write_text(json.dumps({"model_type": "llama", "quantization_config": qc}))
    return weights, scales, inputs


@pytest.mark.parametrize("inverse", [False, True])
@pytest.mark.parametrize("recipe", list(CONFIGS))
def test_load_packed_qkv_from_checkpoint(tmp_path, recipe, inverse):
    if inverse and recipe == "mxfp8":
        pytest.skip("UE8M0 codes have no direction")
    weights, scales, inputs = write_fp8_checkpoint(tmp_path, recipe, inverse=inverse)
    with CheckpointReader(tmp_path) as reader:
        layer = load_fp8_linear(reader, QKV, [p for p, _ in PARTS], device="cpu")
        assert load_fp8_linear(reader, "model.layers.0.mlp.down_proj", device="cpu") is None  # ignored
    assert torch.equal(_bits(layer.weight.data), _bits(torch.cat(weights)))
    assert layer.layout.names == ("q_proj", "k_proj", "v_proj")
    if recipe in ("w8a8_rowwise", "w8a16"):
        expect = torch.cat(scales)
    elif recipe in ("w8a8_dynamic_per_tensor", "w8a8_static_per_tensor"):
        expect = torch.cat([s.expand(rows) for s, (_, rows) in zip(scales, PARTS)])
    elif recipe == "w8a8_block128":
        expect = torch.cat(scales)
    else:
        expect = torch.cat(scales)
    got = layer.weight_scale_inv if recipe == "w8a8_block128" else layer.weight_scale
    got = got.detach().reshape(expect.shape)
    if inverse:  # 1 / (1 / s) in fp32 is within an ulp of s
        torch.testing.assert_close(got.float(), expect.float(), rtol=2e-7, atol=0)
    else:
        assert torch.equal(got.to(expect.dtype), expect)
    if recipe == "w8a8_static_per_tensor":
        # the reference's loader takes each projection's scalar in turn: the last one stays
        torch.testing.assert_close(layer.input_scale.detach(), inputs[-1], rtol=2e-7 if inverse else 0, atol=0)


def test_ingestion_refusals(tmp_path):
    write_fp8_checkpoint(tmp_path, "w8a8_rowwise")
    with CheckpointReader(tmp_path) as reader:
        with pytest.raises(UnsupportedWeightFormatError, match="F8_E4M3"):
            load_fp8_linear(reader, "model.layers.0.mlp.down_proj", device="cpu",
                            config={"fp8_recipe": "w8a8_rowwise"})
        with pytest.raises(ValueError, match="missing scale tensors"):
            load_fp8_linear(reader, QKV, ["q_proj", "k_proj"], device="cpu",
                            config={"quant_method": "fp8", "weight_block_size": [128, 128]})
        with pytest.raises(KeyError, match="no tensor"):
            load_fp8_linear(reader, QKV, ["q_proj", "o_proj"], device="cpu")
    (tmp_path / "config.json").write_text(json.dumps({"model_type": "llama"}))
    with CheckpointReader(tmp_path) as reader, pytest.raises(CheckpointCorruptError, match="quantization_config"):
        load_fp8_linear(reader, QKV, ["q_proj"], device="cpu")
