"""CPU tests of the host side: recipe parsing, spec validation, layer lifecycle
(parameters, sentinels, scale loading, load-time validation), operator validators
and meta kernels, and the C ABI's exported symbols and argument checks.

Expected values are the reference's documented contracts
(``python/ayaka/model_loader/fp8.py``, ``weights/spec.py``, ``layers/linear/fp8.py``).
"""

import ctypes
import pathlib
import re
from types import SimpleNamespace

import pytest
import torch
from torch import nn

from ayaka.layers.linear import fp8 as L
from ayaka.model_loader import fp8 as ML
from ayaka.weights.spec import FP8Recipe, FP8RecipeSpec, FP8ScaleDirection, QuantSpec
from ayaka.types import DType

ROOT = pathlib.Path(__file__).resolve().parents[1]

# ------------------------------------------------------------------ recipe detection
RECIPE_TABLE = [
    ({"fp8_recipe": "w8a8_rowwise"}, FP8Recipe.W8A8_ROWWISE, torch.float32),
    ({"quant_method": "fp8", "activation_scheme": "dynamic"}, FP8Recipe.W8A8_DYNAMIC_PER_TENSOR, torch.float32),
    ({"quant_method": "fp8", "activation_scheme": "static"}, FP8Recipe.W8A8_STATIC_PER_TENSOR, torch.float32),
    ({"quant_method": "fp8", "activation_scheme": "dynamic", "weight_block_size": [128, 128]}, FP8Recipe.W8A8_BLOCK128, torch.bfloat16),
    ({"weight_block_size": [128, 128], "scale_format": "float32"}, FP8Recipe.W8A8_BLOCK128, torch.float32),
    ({"quant_algo": "MXFP8"}, FP8Recipe.MXFP8, torch.uint8),
    ({"weight_block_size": [1, 32]}, FP8Recipe.MXFP8, torch.uint8),
    ({"activation_scheme": "dynamic", "scale_dtype": "e8m0"}, FP8Recipe.MXFP8, torch.uint8),
    ({"quant_algo": "w8a16"}, FP8Recipe.W8A16, torch.float32),
    # weight-only wins over MX hints
    ({"activation_scheme": "none", "scale_format": "ue8m0", "weight_block_size": [1, 32]}, FP8Recipe.W8A16, torch.uint8),
    ({"activation_scheme": "weight_only", "scale_format": "bf16"}, FP8Recipe.W8A16, torch.bfloat16),
    ({"activation_scheme": "dynamic", "weight_scheme": "rowwise"}, FP8Recipe.W8A8_ROWWISE, torch.float32),
    ({"kv_cache_scheme": {"type": "float"}}, FP8Recipe.KV_CACHE, torch.float32),
    ({}, FP8Recipe.W8A8_DYNAMIC_PER_TENSOR, torch.float32),
]


@pytest.mark.parametrize("config,recipe,scale_dtype", RECIPE_TABLE)
def test_parse_fp8_config_recipes(config, recipe, scale_dtype):
    parsed = ML.parse_fp8_config(config)
    assert parsed.recipe.recipe is recipe
    assert parsed.scale_dtype is scale_dtype
    if recipe is FP8Recipe.KV_CACHE:
        assert parsed.quant is None
    else:
        assert parsed.quant.fp8_recipe is parsed.recipe and parsed.quant.weight_dtype is DType.FP8_E4M3


def test_parse_fp8_config_details():
    p = ML.parse_fp8_config({"activation_scheme": "dynamic"})
    assert p.recipe.amax_floor == 1e-10 and p.recipe.calibration_source is None
    p = ML.parse_fp8_config({"activation_scheme": "dynamic", "amax_floor": 1e-6, "ignored_layers": ["lm_head"]})
    assert p.recipe.amax_floor == 1e-6 and p.ignored_layers == ("lm_head",)
    p = ML.parse_fp8_config({"activation_scheme": "static"})
    assert p.recipe.amax_floor is None and p.recipe.calibration_source == "quantization_config"
    p = ML.parse_fp8_config({"weight_block_size": [128, 128], "weight_scale_inv": True})
    assert p.recipe.scale_direction is FP8ScaleDirection.INVERSE
    assert p.recipe.activation_block == (1, 128) and p.recipe.weight_block == (128, 128)
    p = ML.parse_fp8_config({"quant_algo": "w8a16", "weight_block_size": [1, 64], "scale_dtype": "uint8"})
    assert p.recipe.weight_block == (1, 64) and p.scale_dtype is torch.uint8


@pytest.mark.parametrize("config,exc,fragment", [
    ([("a", 1)], TypeError, "mapping"),
    ({"fp8_recipe": "w4a4"}, ValueError, "unknown fp8 recipe"),
    ({"weight_block_size": [64, 64]}, ValueError, "unsupported weight_block_size"),
    ({"quant_algo": "block", "weight_block_size": [64, 128]}, ValueError, "requires weight_block_size=[128, 128]"),
    ({"weight_block_size": [128]}, ValueError, "integer pair"),
    ({"scale_format": "fp16"}, ValueError, "unknown scale format"),
    ({"fp8_recipe": "mxfp8", "activation_scheme": "none"}, ValueError, "requires an activation scheme"),
])
def test_parse_fp8_config_errors(config, exc, fragment):
    with pytest.raises(exc, match=re.escape(fragment)):
        ML.parse_fp8_config(config)


def test_scale_keys_and_normalisation():
    assert ML.expected_scale_keys(FP8Recipe.W8A8_BLOCK128) == ("weight_scale_inv",)
    assert ML.expected_scale_keys(FP8Recipe.W8A8_STATIC_PER_TENSOR) == ("weight_scale", "input_scale")
    assert ML.expected_scale_keys(FP8Recipe.KV_CACHE) == ("k_scale", "v_scale")
    assert ML.classify_scale_key("model.layers.0.mlp.down_proj.weight_scale_inv") == "weight_scale_inv"
    assert ML.classify_scale_key("model.layers.0.self_attn.k_scale") == "kv_scale"
    assert ML.classify_scale_key("model.layers.0.mlp.down_proj.weight") is None
    ML.validate_scale_key_set(["a.weight", "a.weight_scale", "a.input_scale"], FP8Recipe.W8A8_STATIC_PER_TENSOR)
    with pytest.raises(ValueError, match="missing scale tensors"):
        ML.validate_scale_key_set(["a.weight_scale"], FP8Recipe.W8A8_BLOCK128)
    with pytest.raises(ValueError, match="unexpected scale tensor kind"):
        ML.validate_scale_key_set(["a.weight_scale", "a.input_scale"], FP8Recipe.W8A8_ROWWISE)
    s = torch.tensor([2.0, 4.0])
    assert torch.equal(ML.normalize_scale(s, direction=FP8ScaleDirection.INVERSE), torch.tensor([0.5, 0.25]))
    assert ML.normalize_scale(s, direction=FP8ScaleDirection.DEQUANT) is s
    codes = torch.tensor([127], dtype=torch.uint8)
    assert ML.normalize_scale(codes, direction=FP8ScaleDirection.INVERSE) is codes
    with pytest.raises(ValueError):
        ML.normalize_scale(torch.tensor([0.0]), direction=FP8ScaleDirection.INVERSE)
    blk = torch.arange(12.0).reshape(2, 6)
    assert torch.equal(ML.shard_scale_k(blk, rank=1, world_size=3), blk[:, 2:4])
    with pytest.raises(ValueError, match="must divide"):
        ML.shard_scale_k(blk, rank=0, world_size=4)
    assert ML.scale_blocks_for_k(300, 128) == 3


def test_recipe_spec_contract_violations():
    base = ML.parse_fp8_config({"weight_block_size": [128, 128], "scale_format": "float32"}).recipe
    fields = {f: getattr(base, f) for f in base.__dataclass_fields__}
    with pytest.raises(ValueError, match="requires activation scheme/block"):
        FP8RecipeSpec(**{**fields, "weight_block": (1, 32)})
    with pytest.raises(ValueError, match="amax_floor must be finite"):
        FP8RecipeSpec(**{**fields, "amax_floor": float("inf")})
    with pytest.raises(ValueError, match="recipe must be one of"):
        FP8RecipeSpec(**{**fields, "recipe": "int4"})
    with pytest.raises(ValueError, match="duplicates"):
        FP8RecipeSpec(**{**fields, "excluded_layers": ("a", "a")})
    with pytest.raises(ValueError, match="FP8 QuantSpec requires"):
        QuantSpec(method="fp8")
    with pytest.raises(ValueError, match="scale_dtype=fp32"):
        QuantSpec(method="fp8", weight_dtype=DType.FP8_E4M3, scale_dtype=DType.BF16, fp8_recipe=base)
    assert '"recipe":"w8a8_block128"' in base.cache_key


# ------------------------------------------------------------------ layer lifecycle
def _layer(method, n=256, k=256, parts=None):
    layer = nn.Module()
    method.create_weights(layer, output_partition_sizes=parts or [n], input_size_per_partition=k,
                          device="cpu", weight_loader=lambda *a: None)
    return layer


@pytest.mark.parametrize("method,name,shape,dtype", [
    (L.FP8PerTensorLinearMethod("static"), "weight_scale", (256,), torch.float32),
    (L.FP8RowwiseLinearMethod(), "weight_scale", (256,), torch.float32),
    (L.FP8BlockLinearMethod(), "weight_scale_inv", (2, 2), torch.bfloat16),
    (L.FP8BlockLinearMethod(torch.float32), "weight_scale_inv", (2, 2), torch.float32),
    (L.FP8W8A16LinearMethod(), "weight_scale", (256, 1), torch.float32),
    (L.FP8W8A16LinearMethod(torch.uint8, (1, 32)), "weight_scale", (256, 8), torch.uint8),
    (L.FP8Mxfp8LinearMethod(), "weight_scale", (256, 8), torch.uint8),
])
def test_create_weights_layout_and_sentinels(method, name, shape, dtype):
    layer = _layer(method)
    assert layer.weight.shape == (256, 256) and layer.weight.dtype is torch.float8_e4m3fn
    scale = getattr(layer, name)
    assert tuple(scale.shape) == shape and scale.dtype is dtype
    assert scale.weight_loader is L._scale_loader
    if dtype is torch.uint8:
        assert torch.all(scale == 0xFF)
    else:
        assert torch.isnan(scale.float()).all()
    with pytest.raises(ValueError, match="not loaded from the checkpoint"):
        method.process_weights_after_loading(layer)


def test_process_weights_rejects_bad_scales_and_records_uniformity():
    m = L.FP8PerTensorLinearMethod("static")
    layer = _layer(m, n=4, k=32)
    layer.weight_scale.data.fill_(0.5)
    with pytest.raises(ValueError, match="input_scale not loaded"):
        m.process_weights_after_loading(layer)
    layer.input_scale.data.fill_(0.1)
    m.process_weights_after_loading(layer)
    assert layer._fp8_uniform_scale is True
    layer.weight_scale.data[1] = float("inf")
    with pytest.raises(ValueError, match="must be finite"):
        m.process_weights_after_loading(layer)
    layer.weight_scale.data[1] = -1.0
    with pytest.raises(ValueError, match="must be positive"):
        m.process_weights_after_loading(layer)
    mx = L.FP8Mxfp8LinearMethod()
    lmx = _layer(mx, n=4, k=64)
    lmx.weight_scale.data.fill_(127)
    mx.process_weights_after_loading(lmx)
    lmx.weight_scale.data[0, 0] = 0xFF
    with pytest.raises(ValueError, match="not loaded"):
        mx.process_weights_after_loading(lmx)
    with pytest.raises(ValueError, match="divisible by 32"):
        _layer(L.FP8Mxfp8LinearMethod(), n=4, k=48)


def test_scale_loader_broadcast_and_packed_projections():
    m = L.FP8RowwiseLinearMethod()
    layer = _layer(m, n=6, k=32)
    L._scale_loader(layer, layer.weight_scale, torch.tensor(0.25))
    assert torch.all(layer.weight_scale == 0.25)
    # packed gate/up with per-projection row slices
    part = lambda name, off, size: SimpleNamespace(name=name, local_offset=off, local_size=size)  # noqa: E731
    parts = {"gate": part("gate", 0, 2), "up": part("up", 2, 4)}

    class Layout:
        @property
        def names(self):
            return tuple(parts)

        def __getitem__(self, key):
            return parts[key]

    layer.layout = Layout()
    L._scale_loader(layer, layer.weight_scale, torch.tensor([1.0, 2.0]), "gate")
    L._scale_loader(layer, layer.weight_scale, torch.tensor(3.0), "up")
    assert layer.weight_scale.tolist() == [1.0, 2.0, 3.0, 3.0, 3.0, 3.0]
    # block scales narrow by 128-row blocks
    b = L.FP8BlockLinearMethod(torch.float32)
    bl = _layer(b, n=384, k=256)
    parts = {"q": part("q", 0, 128), "kv": part("kv", 128, 256)}
    bl.layout = Layout()
    L._scale_loader(bl, bl.weight_scale_inv, torch.full((1, 2), 0.5), "q")
    L._scale_loader(bl, bl.weight_scale_inv, torch.full((2, 2), 0.25), "kv")
    assert bl.weight_scale_inv.tolist() == [[0.5, 0.5], [0.25, 0.25], [0.25, 0.25]]
    with pytest.raises(L.WeightLoadError, match="does not fit"):
        L._scale_loader(bl, bl.weight_scale_inv, torch.ones(3), "q")


def test_fp8_config_method_selection():
    for config, cls in [({"activation_scheme": "static"}, L.FP8PerTensorLinearMethod),
                        ({"activation_scheme": "dynamic"}, L.FP8PerTensorLinearMethod),
                        ({"fp8_recipe": "w8a8_rowwise"}, L.FP8RowwiseLinearMethod),
                        ({"weight_block_size": [128, 128]}, L.FP8BlockLinearMethod),
                        ({"quant_algo": "w8a16"}, L.FP8W8A16LinearMethod),
                        ({"quant_algo": "mxfp8"}, L.FP8Mxfp8LinearMethod)]:
        cfg = L.FP8Config.from_config({**config, "ignored_layers": ["model.lm_head"]})
        assert isinstance(cfg.get_quant_method(None, "model.layers.0.mlp"), cls)
        assert cfg.get_quant_method(None, "model.lm_head") is None
        assert cfg.get_quant_method(None, "model.lm_head.sub") is None
        assert cfg.get_capabilities().weight_bits == 8
        # The reference reports {"cpu", "cuda"} (layers/linear/fp8.py:193); this package
        # has no CPU path, so its methods report "cuda" only (a documented divergence).
        assert cfg._make_method().get_capabilities().supported_devices == frozenset({"cuda"})
    assert L.FP8Config.from_config({"weight_block_size": [128, 128]}).scale_dtype is torch.bfloat16
    assert isinstance(L.FP8Config("w8a8_block128", scale_dtype=torch.float32)._make_method(), L.FP8BlockLinearMethod)
    with pytest.raises(L.CapabilityError):
        L.FP8Config("kv_cache").get_quant_method(None, "x")
    with pytest.raises(ValueError):
        L.FP8PerTensorLinearMethod("sometimes")
    with pytest.raises(ValueError):
        L.FP8BlockLinearMethod(torch.float16)


# ------------------------------------------------------------------ operator validators
def test_ops_reject_cpu_tensors_with_capability_error():
    import ayaka.kernel.hip as H
    from ayaka.utils.import_utils import CapabilityError

    x = torch.randn(4, 64).to(torch.bfloat16)
    with pytest.raises(CapabilityError):
        H.per_token_quant_fp8(x)
    # the Python bodies validate like the reference
    with pytest.raises(ValueError, match="x must be a CUDA tensor"):
        H.per_token_quant_fp8.kernel(x)
    with pytest.raises(TypeError, match="x must have dtype"):
        H.per_token_quant_fp8.kernel(torch.zeros(4, 8, dtype=torch.int32))
    w = torch.zeros(8, 64).to(torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="must be a CUDA tensor"):
        H.fp8_scaled_mm.kernel(w, w.t(), torch.tensor(1.0), torch.tensor(1.0))
    with pytest.raises(TypeError, match="input must have dtype"):
        H.fp8_weight_only_gemv.kernel(torch.zeros(64), w, torch.ones(8))


def test_meta_kernels_give_output_shapes():
    import ayaka.kernel.hip  # noqa: F401

    ops = torch.ops.ayaka
    x = torch.empty(2, 3, 256, device="meta", dtype=torch.bfloat16)
    q, s = ops.per_token_group_quant_fp8(x, 128)
    assert q.shape == (6, 256) and s.shape == (6, 2) and q.dtype is torch.float8_e4m3fn
    q, c = ops.per_token_group_quant_mxfp8(x, 32)
    assert c.shape == (6, 8) and c.dtype is torch.uint8
    a = torch.empty(6, 256, device="meta", dtype=torch.float8_e4m3fn)
    w = torch.empty(512, 256, device="meta", dtype=torch.float8_e4m3fn)
    y = ops.fp8_scaled_mm(a, w.t(), torch.empty((), device="meta"), torch.empty((), device="meta"))
    assert y.shape == (6, 512) and y.dtype is torch.float32
    y = ops.fp8_weight_only_gemv(torch.empty(256, device="meta", dtype=torch.bfloat16), w, torch.empty(512, 1, device="meta"))
    assert y.shape == (512,) and y.dtype is torch.bfloat16


def test_reference_mode_is_refused(monkeypatch):
    import ayaka.kernel.hip as H
    from ayaka.kernel.ops import force_reference
    from ayaka.utils.import_utils import CapabilityError

    monkeypatch.setenv("AYAKA_FORCE_REFERENCE_OPS", "1")
    with pytest.raises(CapabilityError, match="no plain-torch reference mode"):
        H.per_token_quant_fp8(torch.zeros(1, 8))
    with pytest.raises(CapabilityError):
        with force_reference():
            pass


# ------------------------------------------------------------------ C ABI
def _header_symbols():
    text = (ROOT / "include" / "ayaka_fp8.h").read_text()
    return sorted(set(re.findall(r"\b(ayk_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    from ayaka.kernel.hip import _lib

    lib = _lib.load_library()
    syms = _header_symbols()
    assert len(syms) >= 15
    for name in syms:
        assert hasattr(lib, name), f"{name} declared in include/ayaka_fp8.h but not exported"
    assert set(syms) == set(_lib.SIGNATURES), "ctypes prototypes must cover exactly the header"
    assert lib.ayk_abi_version() == 100


def test_c_abi_rejects_bad_arguments_without_a_gpu():
    from ayaka.kernel.hip import _lib

    lib = _lib.load_library()
    assert lib.ayk_per_token_quant_fp8(None, _lib.AYK_BF16, 4, 0, 0, None, 0, None, None) == _lib.AYK_EINVAL
    assert b"bad shape" in lib.ayk_last_error()
    assert lib.ayk_per_token_group_quant_fp8(None, _lib.AYK_BF16, 4, 128, 128, 96, None, 128, None, None) == _lib.AYK_EINVAL
    assert b"power of two" in lib.ayk_last_error()
    # scale strides that describe neither [rows, k/group] nor [k/group, rows]
    assert lib.ayk_per_token_group_quant_fp8_strided(None, _lib.AYK_BF16, 4, 256, 256, 128, None, 256, None, 1, 1,
                                                     None) == _lib.AYK_EINVAL
    assert b"scale strides" in lib.ayk_last_error()
    assert lib.ayk_per_token_group_quant_fp8_strided(None, _lib.AYK_BF16, 4, 256, 256, 128, None, 256, None, 2, 3,
                                                     None) == _lib.AYK_EINVAL
    assert lib.ayk_fp8_scaled_mm(None, 40, None, 40, 4, 4, 40, None, 0, 0, None, 0, 0, None, 0, None, 2, 4, None, 0, None) == _lib.AYK_EINVAL
    assert b"multiple of 16" in lib.ayk_last_error()
    assert lib.ayk_mxfp8_scaled_mm(None, 48, None, 1, None, 48, None, 1, 2, 2, 48, None, 0, None, 2, 2, None, 0, None) == _lib.AYK_EINVAL
    assert lib.ayk_mxfp8_scaled_mm_workspace_bytes(64, 8192, 28672) > 0
    # the decode-batch kernel's grid split (Llama-3-70B down at M = 64: 64 workgroups x 4)
    assert lib.ayk_mxfp8_scaled_mm_workspace_bytes(64, 8192, 28672) >= 4 * 64 * 8192 * 4
    assert lib.ayk_fp8_blockwise_mm_workspace_bytes(32, 7168, 18432) >= 4 * 32 * 7168 * 4
    assert lib.ayk_fp8_weight_only_gemv(None, _lib.AYK_F32, None, 16, 4, 16, None, 0, 1, 1, 16, None, None, 0, None) == _lib.AYK_EINVAL
    # zero-sized problems are no-ops that succeed without touching a device
    assert lib.ayk_per_token_quant_fp8(None, _lib.AYK_BF16, 0, 16, 16, None, 16, None, None) == _lib.AYK_OK
    assert lib.ayk_fp8_weight_only_gemv_workspace_bytes(512, 14336) > 0  # split-K shape
    assert lib.ayk_fp8_weight_only_gemv_workspace_bytes(28672, 4096) == 0
    # GEMM split-K plans: too few tiles split K, a full round does not
    assert lib.ayk_fp8_scaled_mm_workspace_bytes(512, 3584, 18944) > 0
    assert lib.ayk_fp8_scaled_mm_workspace_bytes(4096, 28672, 4096) == 0  # seven whole rounds of tiles
    # 2368 tiles: a last round of 64 tiles split four ways over K (256 x 256 fp32 each)
    assert lib.ayk_fp8_scaled_mm_workspace_bytes(4096, 37888, 3584) == 4 * 64 * 256 * 256 * 4
    assert lib.ayk_fp8_scaled_mm_workspace_bytes(8192, 37888, 3584) == 0  # a two-way tail split does not pay
    assert lib.ayk_int8_scaled_mm_workspace_bytes(512, 768, 8192) == 0  # INT8 never splits K
    # block-128 size query mirrors the launch: N < 128 at M <= 64 still splits K
    assert lib.ayk_fp8_blockwise_mm_workspace_bytes(16, 64, 4096) > 0
    assert lib.ayk_fp8_blockwise_mm_workspace_bytes(40, 96, 8192) > 0
    assert lib.ayk_fp8_blockwise_mm_workspace_bytes(32, 7168, 18432) > 0
    assert lib.ayk_fp8_blockwise_mm_workspace_bytes(4096, 18432, 7168) == 0
