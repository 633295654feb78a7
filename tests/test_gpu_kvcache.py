"""KV-cache writes and gathers (static per-tensor FP8 quantization) against the oracle:
bit-exact cache bytes for every source / cache dtype pair, masked slots, untouched
rows, gather with and without dequantization, and the reference's error contract."""

import sys

import pytest
import torch

from ayaka.utils.import_utils import CapabilityError
from oracle import fp8_oracle as ora

pytestmark = pytest.mark.gpu

CACHE_DTYPES = [torch.float8_e4m3fn, torch.float8_e5m2, torch.bfloat16, torch.float16]


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _source(n, heads, dim, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, heads, dim, generator=g) * 40
    flat = x.view(-1)
    special = torch.tensor([float("nan"), -float("nan"), float("inf"), -float("inf"), 1e6, -1e6, 3e-8, -5e-9, 0.0, -0.0])
    flat[: special.numel()] = special
    flat[special.numel(): special.numel() + 64] = torch.randn(64, generator=g) * 1e-5  # subnormal range
    return x.to(dtype)


def _bytes(t):
    return t.contiguous().view(torch.uint8) if t.dtype.itemsize == 1 else t.contiguous().view(torch.int16 if t.dtype.itemsize == 2 else torch.int32)


@pytest.mark.parametrize("cache_dtype", CACHE_DTYPES)
@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_write_kv_bit_exact(gpu, src_dtype, cache_dtype):
    from ayaka.kernel.hip import write_kv

    pages, page_size, heads, dim, n = 32, 16, 8, 128, 100
    _say(f"write_kv src={src_dtype} cache={cache_dtype}")
    key, value = _source(n, heads, dim, src_dtype, 1), _source(n, heads, dim, src_dtype, 2)
    g = torch.Generator().manual_seed(3)
    slots = torch.randperm(pages * page_size, generator=g)[:n]
    slots[::9] = -1  # masked padding tokens
    k_cache = torch.full((pages, page_size, heads, dim), 0.25).to(cache_dtype)
    v_cache = torch.full((pages, page_size, heads, dim), -0.5).to(cache_dtype)
    k_ref, v_ref = k_cache.clone(), v_cache.clone()
    ora.kv_write(key, k_ref, slots, 0.5)
    ora.kv_write(value, v_ref, slots, 3.0)
    kg, vg = k_cache.to(gpu), v_cache.to(gpu)
    write_kv(key.to(gpu), value.to(gpu), kg, vg, slots.to(gpu), 0.5, 3.0)
    assert torch.equal(_bytes(kg.cpu()), _bytes(k_ref)), "key cache differs"
    assert torch.equal(_bytes(vg.cpu()), _bytes(v_ref)), "value cache differs"


@pytest.mark.parametrize("cache_dtype", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_scatter_cache_one_plane_with_strided_source(gpu, cache_dtype):
    from ayaka.kernel.hip import scatter_cache

    _say(f"scatter_cache {cache_dtype}")
    pages, page_size, heads, dim, n = 8, 16, 4, 64, 40
    wide = _source(n, 2 * heads, dim, torch.bfloat16, 4)
    src = wide[:, :heads]  # every row strided: the key half of a fused qkv-like buffer
    slots = torch.randperm(pages * page_size, generator=torch.Generator().manual_seed(5))[:n]
    cache = torch.zeros(pages, page_size, heads, dim).to(cache_dtype)
    ref = cache.clone()
    ora.kv_write(src.contiguous(), ref, slots, 0.125)
    cg = cache.to(gpu)
    scatter_cache(src.to(gpu), cg, slots.to(gpu), 0.125)
    assert torch.equal(_bytes(cg.cpu()), _bytes(ref))


@pytest.mark.parametrize("cache_dtype", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("dest_dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_gather_cache_dequantize(gpu, cache_dtype, dest_dtype):
    from ayaka.kernel.hip import gather_cache

    _say(f"gather_cache {cache_dtype} -> {dest_dtype}")
    pages, page_size, heads, dim = 8, 16, 4, 64
    g = torch.Generator().manual_seed(6)
    cache = (torch.randn(pages, page_size, heads, dim, generator=g) * 30).to(cache_dtype)
    slots = torch.randint(0, pages * page_size, (50,), generator=g)  # repeats allowed
    ref = ora.kv_gather(cache, slots, dest_dtype, 0.75, True)
    dest = torch.empty(50, heads, dim, dtype=dest_dtype, device=gpu)
    gather_cache(cache.to(gpu), slots.to(gpu), dest, 0.75, True)
    assert torch.equal(_bytes(dest.cpu()), _bytes(ref.reshape(50, heads, dim)))
    raw = torch.empty(50, heads, dim, dtype=cache_dtype, device=gpu)
    gather_cache(cache.to(gpu), slots.to(gpu), raw, 1.0, False)
    assert torch.equal(_bytes(raw.cpu()), _bytes(ora.kv_gather(cache, slots, cache_dtype, 1.0, False).reshape(50, heads, dim)))


def test_kv_cache_contract(gpu):
    from ayaka.kernel.hip import gather_cache, write_kv

    _say("kv cache contract")
    key = torch.randn(4, 2, 8, device=gpu, dtype=torch.bfloat16)
    cache = torch.zeros(2, 4, 2, 8, device=gpu, dtype=torch.float8_e4m3fn)
    slots = torch.arange(4, device=gpu)
    with pytest.raises(ValueError, match="finite and positive"):
        write_kv(key, key, cache, cache.clone(), slots, 0.0, 1.0)
    with pytest.raises(ValueError, match="slot count"):
        write_kv(key[:3], key[:3], cache, cache.clone(), slots, 1.0, 1.0)
    with pytest.raises(ValueError, match="int64"):
        write_kv(key, key, cache, cache.clone(), slots.int(), 1.0, 1.0)
    with pytest.raises(CapabilityError):  # no CPU kernel is registered
        write_kv(key.cpu(), key.cpu(), cache.cpu(), cache.cpu(), slots.cpu(), 1.0, 1.0)
    with pytest.raises(ValueError, match="dequantize"):
        gather_cache(cache.to(torch.bfloat16), slots, torch.empty(4, 2, 8, device=gpu), 1.0, True)
