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


def _same(got, ref) -> bool:
    """Bit-identical, except that a NaN in a 16/32-bit float tensor may carry any payload
    (torch's own fp32 -> bf16 cast gives 0xFFFF on CPU, 0x7FC0 in its scalar code). fp8
    NaN encodings are fixed by the format and compared as bytes."""
    got, ref = got.cpu(), ref.cpu()
    if got.dtype.itemsize == 1:
        return torch.equal(_bytes(got), _bytes(ref))
    nan = torch.isnan(ref)
    return torch.equal(torch.isnan(got), nan) and torch.equal(_bytes(got)[~nan], _bytes(ref)[~nan])


@pytest.mark.parametrize("cache_dtype", CACHE_DTYPES)
@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_write_kv_bit_exact(gpu, src_dtype, cache_dtype):
    from ayaka.kernel.hip import write_kv

    pages, page_size, heads, dim, n = 32, 16, 8, 128, 100
    _say(f"write_kv src={src_dtype} cache={cache_dtype}")
    key, value = _source(n, heads, dim, src_dtype, 1), _source(n, heads, dim, src_dtype, 2)
    g = torch.Generator().manual_seed(3)
    slots = torch.randperm(pages * page_size, generator=g)[:n]
    slots[4::9] = -1  # masked padding tokens (token 0, holding the NaN/inf cases, is written)
    k_cache = torch.full((pages, page_size, heads, dim), 0.25).to(cache_dtype)
    v_cache = torch.full((pages, page_size, heads, dim), -0.5).to(cache_dtype)
    k_ref, v_ref = k_cache.clone(), v_cache.clone()
    ora.kv_write(key, k_ref, slots, 0.5)
    ora.kv_write(value, v_ref, slots, 3.0)
    kg, vg = k_cache.to(gpu), v_cache.to(gpu)
    write_kv(key.to(gpu), value.to(gpu), kg, vg, slots.to(gpu), 0.5, 3.0)
    assert _same(kg, k_ref), "key cache differs"
    assert _same(vg, v_ref), "value cache differs"


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
    assert _same(cg, ref)


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
    assert _same(dest, ref.reshape(50, heads, dim))
    raw = torch.empty(50, heads, dim, dtype=cache_dtype, device=gpu)
    gather_cache(cache.to(gpu), slots.to(gpu), raw, 1.0, False)
    assert _same(raw, ora.kv_gather(cache, slots, cache_dtype, 1.0, False).reshape(50, heads, dim))


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


# (heads, head_dim, source storage offset): width 15 and a source one element off a
# 16-byte boundary take the per-element kernels; width 16 the 8-element vector kernels.
LAYOUTS = [(3, 5, 0), (2, 8, 1), (2, 8, 0)]


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("cache_dtype", CACHE_DTYPES + [torch.float32])
@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float32])
def test_write_kv_ragged_and_unaligned_rows(gpu, src_dtype, cache_dtype, layout):
    from ayaka.kernel.hip import write_kv

    heads, dim, offset = layout
    _say(f"write_kv layout={layout} src={src_dtype} cache={cache_dtype}")
    pages, page_size, n = 6, 8, 33
    key, value = _source(n, heads, dim, src_dtype, 11), _source(n, heads, dim, src_dtype, 12)
    slots = torch.randperm(pages * page_size, generator=torch.Generator().manual_seed(13))[:n]
    slots[5] = -3
    k_cache = torch.zeros(pages, page_size, heads, dim).to(cache_dtype)
    v_cache = torch.ones(pages, page_size, heads, dim).to(cache_dtype)
    k_ref, v_ref = k_cache.clone(), v_cache.clone()
    ora.kv_write(key, k_ref, slots, 2.0)
    ora.kv_write(value, v_ref, slots, 0.03125)

    def shifted(x):  # same values, data pointer `offset` elements past an aligned base
        base = torch.empty(x.numel() + 8, dtype=x.dtype, device=gpu)
        view = base[offset: offset + x.numel()].view(x.shape)
        view.copy_(x.to(gpu))
        return view

    kg, vg = k_cache.to(gpu), v_cache.to(gpu)
    write_kv(shifted(key), shifted(value), kg, vg, slots.to(gpu), 2.0, 0.03125)
    assert _same(kg, k_ref), "key cache differs"
    assert _same(vg, v_ref), "value cache differs"


@pytest.mark.parametrize("layout", [(3, 5), (2, 8)])
@pytest.mark.parametrize("cache_dtype", CACHE_DTYPES)
def test_gather_cache_ragged_rows_and_same_dtype_copy(gpu, cache_dtype, layout):
    from ayaka.kernel.hip import gather_cache

    heads, dim = layout
    _say(f"gather_cache layout={layout} cache={cache_dtype}")
    pages, page_size = 4, 8
    g = torch.Generator().manual_seed(14)
    cache = _source(pages * page_size, heads, dim, torch.float32, 15).view(pages, page_size, heads, dim).to(cache_dtype)
    slots = torch.randint(0, pages * page_size, (21,), generator=g)
    cg, sg = cache.to(gpu), slots.to(gpu)
    same = torch.empty(21, heads, dim, dtype=cache_dtype, device=gpu)
    gather_cache(cg, sg, same, 1.0, False)
    ref = ora.kv_gather(cache, slots, cache_dtype, 1.0, False).reshape(21, heads, dim)
    assert _same(same, ref)
    if cache_dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
        deq = torch.empty(21, heads, dim, dtype=torch.bfloat16, device=gpu)
        gather_cache(cg, sg, deq, 0.375, True)
        ref = ora.kv_gather(cache, slots, torch.bfloat16, 0.375, True).reshape(21, heads, dim)
        assert _same(deq, ref)
    else:
        widened = torch.empty(21, heads, dim, dtype=torch.float32, device=gpu)
        gather_cache(cg, sg, widened, 1.0, False)
        ref = ora.kv_gather(cache, slots, torch.float32, 1.0, False).reshape(21, heads, dim)
        assert _same(widened, ref)


def _fp32_patterns(chunk: int, count: int, device) -> torch.Tensor:
    """fp32 values whose bit patterns are chunk * count .. (chunk + 1) * count - 1."""
    start = chunk * count
    start = start - (1 << 32) if start >= (1 << 31) else start  # int32 two's complement
    return (torch.arange(count, dtype=torch.int32, device=device) + start).view(torch.float32)


@pytest.mark.parametrize("cache_dtype", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_write_every_fp32_pattern(gpu, cache_dtype):
    """All 2^32 fp32 bit patterns through the vector write (inverse scale 1), against
    torch's clamp + round-to-nearest-even cast on the same device, in 2^28-element chunks."""
    from ayaka.kernel.hip import scatter_cache

    limit = torch.finfo(cache_dtype).max
    count, heads, dim = 1 << 28, 8, 128
    n = count // (heads * dim)
    slots = torch.arange(n, device=gpu)
    cache = torch.empty(n // 16, 16, heads, dim, dtype=cache_dtype, device=gpu)
    for chunk in range(1 << 4):
        _say(f"write_kv fp32 sweep {cache_dtype} chunk {chunk}")
        x = _fp32_patterns(chunk, count, gpu)
        scatter_cache(x.view(n, heads, dim), cache, slots, 1.0)
        ref = x.clamp(-limit, limit).to(cache_dtype)
        bad = int((cache.view(-1).view(torch.uint8) != ref.view(torch.uint8)).sum())
        assert bad == 0, f"{bad} codes differ in chunk {chunk}"
        del x, ref


@pytest.mark.parametrize("src_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cache_dtype", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_write_every_16bit_pattern(gpu, src_dtype, cache_dtype):
    """All 2^16 bf16 / fp16 patterns at two inverse scales, against the oracle."""
    from ayaka.kernel.hip import write_kv

    _say(f"write_kv 16-bit sweep {src_dtype} -> {cache_dtype}")
    x = torch.arange(1 << 16, dtype=torch.int32).to(torch.int16).view(src_dtype).view(64, 8, 128)
    slots = torch.arange(64)
    k_ref = torch.zeros(4, 16, 8, 128).to(cache_dtype)
    v_ref = k_ref.clone()
    ora.kv_write(x, k_ref, slots, 1.0)
    ora.kv_write(x, v_ref, slots, 0.3)
    kg, vg = k_ref.clone().zero_().to(gpu), v_ref.clone().zero_().to(gpu)
    write_kv(x.to(gpu), x.to(gpu), kg, vg, slots.to(gpu), 1.0, 0.3)
    assert torch.equal(_bytes(kg.cpu()), _bytes(k_ref))
    assert torch.equal(_bytes(vg.cpu()), _bytes(v_ref))


@pytest.mark.parametrize("cache_dtype", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("dest_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,heads,dim", [(37, 2, 128), (5000, 8, 128)])
def test_gather_fp8_to_16bit_rows_of_16(gpu, cache_dtype, dest_dtype, n, heads, dim):
    """fp8 cache into a 16-bit destination with rows of whole 16-element chunks (the
    16-byte-chunk gather), with out-of-range slots (zero rows), dequantized and plain."""
    from ayaka.kernel.hip import gather_cache

    _say(f"gather_cache wide n={n} width={heads * dim} {cache_dtype} -> {dest_dtype}")
    pages, page_size = 64, 16
    g = torch.Generator().manual_seed(21)
    cache = (torch.randn(pages, page_size, heads, dim, generator=g) * 30).to(cache_dtype)
    slots = torch.randint(0, pages * page_size, (n,), generator=g)
    slots[3] = -1
    slots[n // 2] = pages * page_size + 5
    cg, sg = cache.to(gpu), slots.to(gpu)
    for deq, scale in ((True, 0.75), (False, 1.0)):
        dest = torch.full((n, heads, dim), 7.0, dtype=dest_dtype, device=gpu)
        gather_cache(cg, sg, dest, scale, deq)
        valid = (slots >= 0) & (slots < pages * page_size)
        ref = ora.kv_gather(cache, torch.where(valid, slots, 0), dest_dtype, scale, deq).reshape(n, heads, dim)
        ref[~valid] = 0  # the kernel's contract for slots outside the cache: a zero row
        assert _same(dest, ref), f"dequantize={deq}"


def _kv_sweep_cases(n=24, seed=77):
    import random

    rng = random.Random(seed)
    cases = []
    for _ in range(n):
        heads, dim = rng.choice([(1, 8), (2, 24), (8, 64), (4, 128), (3, 40), (1, 576)])
        cases.append((rng.randint(1, 300), heads, dim, rng.choice([1, 8, 16, 32]),
                      rng.choice(["bfloat16", "float16", "float32"]),
                      rng.choice(["float8_e4m3fn", "float8_e5m2", "bfloat16", "float16"])))
    return cases


@pytest.mark.parametrize("n,heads,dim,page_size,src,cache", _kv_sweep_cases())
def test_kv_cache_shape_sweep(gpu, n, heads, dim, page_size, src, cache):
    """Seeded random token counts, head layouts, page sizes and dtype pairs: the write
    (masked slots included) and the dequantizing gather, bit-exact against the oracle."""
    from ayaka.kernel.hip import gather_cache, write_kv

    _say(f"kv sweep n={n} heads={heads} dim={dim} page={page_size} src={src} cache={cache}")
    src_dt, cache_dt = getattr(torch, src), getattr(torch, cache)
    g = torch.Generator().manual_seed(n * 31 + heads * 7 + dim)
    pages = -(-(n + 5) // page_size)
    key, value = _source(n, heads, dim, src_dt, n + 1), _source(n, heads, dim, src_dt, n + 2)
    slots = torch.randperm(pages * page_size, generator=g)[:n]
    slots[3::7] = -1
    k_cache = torch.full((pages, page_size, heads, dim), 0.25).to(cache_dt)
    v_cache = torch.full((pages, page_size, heads, dim), -0.5).to(cache_dt)
    k_ref, v_ref = k_cache.clone(), v_cache.clone()
    ora.kv_write(key, k_ref, slots, 0.5)
    ora.kv_write(value, v_ref, slots, 3.0)
    kg, vg = k_cache.to(gpu), v_cache.to(gpu)
    write_kv(key.to(gpu), value.to(gpu), kg, vg, slots.to(gpu), 0.5, 3.0)
    assert _same(kg, k_ref), "key cache differs"
    assert _same(vg, v_ref), "value cache differs"
    read = torch.randint(0, pages * page_size, (n,), generator=g)
    dest_dt = torch.bfloat16 if cache_dt.itemsize == 1 else cache_dt
    dequant = cache_dt.itemsize == 1
    dest = torch.empty(n, heads, dim, dtype=dest_dt, device=gpu)
    gather_cache(kg, read.to(gpu), dest, 0.75 if dequant else 1.0, dequant)
    ref = ora.kv_gather(k_ref, read, dest_dt, 0.75 if dequant else 1.0, dequant).reshape(n, heads, dim)
    assert _same(dest, ref), "gather differs"
