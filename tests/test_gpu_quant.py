"""GPU parity: the HIP quantizers are bit-exact against the CPU oracle.

Compares e4m3 bytes and scales exactly (``torch.equal`` on raw bits) for every
activation dtype, odd and large K, zero rows, outlier channels, and the MX exponent
boundary inputs (amax just above 448 * 2^k) where the ceiling of log2 decides.
"""

import sys

import pytest
import torch

from oracle import fp8_oracle as ora

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    a = a.cpu()
    b = b.cpu()
    if a.dtype == torch.float8_e4m3fn:
        a, b = a.view(torch.uint8), b.view(torch.uint8)
    elif a.dtype == torch.float32:
        a, b = a.view(torch.int32), b.view(torch.int32)
    return torch.equal(a, b)


def _activation(m: int, k: int, dtype: torch.dtype, seed: int, outliers: bool = True) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g)
    if outliers and k >= 100:
        idx = torch.randperm(k, generator=g)[: max(1, k // 100)]
        x[:, idx] *= 20.0
    if m > 2:
        x[1] = 0.0  # all-zero row: the 1e-10 floor / MX code 0
        x[2, : k // 2] = 0.0
    return x.to(dtype)


DTYPES = [torch.bfloat16, torch.float16, torch.float32]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,k", [(1, 1), (3, 7), (8, 1024), (5, 4104), (4, 18944), (2, 70000)])
def test_per_token_quant_bit_exact(gpu, dtype, m, k):
    from ayaka.kernel.hip import per_token_quant_fp8

    _say(f"per_token_quant_fp8 dtype={dtype} m={m} k={k}")
    x = _activation(m, k, dtype, seed=m * 1000 + k)
    q, s = per_token_quant_fp8(x.to(gpu))
    torch.cuda.synchronize()
    rq, rs = ora.per_token_quant(x)
    assert _bits_equal(s, rs), "scales differ"
    assert _bits_equal(q, rq), f"codes differ at {int((q.cpu().view(torch.uint8) != rq.view(torch.uint8)).sum())} positions"


def test_per_token_quant_strided_and_3d(gpu):
    from ayaka.kernel.hip import per_token_quant_fp8

    _say("per_token_quant_fp8 strided rows + 3-D input")
    base = _activation(6, 512, torch.bfloat16, seed=7)
    strided = base.to(gpu)[:, :256]  # row stride 512 > K
    q, s = per_token_quant_fp8(strided)
    rq, rs = ora.per_token_quant(base[:, :256])
    assert _bits_equal(q, rq) and _bits_equal(s, rs)
    x3 = _activation(6, 256, torch.bfloat16, seed=8).reshape(2, 3, 256)
    q3, s3 = per_token_quant_fp8(x3.to(gpu))
    rq3, rs3 = ora.per_token_quant(x3)
    assert q3.shape == (6, 256) and _bits_equal(q3, rq3) and _bits_equal(s3, rs3)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,k,group", [(1, 128, 128), (33, 7168, 128), (4, 18432, 128), (3, 64, 16), (2, 2048, 1024), (2, 8, 8), (3, 12, 4)])
def test_group_quant_bit_exact(gpu, dtype, m, k, group):
    from ayaka.kernel.hip import per_token_group_quant_fp8

    _say(f"per_token_group_quant_fp8 dtype={dtype} m={m} k={k} group={group}")
    x = _activation(m, k, dtype, seed=k + group)
    q, s = per_token_group_quant_fp8(x.to(gpu), group)
    rq, rs = ora.per_token_group_quant(x, group)
    assert _bits_equal(s, rs), "scales differ"
    assert _bits_equal(q, rq), "codes differ"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,k,group", [(300, 7168, 128), (65, 18432, 128), (3, 64, 16), (5, 12, 4), (1, 256, 128)])
def test_group_quant_column_major_scales(gpu, dtype, m, k, group):
    """The column-major variant writes the same codes and the same scales, transposed
    (vector kernel, and the scalar kernel for groups of fewer than 8 elements)."""
    from ayaka.kernel.hip.quant.fp8_quant import per_token_group_quant_fp8_colmajor

    _say(f"per_token_group_quant_fp8_colmajor dtype={dtype} m={m} k={k} group={group}")
    x = _activation(m, k, dtype, seed=3 * k + group)
    q, s_t = per_token_group_quant_fp8_colmajor(x.to(gpu), group)
    rq, rs = ora.per_token_group_quant(x, group)
    assert s_t.shape == (k // group, m) and s_t.is_contiguous()
    assert _bits_equal(s_t.t(), rs), "scales differ"
    assert _bits_equal(q, rq), "codes differ"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("m,k,group", [(1, 32, 32), (64, 8192, 32), (3, 28672, 32), (2, 96, 96), (2, 64, 64), (5, 40, 8)])
def test_mx_quant_bit_exact(gpu, dtype, m, k, group):
    from ayaka.kernel.hip import per_token_group_quant_mxfp8

    _say(f"per_token_group_quant_mxfp8 dtype={dtype} m={m} k={k} group={group}")
    g = torch.Generator().manual_seed(k)
    torch.manual_seed(k)
    x = (torch.distributions.StudentT(3.0).sample((m, k)) if m > 1 else torch.randn(m, k, generator=g)).to(dtype)
    if m > 2:
        x[1] = 0.0
    q, c = per_token_group_quant_mxfp8(x.to(gpu), group)
    rq, rc = ora.per_token_group_quant_mxfp8(x, group)
    assert torch.equal(c.cpu(), rc), "exponent codes differ"
    assert _bits_equal(q, rq), "codes differ"


def test_mx_quant_exponent_boundaries(gpu):
    """Groups whose amax / 448 sits on and up to 129 ulps above every power of two."""
    from ayaka.kernel.hip import per_token_group_quant_mxfp8

    _say("per_token_group_quant_mxfp8 exponent boundaries")
    ks = torch.arange(-133, 121, dtype=torch.float64)
    # every mantissa offset up to 129 (the bit-level exponent path starts at 64) and a few large ones
    ns = torch.cat([torch.arange(130, dtype=torch.float64), torch.tensor([1000.0, 2.0**22, 2.0**23 - 1])])
    amax = (448.0 * torch.exp2(ks)[:, None] * (1 + ns[None, :] * 2.0**-23)).reshape(-1).float()
    amax = amax[torch.isfinite(amax) & (amax > 0)]
    rows = amax.numel()
    g = torch.Generator().manual_seed(3)
    x = (torch.rand(rows, 32, generator=g) * 2 - 1) * amax[:, None]
    x[:, 5] = amax  # the group maximum, exactly
    x[:, 9] = -amax * 0.999
    q, c = per_token_group_quant_mxfp8(x.to(gpu), 32)
    rq, rc = ora.per_token_group_quant_mxfp8(x, 32)
    assert torch.equal(c.cpu(), rc), "exponent codes differ"
    assert _bits_equal(q, rq)


def _nan_aware_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Same NaN positions, identical bits elsewhere (a NaN's payload and sign are not
    part of the contract)."""
    a, b = a.cpu(), b.cpu()
    af, bf = a.float(), b.float()
    nan_a, nan_b = torch.isnan(af), torch.isnan(bf)
    if not torch.equal(nan_a, nan_b):
        return False
    view = torch.uint8 if a.dtype in (torch.float8_e4m3fn, torch.uint8) else torch.int32
    return torch.equal(a.view(view)[~nan_a], b.view(view)[~nan_b])


@pytest.mark.parametrize("dtype", DTYPES)
def test_dynamic_quant_nan_and_inf(gpu, dtype):
    """Rows and groups holding NaN or +-inf take the exact element-wise path; their
    neighbours the finite one. Codes, scales and MX exponents against the oracle."""
    from ayaka.kernel.hip import per_token_group_quant_fp8, per_token_group_quant_mxfp8, per_token_quant_fp8

    _say(f"dynamic quant NaN / inf dtype={dtype}")
    k = 1024 if dtype == torch.float32 else 9216  # 16-bit rows past 1024 vectors: one workgroup per row
    x = _activation(8, k, dtype, seed=11).float()
    x[0, 5] = float("nan")
    x[3, 700] = float("inf")
    x[4, 129] = -float("inf")
    x[4, 900] = float("nan")
    x[5, 0] = -0.0
    x = x.to(dtype)
    q, s = per_token_quant_fp8(x.to(gpu))
    rq, rs = ora.per_token_quant(x)
    assert _nan_aware_equal(s, rs) and _nan_aware_equal(q, rq), "per-token"
    q, s = per_token_group_quant_fp8(x.to(gpu), 128)
    rq, rs = ora.per_token_group_quant(x, 128)
    assert _nan_aware_equal(s, rs) and _nan_aware_equal(q, rq), "group-128"
    q, c = per_token_group_quant_mxfp8(x.to(gpu), 32)
    rq, rc = ora.per_token_group_quant_mxfp8(x, 32)
    assert torch.equal(c.cpu(), rc) and _nan_aware_equal(q, rq), "mxfp8"


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(1,), (5, 7), (64, 1024), (3, 4, 333)])
def test_static_quant_bit_exact(gpu, dtype, shape):
    from ayaka.kernel.hip import static_quant_fp8

    _say(f"static_quant_fp8 dtype={dtype} shape={shape}")
    g = torch.Generator().manual_seed(11)
    x = (torch.randn(*shape, generator=g) * 30).to(dtype)
    scale = torch.tensor(0.0371, dtype=torch.float32)
    q = static_quant_fp8(x.to(gpu), scale.to(gpu))
    assert q.shape == x.shape
    assert _bits_equal(q, ora.static_quant(x, scale))
    out = torch.empty(shape, dtype=torch.float8_e4m3fn, device=gpu)
    r = static_quant_fp8(x.to(gpu), scale.to(gpu), out=out)
    assert r is out and _bits_equal(out, ora.static_quant(x, scale))


def test_encode_every_fp32_neighbourhood(gpu):
    """Every e4m3 value, midpoint and their fp32 neighbours through static quant (scale 1)."""
    from ayaka.kernel.hip import static_quant_fp8

    _say("static_quant_fp8 codec sweep")
    vals = ora.e4m3_values(torch.arange(256, dtype=torch.uint8))
    fin = torch.sort(vals[torch.isfinite(vals) & (vals >= 0)]).values
    mids = (fin[1:] + fin[:-1]) / 2
    base = torch.cat([fin, mids, torch.tensor([464.0, 470.0, 479.9, 480.0, 1e-30, 2.0**-10, 3 * 2.0**-11])])
    bits = base.view(torch.int32)
    nb = torch.cat([bits - 1, bits, bits + 1]).clamp_min(0).view(torch.float32)
    x = torch.cat([nb, -nb, torch.tensor([float("nan"), float("inf"), -float("inf"), -0.0])])
    one = torch.ones((), dtype=torch.float32)
    q = static_quant_fp8(x.to(gpu), one.to(gpu))
    ref = ora.static_quant(x, one)
    qb, rb = q.cpu().view(torch.uint8), ref.view(torch.uint8)
    nan_r = torch.isnan(ref.float())
    assert torch.equal(torch.isnan(q.cpu().float()), nan_r)
    assert torch.equal(qb[~nan_r], rb[~nan_r])


@pytest.mark.parametrize("scale", [1.0, 0.3701171875, 7.3e-5])
def test_static_quant_every_fp32_pattern(gpu, scale):
    """All 2^32 fp32 bit patterns through static quant, against torch's IEEE division,
    clamp and round-to-nearest-even e4m3 cast on the same device, in 2^28 chunks. Scale 1
    pins the hardware conversion for every input; the other scales pin the quotient taken
    from a reciprocal with Markstein's correction, code for code."""
    from ayaka.kernel.hip import static_quant_fp8

    count = 1 << 28
    s = torch.tensor(scale, dtype=torch.float32, device=gpu)
    out = torch.empty(count, dtype=torch.float8_e4m3fn, device=gpu)
    for chunk in range(1 << 4):
        _say(f"static_quant_fp8 fp32 sweep scale={scale} chunk {chunk}")
        start = chunk * count
        start = start - (1 << 32) if start >= (1 << 31) else start
        x = (torch.arange(count, dtype=torch.int32, device=gpu) + start).view(torch.float32)
        static_quant_fp8(x.view(1 << 14, 1 << 14), s, out=out.view(1 << 14, 1 << 14))
        ref = (x / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        bad = int((out.view(torch.uint8) != ref.view(torch.uint8)).sum())
        assert bad == 0, f"{bad} codes differ in chunk {chunk}"
        del x, ref
