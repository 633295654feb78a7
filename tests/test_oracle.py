"""Pin the CPU oracle (``oracle/fp8_oracle.py``) to independent facts.

The reference ships no FP8 golden vectors, so every oracle function is checked
against something other than its own formula: exhaustive codec tables built from
the e4m3 / UE8M0 bit layouts, nearest-value search by brute force, closed-form
known answers, fp64 loops on tiny shapes, and invariants chosen so that a dropped
term, a wrong index or a transposed operand fails at least one of them.
"""

import math

import pytest
import torch

from oracle import fp8_oracle as ora

FP8 = torch.float8_e4m3fn


def _e4m3_table() -> torch.Tensor:
    """All 256 e4m3fn values from the bit layout (1 sign, 4 exponent bias 7, 3 mantissa)."""
    vals = []
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e, m = (c >> 3) & 0xF, c & 7
        if e == 0xF and m == 7:
            vals.append(float("nan"))
        elif e == 0:
            vals.append(s * m * 2.0**-9)
        else:
            vals.append(s * (1 + m / 8) * 2.0 ** (e - 7))
    return torch.tensor(vals, dtype=torch.float64)


def _nearest_e4m3_codes(v: torch.Tensor) -> torch.Tensor:
    """Round-to-nearest-even onto the finite e4m3 grid by exhaustive search (|v| <= 448)."""
    table = _e4m3_table()
    codes = torch.arange(256)
    finite = ~torch.isnan(table)
    t, c = table[finite], codes[finite]
    d = (v.double()[:, None] - t[None, :]).abs()
    best = d.min(dim=1, keepdim=True).values
    cand = d == best
    # ties: the even mantissa (code bit 0 clear); among equal values (+0/-0) take the sign of v
    even = (c % 2 == 0)[None, :]
    pick = torch.where(cand & even, 1, 0) * 4 + cand.int() * 2
    sign_ok = ((c >= 128)[None, :] == (torch.signbit(v))[:, None])
    pick = pick + sign_ok.int()
    return c[pick.argmax(dim=1)]


def test_e4m3_decode_table():
    got = ora.e4m3_values(torch.arange(256, dtype=torch.uint8)).double()
    ref = _e4m3_table()
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    ok = ~torch.isnan(ref)
    assert torch.equal(got[ok], ref[ok])
    assert got[ok].max().item() == 448.0 and got[1].item() == 2.0**-9


def test_e4m3_encode_is_round_nearest_even():
    table = _e4m3_table()
    fin = torch.sort(table[~torch.isnan(table)].unique()).values
    mids = (fin[1:] + fin[:-1]) / 2
    g = torch.Generator().manual_seed(0)
    rnd = (torch.rand(20000, generator=g, dtype=torch.float64) * 2 - 1) * 448
    tiny = (torch.rand(5000, generator=g, dtype=torch.float64) * 2 - 1) * 2.0**-6
    v = torch.cat([fin, mids, -mids, rnd, tiny, torch.tensor([0.0, -0.0, 448.0, -448.0])]).float()
    got = v.to(FP8).view(torch.uint8).long()
    ref = _nearest_e4m3_codes(v)
    assert torch.equal(got, ref)


def test_e8m0_decode_table():
    codes = torch.arange(256, dtype=torch.uint8)
    got = ora.e8m0_values(codes).double()
    assert got[0].item() == 0.0 and math.isnan(got[255].item())
    for c in range(1, 255):
        assert got[c].item() == 2.0 ** (c - 127)


# ------------------------------------------------------------------ quantizers
def test_per_token_quant_known_answers():
    x = torch.zeros(3, 64)
    x[1, 5] = 3.0
    x[2] = -0.25
    x[2, 7] = 7.0
    q, s = ora.per_token_quant(x.to(torch.bfloat16))
    assert s[0].item() == torch.tensor(1e-10, dtype=torch.float32).item() / torch.tensor(448.0).item() or \
        s[0].item() == (torch.tensor(1e-10, dtype=torch.float32) / 448.0).item()
    assert torch.all(q[0].float() == 0)
    assert q[1, 5].float().item() == 448.0 and torch.all(q[1, :5].float() == 0)
    assert q[2, 7].float().item() == 448.0
    assert q[2, 0].float().item() == _e4m3_table()[_nearest_e4m3_codes(torch.tensor([-0.25 / (7.0 / 448)]))].item()


def test_per_token_quant_brute_force():
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(6, 200, generator=g) * torch.logspace(-3, 3, 6)[:, None]).to(torch.bfloat16)
    q, s = ora.per_token_quant(x)
    xf = x.double()
    for r in range(6):
        amax = max(xf[r].abs().max().item(), float(torch.tensor(1e-10, dtype=torch.float32)))
        scale = torch.tensor(amax, dtype=torch.float32) / torch.tensor(448.0)
        assert s[r].item() == scale.item()
        quot = (x[r].float() / scale).clamp(-448, 448)
        assert torch.equal(q[r].view(torch.uint8).long(), _nearest_e4m3_codes(quot))


def test_group_quant_equals_rowwise_per_group():
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(5, 512, generator=g) * 3).to(torch.bfloat16)
    x[2, 128:256] = 0
    q, s = ora.per_token_group_quant(x, 128)
    assert s.shape == (5, 4)
    for j in range(4):
        qj, sj = ora.per_token_quant(x[:, j * 128:(j + 1) * 128])
        assert torch.equal(s[:, j], sj)
        assert torch.equal(q[:, j * 128:(j + 1) * 128].view(torch.uint8), qj.view(torch.uint8))


def test_mx_quant_exponent_closed_form():
    ks = list(range(-120, 110, 7))
    rows = []
    expect = []
    for k in ks:
        for f, bump in ((1.0, 0), (1 + 2.0**-10, 1), (0.75, 0)):
            amax = 448.0 * 2.0**k * f
            r = torch.zeros(32, dtype=torch.float32)
            r[3] = amax
            rows.append(r)
            expect.append(max(-126, min(127, k + bump)) + 127)
    rows.append(torch.zeros(32))
    expect.append(0)
    x = torch.stack(rows)
    q, code = ora.per_token_group_quant_mxfp8(x, 32)
    assert code.reshape(-1).tolist() == expect
    assert torch.all(q[-1].view(torch.uint8) == 0)


def test_mx_quant_brute_force():
    """Exponent from a correctly rounded fp32 log2 (double log2, then fp32) and nearest e4m3."""
    torch.manual_seed(3)
    x = torch.distributions.StudentT(3.0).sample((8, 64)).float()
    x[5] = 0
    q, code = ora.per_token_group_quant_mxfp8(x, 32)
    for r in range(8):
        for gidx in range(2):
            grp = x[r, gidx * 32:(gidx + 1) * 32]
            amax = grp.abs().max().item()
            if amax == 0:
                assert code[r, gidx].item() == 0
                continue
            ratio = float(torch.tensor(amax, dtype=torch.float32) / torch.tensor(448.0))
            e = math.ceil(float(torch.tensor(math.log2(max(ratio, 1e-38)), dtype=torch.float32)))
            e = max(-126, min(127, e))
            assert code[r, gidx].item() == e + 127
            quot = (grp.double() / 2.0**e).clamp(-448, 448)
            assert torch.equal(q[r, gidx * 32:(gidx + 1) * 32].view(torch.uint8).long(), _nearest_e4m3_codes(quot))


def test_torch_log2_never_changes_the_mx_ceiling():
    """The oracle's fp32 log2 (torch) gives the same ceiling as a correctly rounded log2
    for every ratio within 4096 ulps above or below a power of two -- the only inputs
    where rounding can decide the exponent. The HIP kernel uses the correctly rounded form."""
    ks = torch.arange(-126, 128, dtype=torch.float64)
    ns = torch.arange(0, 4097, dtype=torch.float64)
    up = (torch.exp2(ks)[:, None] * (1 + ns[None, :] * 2.0**-23)).float().reshape(-1)
    dn = (torch.exp2(ks)[:, None] * (1 - ns[None, :] * 2.0**-24)).float().reshape(-1)
    r = torch.cat([up, dn])
    r = r[torch.isfinite(r)]
    cr = torch.tensor([math.log2(v) for v in r.double().tolist()], dtype=torch.float64).float()
    assert torch.equal(torch.ceil(torch.log2(r)), torch.ceil(cr))


def test_static_quant_divides():
    x = torch.tensor([1.0, -3.0, 1000.0, 0.3])
    s = torch.tensor(0.1)
    q = ora.static_quant(x, s)
    quot = (x / s).clamp(-448, 448)
    assert torch.equal(q.view(torch.uint8).long(), _nearest_e4m3_codes(quot))


# ------------------------------------------------------------------ GEMM / GEMV
def _rand_fp8(shape, seed, scale=8.0):
    return (torch.randn(*shape, generator=torch.Generator().manual_seed(seed)) * scale).clamp(-448, 448).to(FP8)


def test_scaled_mm_brute_force_and_invariants():
    a, w = _rand_fp8((3, 5), 1), _rand_fp8((4, 5), 2)
    sa, sb, bias = torch.tensor([0.5, 2.0, 0.25]), torch.tensor([1.0, 0.125, 4.0, 2.0]), torch.tensor([1.0, -1.0, 0.5, 0.0])
    y = ora.fp8_scaled_mm(a, w, sa, sb, bias)
    af, wf = a.double(), w.double()
    for i in range(3):
        for j in range(4):
            ref = sum(af[i, k] * wf[j, k] for k in range(5)) * sa[i].item() * sb[j].item() + bias[j].item()
            assert abs(y[i, j].item() - ref) <= 1e-5 * max(1.0, abs(ref))
    sa2 = sa.clone()
    sa2[1] *= 2
    y2 = ora.fp8_scaled_mm(a, w, sa2, sb, None)
    y1 = ora.fp8_scaled_mm(a, w, sa, sb, None)
    assert torch.equal(y2[1], 2 * y1[1]) and torch.equal(y2[0], y1[0])
    zero = torch.zeros(4, 5).to(FP8)
    assert torch.equal(ora.fp8_scaled_mm(a, zero, sa, sb, bias), bias.expand(3, 4))


def test_int8_matmul_exact_brute_force_and_past_fp32():
    g = torch.Generator().manual_seed(7)
    a = torch.randint(-128, 128, (3, 37), generator=g, dtype=torch.int8)
    w = torch.randint(-128, 128, (4, 37), generator=g, dtype=torch.int8)
    y = ora.int8_matmul_exact(a, w)
    for i in range(3):
        for j in range(4):
            assert y[i, j].item() == sum(int(a[i, k]) * int(w[j, k]) for k in range(37))
    # Sums above 2^24 stay exact (an fp32 accumulation would round them): 2048 products
    # of -128 * -127 plus one of 1 * 1 -> 33292289, odd and above 2^25.
    a2 = torch.full((1, 2049), -128, dtype=torch.int8)
    w2 = torch.full((1, 2049), -127, dtype=torch.int8)
    a2[0, -1], w2[0, -1] = 1, 1
    assert ora.int8_matmul_exact(a2, w2).item() == 2048 * 128 * 127 + 1
    assert (a2.float() @ w2.float().t()).item() != 2048 * 128 * 127 + 1  # what fp32 would give


def test_int8_scaled_mm_known_answers_and_invariants():
    a = torch.tensor([[1, -2, 3, 4], [127, -128, 0, 5]], dtype=torch.int8)
    w = torch.tensor([[1, 1, 1, 1], [2, 0, -1, 3], [-128, 127, 64, -64]], dtype=torch.int8)
    sa, sb = torch.tensor([0.5, 0.25]), torch.tensor([2.0, 1.0, 0.125])
    bias = torch.tensor([1.0, -1.0, 0.5])
    y = ora.int8_scaled_mm(a, w, sa, sb, bias)
    acc = [[6, 11, -128 - 254 + 192 - 256], [4, 254 + 15, -16256 - 16256 - 320]]
    for i in range(2):
        for j in range(3):
            assert y[i, j].item() == acc[i][j] * sa[i].item() * sb[j].item() + bias[j].item()
    # Row scale moves one row only; a zero weight leaves the bias.
    sa2 = sa.clone()
    sa2[0] *= 4
    assert torch.equal(ora.int8_scaled_mm(a, w, sa2, sb)[0], 4 * ora.int8_scaled_mm(a, w, sa, sb)[0])
    assert torch.equal(ora.int8_scaled_mm(a, torch.zeros_like(w), sa, sb, bias), bias.expand(2, 3))


def test_blockwise_mm_reduces_to_plain_and_brute_force():
    a, w = _rand_fp8((3, 300), 3), _rand_fp8((130, 300), 4)
    ones_a, ones_b = torch.ones(3, 3), torch.ones(2, 3)
    plain = a.double() @ w.double().t()
    assert torch.allclose(ora.fp8_blockwise_mm(a, w, ones_a, ones_b).double(), plain, rtol=1e-6, atol=1e-3)
    g = torch.Generator().manual_seed(5)
    sa, sb = torch.rand(3, 3, generator=g), torch.rand(2, 3, generator=g)
    y = ora.fp8_blockwise_mm(a, w, sa, sb)
    ref = torch.zeros(3, 130, dtype=torch.float64)
    for kb in range(3):
        lo, hi = kb * 128, min(300, kb * 128 + 128)
        part = a.double()[:, lo:hi] @ w.double()[:, lo:hi].t()
        ref += part * sa[:, kb].double()[:, None] * sb[torch.arange(130) // 128, kb].double()[None, :]
    assert torch.allclose(y.double(), ref, rtol=1e-5, atol=1e-3)
    y_cm = ora.fp8_blockwise_mm(a, w, sa.t().contiguous(), sb, a_scale_col_major=True)
    assert torch.equal(y, y_cm)


def test_mxfp8_mm_reduces_to_plain_and_brute_force():
    a, w = _rand_fp8((2, 64), 6), _rand_fp8((3, 64), 7)
    c127a, c127w = torch.full((2, 2), 127, dtype=torch.uint8), torch.full((3, 2), 127, dtype=torch.uint8)
    plain = a.double() @ w.double().t()
    assert torch.allclose(ora.mxfp8_scaled_mm(a, c127a, w, c127w).double(), plain, rtol=1e-6, atol=1e-4)
    ca = torch.tensor([[120, 130], [0, 127]], dtype=torch.uint8)
    cw = torch.tensor([[127, 125], [129, 0], [127, 127]], dtype=torch.uint8)
    y = ora.mxfp8_scaled_mm(a, ca, w, cw)
    for i in range(2):
        for j in range(3):
            ref = 0.0
            for g in range(2):
                sa = 0.0 if ca[i, g] == 0 else 2.0 ** (int(ca[i, g]) - 127)
                sw = 0.0 if cw[j, g] == 0 else 2.0 ** (int(cw[j, g]) - 127)
                ref += sum(a.double()[i, k].item() * w.double()[j, k].item() for k in range(g * 32, g * 32 + 32)) * sa * sw
            assert abs(y[i, j].item() - ref) <= 1e-5 * max(1.0, abs(ref))


@pytest.mark.parametrize("sdt", ["float32", "bfloat16", "e8m0"])
def test_weight_only_gemv_brute_force(sdt):
    n, k, by, bx = 5, 40, 2, 16
    w = _rand_fp8((n, k), 8)
    srs = 3
    if sdt == "e8m0":
        scale = torch.randint(120, 130, (3, srs), dtype=torch.uint8, generator=torch.Generator().manual_seed(9))
        sv = 2.0 ** (scale.double() - 127)
    else:
        scale = torch.rand(3, srs, generator=torch.Generator().manual_seed(9)).to(getattr(torch, sdt))
        sv = scale.double()
    x = torch.randn(k, generator=torch.Generator().manual_seed(10)).to(torch.bfloat16)
    y = ora.fp8_weight_only_gemv(x, w, scale, srs, by, bx, sdt)
    for j in range(n):
        ref = sum(x.double()[kk].item() * w.double()[j, kk].item() * sv[j // by, kk // bx].item() for kk in range(k))
        assert y[j].item() == torch.tensor(ref).float().to(torch.bfloat16).item()


def test_weight_only_gemm_rounds_dequantized_weight():
    n, k = 3, 8
    w = _rand_fp8((n, k), 11)
    scale = torch.tensor([[0.3], [0.7], [1.1]])
    x = torch.randn(2, k, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    y = ora.fp8_weight_only_gemm(x, w, scale, 1, 1, k, "float32")
    for i in range(2):
        for j in range(n):
            deq = [float(torch.tensor(w.double()[j, kk].item() * scale[j, 0].item()).float().to(torch.bfloat16)) for kk in range(k)]
            ref = sum(x.double()[i, kk].item() * deq[kk] for kk in range(k))
            assert abs(y[i, j].float().item() - ref) <= 2 ** -7 * abs(ref) + 1e-6


def test_blockwise_gemv_matches_blockwise_mm():
    a, w = _rand_fp8((1, 256), 13), _rand_fp8((130, 256), 14)
    g = torch.Generator().manual_seed(15)
    sa, sb, bias = torch.rand(1, 2, generator=g), torch.rand(2, 2, generator=g), torch.randn(130, generator=g)
    y1 = ora.fp8_blockwise_gemv(a.reshape(-1), w, sa.reshape(-1), sb, bias)
    y2 = ora.fp8_blockwise_mm(a, w, sa, sb, bias).reshape(-1)
    assert torch.allclose(y1, y2, rtol=1e-5, atol=1e-3)


def test_linear_dispatch_m1_equals_gemv_and_prefill_quantizes():
    n, k = 64, 256
    wf = torch.randn(n, k, generator=torch.Generator().manual_seed(16)) * 0.02
    scale = wf.abs().amax(dim=1) / 448
    w = (wf / scale[:, None]).to(FP8)
    x = torch.randn(1, k, generator=torch.Generator().manual_seed(17)).to(torch.bfloat16)
    y = ora.fp8_linear("w8a8_rowwise", x, w, scale)
    ref = ora.fp8_weight_only_gemv(x.reshape(-1), w, scale, 1, 1, k, "float32")
    assert torch.equal(y.reshape(-1), ref)
    x8 = torch.randn(8, k, generator=torch.Generator().manual_seed(18)).to(torch.bfloat16)
    q, s = ora.per_token_quant(x8)
    assert torch.equal(ora.fp8_linear("w8a8_rowwise", x8, w, scale), ora.fp8_scaled_mm(q, w, s, scale).to(torch.bfloat16))


def _e5m2_table() -> torch.Tensor:
    """All 256 e5m2 values from the bit layout (1 sign, 5 exponent bias 15, 2 mantissa)."""
    vals = []
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e, m = (c >> 2) & 0x1F, c & 3
        if e == 0x1F:
            vals.append(float("nan") if m else s * float("inf"))
        elif e == 0:
            vals.append(s * m * 2.0**-16)
        else:
            vals.append(s * (1 + m / 4) * 2.0 ** (e - 15))
    return torch.tensor(vals, dtype=torch.float64)


def test_kv_write_e5m2_is_clamped_round_nearest_even():
    """The oracle's e5m2 path (torch's cast after the clamp) against a brute-force nearest
    search on the e5m2 grid built from its bit layout: every finite value, every midpoint,
    values past the clamp and NaN."""
    table = _e5m2_table()
    finite = torch.isfinite(table)
    grid = table[finite].unique()
    mids = (grid[1:] + grid[:-1]) / 2
    v = torch.cat([grid, mids, torch.tensor([6.0e4, -7.0e4, 1e9, 2.0**-18, -(2.0**-17)])]).float()
    cache = torch.zeros(1, v.numel(), 1, 1, dtype=torch.float8_e5m2)
    ora.kv_write(v.reshape(-1, 1, 1), cache, torch.arange(v.numel()), 1.0)
    got = cache.flatten().view(torch.uint8).long()
    vc = v.double().clamp(-57344, 57344)
    codes = torch.arange(256)
    fin_codes = codes[finite]
    d = (vc[:, None] - table[finite][None, :]).abs()
    best = d.min(dim=1, keepdim=True).values
    cand = d == best
    even = (fin_codes % 2 == 0)[None, :]
    sign_ok = (fin_codes >= 128)[None, :] == torch.signbit(vc)[:, None]
    pick = (cand & even).int() * 4 + cand.int() * 2 + sign_ok.int()
    want = fin_codes[pick.argmax(dim=1)]
    assert torch.equal(got, want)
    nan_cache = torch.zeros(1, 2, 1, 1, dtype=torch.float8_e5m2)
    ora.kv_write(torch.tensor([float("nan"), -float("nan")]).reshape(2, 1, 1), nan_cache, torch.arange(2), 1.0)
    assert torch.isnan(nan_cache.float()).all()


def test_kv_write_scales_skips_negative_slots_and_gathers_back():
    x = torch.tensor([[[1.0, -2.0]], [[300.0, 0.5]], [[7.0, 8.0]]])
    cache = torch.zeros(2, 2, 1, 2, dtype=torch.float8_e4m3fn)
    ora.kv_write(x, cache, torch.tensor([3, -1, 0]), 2.0)  # token 1 masked
    flat = cache.float().reshape(4, 2)
    assert flat[3].tolist() == [2.0, -4.0] and flat[0].tolist() == [14.0, 16.0]
    assert flat[1].abs().sum() == 0 and flat[2].abs().sum() == 0
    big = torch.zeros(1, 1, 1, 2, dtype=torch.float8_e4m3fn)
    ora.kv_write(torch.tensor([[[1000.0, -1000.0]]]), big, torch.tensor([0]), 1.0)
    assert big.flatten().float().tolist() == [448.0, -448.0]  # clamped, not NaN
    back = ora.kv_gather(cache, torch.tensor([3, 3, 0]), torch.float32, 0.5, True)
    assert back.reshape(3, 2).tolist() == [[1.0, -2.0], [1.0, -2.0], [7.0, 8.0]]


def test_grouped_blockwise_mm_brute_force_and_expert_order():
    """The grouped oracle against a scalar fp64 sum written from the operator's formula
    out[m, n] = sum_kb sa[m, kb] * sb[e][n // 128][kb] * sum_{k in kb} a[m, k] b[e, n, k]
    on uneven experts (one empty, rows of no expert left alone), and invariance under a
    reordering of the experts' row ranges."""
    g = torch.Generator().manual_seed(21)
    E, n, k = 3, 128, 256
    counts, offsets = [2, 0, 2], [0, 2, 3]  # rows 2 and 5 belong to no expert
    m_total = 6
    a = (torch.randn(m_total, k, generator=g) * 40).clamp(-448, 448).to(ora.E4M3)
    b = (torch.randn(E, n, k, generator=g) * 40).clamp(-448, 448).to(ora.E4M3)
    sa = torch.rand(m_total, k // 128, generator=g) + 0.5
    sb = torch.rand(E, n // 128, k // 128, generator=g) + 0.5
    ps = torch.tensor([[c, n, k] for c in counts], dtype=torch.int32)
    off = torch.tensor(offsets, dtype=torch.int32)
    out = torch.full((m_total, n), 7.0)
    got = ora.grouped_blockwise_mm(a, b, sa, sb, ps, off, out)
    af, bf = a.double().tolist(), b.double().tolist()
    for e, (c, o) in enumerate(zip(counts, offsets)):
        for m in range(o, o + c):
            for col in range(0, n, 37):  # a spread of columns keeps the loop short
                want = 0.0
                for kb in range(k // 128):
                    dot = sum(af[m][kk] * bf[e][col][kk] for kk in range(kb * 128, kb * 128 + 128))
                    want += float(sa[m, kb]) * float(sb[e, col // 128, kb]) * dot
                assert abs(float(got[m, col]) - want) <= 1e-5 * abs(want) + 1e-3, (e, m, col)
    assert torch.equal(got[2], out[2]) and torch.equal(got[5], out[5])
    # experts laid out in the opposite row order give the same rows
    perm_off = torch.tensor([4, 6, 0], dtype=torch.int32)
    a2 = torch.cat([a[3:5], a[2:3], a[5:6], a[0:2]])  # rows: e2 at 0..1, e0 at 4..5
    sa2 = torch.cat([sa[3:5], sa[2:3], sa[5:6], sa[0:2]])
    got2 = ora.grouped_blockwise_mm(a2, b, sa2, sb, ps, perm_off, torch.zeros(6, n))
    assert torch.equal(got2[4:6], got[0:2]) and torch.equal(got2[0:2], got[3:5])
