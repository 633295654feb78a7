"""GPU parity: the MoE FP8 block-128 grouped GEMM against the oracle.

Uneven experts (empty ones, single rows, ragged tails, more than one 128-row tile),
rows that no expert owns (must stay untouched), both pointer-table flavours
(``swap_ab``), the ``[E, K, N]`` transposed weight view, both output dtypes, and the
reference's error contract. Tolerance: the linear-path rule of ``tests/_tol.py``."""

import sys

import pytest
import torch

from oracle import fp8_oracle as ora
from tests._tol import assert_linear_close

pytestmark = pytest.mark.gpu
FP8 = torch.float8_e4m3fn


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _problem(counts, n, k, seed, gap_every=0):
    """Operands for experts with `counts` rows; `gap_every` > 0 leaves a free row after
    every such expert (owned by no expert)."""
    g = torch.Generator().manual_seed(seed)
    offsets, row = [], 0
    for i, c in enumerate(counts):
        offsets.append(row)
        row += c + (1 if gap_every and i % gap_every == 0 else 0)
    m_total, e = max(row, 1), len(counts)
    a = (torch.randn(m_total, k, generator=g) * 40).clamp(-448, 448).to(FP8)
    b = (torch.randn(e, n, k, generator=g) * 40).clamp(-448, 448).to(FP8)
    sa = torch.rand(m_total, k // 128, generator=g) * 1e-3 + 1e-4
    sb = torch.rand(e, n // 128, k // 128, generator=g) * 1e-3 + 1e-4
    ps = torch.tensor([[c, n, k] for c in counts], dtype=torch.int32).reshape(e, 3)
    off = torch.tensor(offsets, dtype=torch.int32)
    return a, b, sa, sb, ps, off


def _workspaces(e, device):
    i64 = lambda: torch.zeros(e, dtype=torch.int64, device=device)  # noqa: E731
    return dict(a_ptrs=i64(), b_ptrs=i64(), out_ptrs=i64(), a_scales_ptrs=i64(), b_scales_ptrs=i64(),
                layout_sfa=torch.zeros(e, 5, dtype=torch.int32, device=device),
                layout_sfb=torch.zeros(e, 5, dtype=torch.int32, device=device),
                workspace=torch.empty(1, dtype=torch.uint8, device=device))


def _run(gpu, a, b, sa, sb, ps, off, out_dtype, swap_ab=None, b_view=None):
    from ayaka.kernel.hip import fp8_blockwise_scaled_grouped_mm

    e, n, k = b.shape
    out = torch.full((a.shape[0], n), 3.0, dtype=out_dtype, device=gpu)
    ws = _workspaces(e, gpu)
    stride = lambda v: torch.full((e,), v, dtype=torch.int64, device=gpu)  # noqa: E731
    fp8_blockwise_scaled_grouped_mm(
        out, ws["a_ptrs"], ws["b_ptrs"], ws["out_ptrs"], ws["a_scales_ptrs"], ws["b_scales_ptrs"], a.to(gpu),
        b_view if b_view is not None else b.to(gpu), sa.to(gpu), sb.to(gpu), stride(k), stride(k), stride(n),
        ws["layout_sfa"], ws["layout_sfb"], ps.to(gpu), off.to(gpu), ws["workspace"], swap_ab=swap_ab)
    return out, ws


CASES = [
    # (counts, n, k, gap_every)
    ([0, 5, 130, 64], 256, 512, 0),
    ([1, 1, 2, 3, 0, 7, 1, 1], 384, 1024, 2),
    ([300, 17, 129], 512, 2048, 1),
    ([96] * 8, 2048, 7168, 0),
    ([3] * 70, 128, 256, 0),  # more experts than a wave has lanes
]


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_grouped_mm_matches_oracle(gpu, case, out_dtype):
    counts, n, k, gap = CASES[case]
    _say(f"grouped mm case={case} E={len(counts)} rows={sum(counts)} n={n} k={k} out={out_dtype}")
    a, b, sa, sb, ps, off = _problem(counts, n, k, seed=case, gap_every=gap)
    out, _ = _run(gpu, a, b, sa, sb, ps, off, out_dtype)
    sentinel = torch.full((a.shape[0], n), 3.0, dtype=out_dtype)
    ref = ora.grouped_blockwise_mm(a, b, sa, sb, ps, off, sentinel.float())
    owned = torch.zeros(a.shape[0], dtype=torch.bool)
    for c, o in zip(counts, off.tolist()):
        owned[o:o + c] = True
    got = out.cpu()
    assert torch.equal(got[~owned], sentinel[~owned]), "rows of no expert were written"
    if owned.any():
        assert_linear_close(got[owned], ref[owned], f"case {case}")


def test_grouped_mm_partial_experts(gpu):
    """Experts narrower and shorter than the operands: N_e < N (one not a multiple of 4,
    which the store tail writes element by element), K_e < K, with the
    scales addressed with row stride K_e / 128 as the reference's tables."""
    counts, n, k = [70, 3, 200], 512, 1024
    _say("grouped mm partial experts")
    a, b, sa, sb, _, off = _problem(counts, n, k, seed=21)
    ps = torch.tensor([[70, 510, 640], [3, 256, 1024], [200, 300, 896]], dtype=torch.int32)
    out, _ = _run(gpu, a, b, sa, sb, ps, off, torch.bfloat16)
    sentinel = torch.full((a.shape[0], n), 3.0, dtype=torch.bfloat16)
    ref = ora.grouped_blockwise_mm(a, b, sa, sb, ps, off, sentinel.float())
    got = out.cpu()
    for (m_e, n_e, _), o in zip(ps.tolist(), off.tolist()):
        assert torch.equal(got[o:o + m_e, n_e:], sentinel[o:o + m_e, n_e:]), "columns past N_e were written"
        assert_linear_close(got[o:o + m_e, :n_e], ref[o:o + m_e, :n_e], f"expert at {o}")


@pytest.mark.parametrize("swap_ab", [False, True])
def test_pointer_tables_and_transposed_weight_view(gpu, swap_ab):
    counts, n, k = [4, 0, 9], 256, 384
    _say(f"grouped mm tables swap_ab={swap_ab}")
    a, b, sa, sb, ps, off = _problem(counts, n, k, seed=11)
    b_t = b.to(gpu).transpose(1, 2)  # [E, K, N] view of [E][N][K] memory
    a_g = a.to(gpu)
    from ayaka.kernel.hip import fp8_blockwise_scaled_grouped_mm

    out = torch.zeros(a.shape[0], n, dtype=torch.bfloat16, device=gpu)
    ws = _workspaces(3, gpu)
    stride = lambda v: torch.full((3,), v, dtype=torch.int64, device=gpu)  # noqa: E731
    sa_g, sb_g = sa.to(gpu), sb.to(gpu)
    fp8_blockwise_scaled_grouped_mm(out, ws["a_ptrs"], ws["b_ptrs"], ws["out_ptrs"], ws["a_scales_ptrs"],
                                    ws["b_scales_ptrs"], a_g, b_t, sa_g, sb_g, stride(k), stride(k), stride(n),
                                    ws["layout_sfa"], ws["layout_sfb"], ps.to(gpu), off.to(gpu), ws["workspace"],
                                    swap_ab=swap_ab)
    ref = ora.grouped_blockwise_mm(a, b, sa, sb, ps, off, torch.zeros(a.shape[0], n))
    assert_linear_close(out.cpu(), ref, "transposed view")
    e = torch.arange(3)
    o = off.long()
    tok = (a_g.data_ptr() + o * k, sa_g.data_ptr() + o * (k // 128) * 4)
    wgt = (b_t.data_ptr() + e * k * n, sb_g.data_ptr() + e * (k * n // 128 // 128) * 4)
    (xa, xsa), (xb, xsb) = (wgt, tok) if swap_ab else (tok, wgt)
    assert ws["a_ptrs"].cpu().tolist() == xa.tolist() and ws["b_ptrs"].cpu().tolist() == xb.tolist()
    assert ws["a_scales_ptrs"].cpu().tolist() == xsa.tolist() and ws["b_scales_ptrs"].cpu().tolist() == xsb.tolist()
    assert ws["out_ptrs"].cpu().tolist() == (out.data_ptr() + o * n * 2).tolist()
    kb, nb = k // 128, n // 128
    rows_a = [nb] * 3 if swap_ab else counts
    rows_b = counts if swap_ab else [nb] * 3
    assert ws["layout_sfa"].cpu().tolist() == [[r, kb, 1, kb, r * kb] for r in rows_a]
    assert ws["layout_sfb"].cpu().tolist() == [[r, kb, 1, kb, r * kb] for r in rows_b]


def test_grouped_mm_contract(gpu):
    from ayaka.kernel.hip import fp8_blockwise_scaled_grouped_mm

    _say("grouped mm contract")
    a, b, sa, sb, ps, off = _problem([4, 4], 256, 256, seed=3)
    base = dict(a=a.to(gpu), b=b.to(gpu), sa=sa.to(gpu), sb=sb.to(gpu), ps=ps.to(gpu), off=off.to(gpu))

    def call(**over):
        d = dict(base, **over)
        e = d["b"].shape[0]
        ws = _workspaces(e, gpu)
        stride = torch.full((e,), 256, dtype=torch.int64, device=gpu)
        out = over.get("out", torch.empty(d["a"].shape[0], 256, dtype=torch.bfloat16, device=gpu))
        fp8_blockwise_scaled_grouped_mm(out, ws["a_ptrs"], ws["b_ptrs"], ws["out_ptrs"], ws["a_scales_ptrs"],
                                        ws["b_scales_ptrs"], d["a"], d["b"], d["sa"], d["sb"], stride, stride, stride,
                                        ws["layout_sfa"], ws["layout_sfb"], d["ps"], d["off"], ws["workspace"])

    with pytest.raises(ValueError, match="problem_sizes must be int32"):
        call(ps=base["ps"].long())
    with pytest.raises(ValueError, match="a must be kFloat8_e4m3fn"):
        call(a=base["a"].to(torch.bfloat16))
    with pytest.raises(ValueError, match="output must be bfloat16 or half"):
        call(out=torch.empty(8, 256, dtype=torch.float32, device=gpu))
    with pytest.raises(ValueError, match="scales_a must be float32"):
        call(sa=base["sa"].double())
    with pytest.raises(ValueError, match="must match expert_offsets"):
        call(off=base["off"][:1])
    with pytest.raises(ValueError, match="memory layout"):
        call(b=base["b"][:, :, :128].contiguous())
    with pytest.raises(ValueError, match="CUDA"):
        call(a=base["a"].cpu())


@pytest.mark.parametrize("partial", [False, True])
def test_grouped_mm_transposed_scales_match(gpu, monkeypatch, partial):
    """From COLUMN_MAJOR_SCALES_MIN_ROWS rows the wrapper hands the kernel a transposed
    copy of scales_a as well: experts over the whole K read it, others (K_e < K, whose
    rows the reference addresses with row stride K_e / 128) keep the original table.
    The output is bit-identical to the row-major-only launch."""
    import ayaka.kernel.hip.moe.moe_grouped_gemm as G

    counts, n, k = [130, 0, 77, 256, 5], 512, 1024
    _say(f"grouped mm transposed scales partial={partial}")
    a, b, sa, sb, ps, off = _problem(counts, n, k, seed=31)
    if partial:
        ps[2, 2] = 640  # expert 2 over K_e = 640 < K
    outs = []
    for rows in (1 << 40, 1):
        monkeypatch.setattr(G, "COLUMN_MAJOR_SCALES_MIN_ROWS", rows)
        out, _ = _run(gpu, a, b, sa, sb, ps, off, torch.bfloat16)
        outs.append(out.cpu())
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


def _random_cases(n_cases=12, seed=5):
    import random

    rng = random.Random(seed)
    cases = []
    for i in range(n_cases):
        e = rng.randint(1, 40)
        hi = rng.choice([4, 140, 300])
        counts = [0 if rng.random() < 0.15 else rng.randint(1, hi) for _ in range(e)]
        if i == n_cases - 1:  # enough rows for the column-major scale path
            counts = [rng.randint(90, 130) for _ in range(40)]
        cases.append((counts, 128 * rng.randint(1, 8), 128 * rng.randint(1, 16), rng.choice([0, 0, 1, 3])))
    return cases


RANDOM_CASES = _random_cases()


@pytest.mark.parametrize("case", range(len(RANDOM_CASES)))
def test_grouped_mm_random_experts(gpu, case):
    """Seeded random expert counts (empty experts included), N, K and free rows."""
    counts, n, k, gap = RANDOM_CASES[case]
    _say(f"grouped mm random case={case} E={len(counts)} rows={sum(counts)} n={n} k={k} gap={gap}")
    a, b, sa, sb, ps, off = _problem(counts, n, k, seed=100 + case, gap_every=gap)
    out, _ = _run(gpu, a, b, sa, sb, ps, off, torch.bfloat16)
    sentinel = torch.full((a.shape[0], n), 3.0, dtype=torch.bfloat16)
    ref = ora.grouped_blockwise_mm(a, b, sa, sb, ps, off, sentinel.float())
    owned = torch.zeros(a.shape[0], dtype=torch.bool)
    for c, o in zip(counts, off.tolist()):
        owned[o:o + c] = True
    got = out.cpu()
    assert torch.equal(got[~owned], sentinel[~owned]), "rows of no expert were written"
    if owned.any():
        assert_linear_close(got[owned], ref[owned], f"random case {case}")
