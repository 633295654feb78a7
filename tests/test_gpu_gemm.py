"""GPU parity of the GEMV / GEMM operators against the CPU oracle.

Every case draws seeded inputs, runs the HIP operator and compares with the oracle
under the rule in ``tests/_tol.py`` (per-element relative error <= 1e-2, absolute
floor 1e-3 of the output scale). Shapes cover tile tails in M, N and K, the
padded-K path, every scale dtype, and decode M in {1, 4, 16, 32}.
"""

import re
import sys

import pytest
import torch

from oracle import fp8_oracle as ora
from tests._tol import assert_linear_close

pytestmark = pytest.mark.gpu
FP8 = torch.float8_e4m3fn


def _say(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def _plan() -> str:
    """Kernels and split of the last GEMM launch (the library's own record)."""
    from ayaka.kernel.hip import _lib

    return _lib.last_plan()


def _fp8(shape, seed, scale=1.0):
    return (torch.randn(*shape, generator=_gen(seed)) * scale).clamp(-448, 448).to(FP8)


# ------------------------------------------------------------------ weight-only GEMV
@pytest.mark.parametrize("xdt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(
    "n,k,by,bx,sdt",
    [
        (3072, 1024, 1, 1024, "float32"),  # per-channel (rowwise / per-tensor decode)
        (3072, 1024, 3072, 1024, "float32"),  # one scalar scale broadcast
        (300, 4096, 1, 4096, "float32"),
        (4096, 14336, 1, 14336, "float32"),  # Cfg2 down (split-K)
        (4098, 1024, 1, 1024, "float32"),  # streaming: 2049 one-pair wavefronts, 3 idle
        (6147, 2048, 1, 2048, "float32"),  # streaming, ragged last pair
        (8190, 1024, 1, 1024, "float32"),  # streaming: 4095 one-pair wavefronts
        (8194, 1024, 1, 1024, "float32"),  # streaming: 4097 pairs, three per wavefront
        (520, 7168, 128, 128, "float32"),  # block-128 decode
        (700, 1792, 128, 128, "bfloat16"),
        (256, 2048, 1, 32, "e8m0"),  # per-32 UE8M0
        (100, 100, 1, 100, "float32"),  # K % 16 != 0: generic path
        (64, 96, 16, 24, "bfloat16"),  # scale block not a multiple of 16: generic path
    ],
)
def test_weight_only_gemv(gpu, xdt, n, k, by, bx, sdt):
    from ayaka.kernel.hip import fp8_weight_only_gemv

    _say(f"fp8_weight_only_gemv x={xdt} n={n} k={k} by={by} bx={bx} scale={sdt}")
    w = _fp8((n, k), seed=n + k)
    srs = -(-k // bx)
    rows = -(-n // by)
    if sdt == "e8m0":
        scale = torch.randint(110, 130, (rows, srs), generator=_gen(1), dtype=torch.uint8)
    else:
        scale = (torch.rand(rows, srs, generator=_gen(2)) * 0.02 + 1e-3).to(torch.float32 if sdt == "float32" else torch.bfloat16)
    x = torch.randn(k, generator=_gen(3)).to(xdt)
    y = fp8_weight_only_gemv(x.to(gpu), w.to(gpu), scale.to(gpu), srs, by, bx, sdt)
    ref = ora.fp8_weight_only_gemv(x, w, scale, srs, by, bx, sdt)
    assert y.dtype == xdt
    assert_linear_close(y, ref, "weight_only_gemv")
    out = torch.empty(n, dtype=xdt, device=gpu)
    r = fp8_weight_only_gemv(x.to(gpu), w.to(gpu), scale.to(gpu), srs, by, bx, sdt, out=out)
    assert r is out
    assert torch.equal(out.cpu(), y.cpu()), "repeat launches must be bit-identical"


@pytest.mark.parametrize("n,k", [(512, 1024), (333, 2048), (2048, 7168)])
def test_blockwise_gemv(gpu, n, k):
    from ayaka.kernel.hip import fp8_blockwise_gemv

    _say(f"fp8_blockwise_gemv n={n} k={k}")
    a = _fp8((k,), seed=5, scale=20)
    b = _fp8((n, k), seed=6, scale=20)
    sa = torch.rand(-(-k // 128), generator=_gen(7)) * 0.1
    sb = torch.rand(-(-n // 128), -(-k // 128), generator=_gen(8)) * 0.01
    bias = torch.randn(n, generator=_gen(9))
    y = fp8_blockwise_gemv(a.to(gpu), b.to(gpu), sa.to(gpu), sb.to(gpu), bias.to(gpu))
    assert y.dtype == torch.float32
    assert_linear_close(y, ora.fp8_blockwise_gemv(a, b, sa, sb, bias), "blockwise_gemv")


# ------------------------------------------------------------------ W8A8 GEMMs
MNK = [(8, 3072, 1024), (17, 300, 256), (64, 256, 384), (200, 1000, 1024), (256, 512, 2048), (129, 130, 528),
       (300, 520, 1024), (513, 772, 2048), (1024, 1024, 3584),
       # 256x256 kernel with 1, 5 and 19 K stages of 64: steps padded to a multiple of four
       (256, 256, 64), (400, 300, 320), (260, 1028, 1216),
       # its 128-byte-row variant (K % 128 == 0) with 1 and 3 pairs of stages: pairs padded to even
       (256, 260, 128), (512, 512, 384),  # from (300, 520, 1024) on: the 256x256 kernels
       # K splits whose N is not a multiple of 4: the one-element-per-thread reduce
       (300, 1002, 8192), (40, 1002, 8192)]


@pytest.mark.parametrize("m,n,k", MNK)
@pytest.mark.parametrize("rowwise", [True, False])
def test_fp8_scaled_mm(gpu, m, n, k, rowwise):
    from ayaka.kernel.hip import fp8_scaled_mm

    _say(f"fp8_scaled_mm m={m} n={n} k={k} rowwise={rowwise}")
    a = _fp8((m, k), seed=m, scale=40)
    w = _fp8((n, k), seed=n, scale=40)
    sa = (torch.rand(m, generator=_gen(1)) * 0.01 + 1e-3) if rowwise else torch.tensor(0.004)
    sb = (torch.rand(n, generator=_gen(2)) * 0.01 + 1e-3) if rowwise else torch.tensor(0.002)
    bias = torch.randn(n, generator=_gen(3)).to(torch.bfloat16)
    ref = ora.fp8_scaled_mm(a, w, sa, sb, bias)
    y = fp8_scaled_mm(a.to(gpu), w.to(gpu).t(), sa.to(gpu), sb.to(gpu), bias.to(gpu))
    assert y.dtype == torch.float32
    assert_linear_close(y, ref, "fp8_scaled_mm fp32")
    out = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    r = fp8_scaled_mm(a.to(gpu), w.to(gpu).t(), sa.to(gpu), sb.to(gpu), bias.to(gpu), out=out)
    assert r is out
    assert_linear_close(out, ref, "fp8_scaled_mm bf16")


@pytest.mark.parametrize("m,n,k,rowwise,out_dtype", [
    (512, 3584, 18944, True, torch.bfloat16),   # 256x256 pair kernel, 28 tiles: 15 K splits
    (300, 520, 4096, False, torch.float16),     # pair kernel, ragged M / N, per-tensor scales
    (128, 1024, 4096, True, torch.float32),     # general kernel (128-row tiles)
    (40, 768, 8192, True, torch.bfloat16),      # general kernel (64-row tiles)
    (8, 3584, 18944, False, torch.bfloat16),    # general kernel (32-row tiles), last split shorter
])
def test_fp8_scaled_mm_split_k(gpu, m, n, k, rowwise, out_dtype):
    """Launches short of one round of tiles split K: scaled fp32 partials in the workspace
    the wrapper allocates from the size query, summed in a fixed order with the bias."""
    from ayaka.kernel.hip import _lib, fp8_scaled_mm

    _say(f"fp8_scaled_mm split-K m={m} n={n} k={k} rowwise={rowwise} out={out_dtype}")
    assert _lib.query("ayk_fp8_scaled_mm_workspace_bytes", m, n, k) > 0, "shape should split"
    a = _fp8((m, k), seed=m + 21, scale=40)
    w = _fp8((n, k), seed=n + 22, scale=40)
    sa = (torch.rand(m, generator=_gen(23)) * 0.01 + 1e-3) if rowwise else torch.tensor(0.004)
    sb = (torch.rand(n, generator=_gen(24)) * 0.01 + 1e-3) if rowwise else torch.tensor(0.002)
    bias = (torch.randn(n, generator=_gen(25)) * 30).to(torch.bfloat16)
    ref = ora.fp8_scaled_mm(a, w, sa, sb, bias)
    out = torch.empty(m, n, dtype=out_dtype, device=gpu)
    fp8_scaled_mm(a.to(gpu), w.to(gpu).t(), sa.to(gpu), sb.to(gpu), bias.to(gpu), out=out)
    assert_linear_close(out, ref, "fp8_scaled_mm split-K")


@pytest.mark.parametrize("m,n,k", [
    (512, 2048, 4096),   # 256x256 pair kernel: 16 tiles, 4 splits of 1024 K (whole code chunks)
    (300, 520, 8704),    # pair kernel, ragged M / N, 17 chunks of 512 K: the last split shorter
    (64, 1024, 8192),    # general kernel, 64-row tiles
    (5, 768, 4096),      # general kernel, 32-row tiles
])
def test_mxfp8_scaled_mm_split_k(gpu, m, n, k):
    """MXFP8 launches short of one round of tiles split K; each split reads its UE8M0
    codes from k0 / 32 on in every code row."""
    from ayaka.kernel.hip import _lib, mxfp8_scaled_mm

    _say(f"mxfp8_scaled_mm split-K m={m} n={n} k={k}")
    assert _lib.query("ayk_mxfp8_scaled_mm_workspace_bytes", m, n, k) > 0, "shape should split"
    torch.manual_seed(m + n + k)
    x = torch.distributions.StudentT(3.0).sample((m, k))
    wf = torch.randn(n, k, generator=_gen(31))
    qa, ca = ora.per_token_group_quant_mxfp8(x, 32)
    qw, cw = ora.per_token_group_quant_mxfp8(wf, 32)
    bias = (torch.randn(n, generator=_gen(32)) * 10).to(torch.bfloat16)
    ref = ora.mxfp8_scaled_mm(qa, ca, qw, cw, bias)
    y = mxfp8_scaled_mm(qa.to(gpu), ca.to(gpu), qw.to(gpu), cw.to(gpu), bias.to(gpu),
                        out=torch.empty(m, n, dtype=torch.bfloat16, device=gpu))
    assert_linear_close(y, ref, "mxfp8_scaled_mm split-K")


# Decode batches (M <= 64, K % 256 == 0): the weight-streaming kernel. Each shape picks
# a different plan: rows per wavefront (32 or 64), activation tiles (M <= 32 or <= 64),
# K parts per row group (1, 2, 4), activation chunk of 2 or 4 pairs, grid K split.
SKINNY_MNK = [
    (9, 3000, 2048),     # 32 rows, 4 K parts, ragged N (2-8 rows take the GEMV-shaped kernel)
    (8, 24576, 2048),    # 32 rows, whole K, two workgroups per CU
    (16, 57344, 1024),   # 64 rows per wavefront, chunks of 4 pairs
    (8, 14336, 2048),    # 64 rows per wavefront, 4 K parts
    (17, 5000, 1280),    # K % 512 != 0: whole K per wavefront, under 128 workgroups
    (40, 20000, 2048),   # two activation tiles, 32 rows, whole K
    (33, 1000, 4096),    # two activation tiles, 2 K parts, grid split 2
    (48, 57344, 1024),   # 64 rows per wavefront, two activation tiles
    (64, 1302, 8192),    # N % 4 != 0 rows: element stores, grid split
    (1, 4096, 4096),     # a single row
]


@pytest.mark.parametrize("m,n,k", SKINNY_MNK)
@pytest.mark.parametrize("rowwise,out_dtype", [(True, torch.bfloat16), (False, torch.float16), (True, torch.float32)])
def test_fp8_scaled_mm_decode_batch(gpu, m, n, k, rowwise, out_dtype):
    from ayaka.kernel.hip import fp8_scaled_mm

    _say(f"fp8_scaled_mm decode batch m={m} n={n} k={k} rowwise={rowwise} out={out_dtype}")
    a = _fp8((m, k), seed=m + 61, scale=40)
    w = _fp8((n, k), seed=n + 62, scale=40)
    sa = (torch.rand(m, generator=_gen(63)) * 0.01 + 1e-3) if rowwise else torch.tensor(0.004)
    sb = (torch.rand(n, generator=_gen(64)) * 0.01 + 1e-3) if rowwise else torch.tensor(0.002)
    bias = (torch.randn(n, generator=_gen(65)) * 10).to(torch.bfloat16)
    ref = ora.fp8_scaled_mm(a, w, sa, sb, bias)
    buf = torch.full((m, n + 6), 7.0, dtype=out_dtype, device=gpu)  # row stride n + 6
    out = buf[:, :n]
    fp8_scaled_mm(a.to(gpu), w.to(gpu).t(), sa.to(gpu), sb.to(gpu), bias.to(gpu), out=out)
    assert _plan().startswith("skinny"), f"decode batch ran {_plan()!r}"
    assert_linear_close(out, ref, "fp8_scaled_mm decode batch")
    assert torch.all(buf[:, n:].float() == 7.0), "wrote past the output columns"


@pytest.mark.parametrize("m,n,k", [(2, 520, 2048), (40, 1000, 3072), (9, 20000, 1024), (64, 4100, 8192),
                                   (64, 2048, 28672), (30, 57344, 512),
                                   (8, 3000, 1280)])  # K not in whole 512-K chunks: one code load per stage
def test_mxfp8_scaled_mm_decode_batch(gpu, m, n, k):
    """MXFP8 decode batches: the UE8M0 code dwords staged with the operands, four 128-K
    pairs per 16-byte load where the code rows allow it; K parts and grid splits start
    their codes at their own K offset."""
    from ayaka.kernel.hip import mxfp8_scaled_mm

    _say(f"mxfp8_scaled_mm decode batch m={m} n={n} k={k}")
    torch.manual_seed(m + n + k + 3)
    x = torch.distributions.StudentT(3.0).sample((m, k))
    wf = torch.randn(n, k, generator=_gen(66))
    qa, ca = ora.per_token_group_quant_mxfp8(x, 32)
    qw, cw = ora.per_token_group_quant_mxfp8(wf, 32)
    bias = (torch.randn(n, generator=_gen(67)) * 10).to(torch.bfloat16)
    ref = ora.mxfp8_scaled_mm(qa, ca, qw, cw, bias)
    y = mxfp8_scaled_mm(qa.to(gpu), ca.to(gpu), qw.to(gpu), cw.to(gpu), bias.to(gpu),
                        out=torch.empty(m, n, dtype=torch.bfloat16, device=gpu))
    assert _plan().startswith("skinny"), f"decode batch ran {_plan()!r}"
    assert_linear_close(y, ref, "mxfp8_scaled_mm decode batch")


def _offset_view(t: torch.Tensor, offset_elems: int) -> torch.Tensor:
    """A contiguous copy of `t` that starts `offset_elems` elements into its buffer (a
    pointer aligned to the element size but not to 16 bytes)."""
    buf = torch.empty(t.numel() + offset_elems, dtype=t.dtype, device=t.device)
    view = buf[offset_elems:].view(t.shape)
    view.copy_(t)
    assert view.is_contiguous() and view.data_ptr() % 16 != 0
    return view


def test_decode_batch_scales_not_16_byte_aligned(gpu):
    """Scale rows that are not 16-byte aligned take the one-load-per-stage path of the
    decode-batch kernel (the four-stage 16-byte loads need aligned rows): MXFP8 codes
    4 bytes into their buffer, block-128 activation scales one float in."""
    from ayaka.kernel.hip import fp8_blockwise_mm, mxfp8_scaled_mm

    _say("decode batch, scale rows off 16-byte alignment")
    m, n, k = 9, 20000, 1024
    torch.manual_seed(81)
    x = torch.distributions.StudentT(3.0).sample((m, k))
    wf = torch.randn(n, k, generator=_gen(82))
    qa, ca = ora.per_token_group_quant_mxfp8(x, 32)
    qw, cw = ora.per_token_group_quant_mxfp8(wf, 32)
    ref = ora.mxfp8_scaled_mm(qa, ca, qw, cw)
    y = mxfp8_scaled_mm(qa.to(gpu), _offset_view(ca.to(gpu), 4), qw.to(gpu), _offset_view(cw.to(gpu), 4),
                        out=torch.empty(m, n, dtype=torch.bfloat16, device=gpu))
    assert _plan().startswith("skinny") and "ch=1" in _plan(), _plan()
    assert_linear_close(y, ref, "mxfp8 decode batch, offset codes")

    m, n, k = 32, 4096, 2048
    kb, nb = k // 128, n // 128
    a = _fp8((m, k), seed=83, scale=30)
    w = _fp8((n, k), seed=84, scale=30)
    sa = torch.exp(torch.rand(m, kb, generator=_gen(85)) * -6.9).float()
    sb = torch.exp(torch.rand(nb, kb, generator=_gen(86)) * -6.9).float()
    ref = ora.fp8_blockwise_mm(a, w, sa, sb, None, False)
    out = fp8_blockwise_mm(a.to(gpu), w.to(gpu), _offset_view(sa.to(gpu), 1), _offset_view(sb.to(gpu), 1))
    assert _plan().startswith("skinny") and "ch=1" in _plan(), _plan()
    assert_linear_close(out, ref, "blockwise decode batch, offset scales")


@pytest.mark.parametrize("m,n,k,rowwise,with_bias", [(2048, 4096, 1024, True, True), (1300, 11712, 1536, False, False),
                                                    (4096, 37888, 512, True, False)])
def test_fp8_scaled_mm_half_outputs_are_the_fp32_result_rounded(gpu, m, n, k, rowwise, with_bias):
    """The 16-bit outputs of the 256 x 256 kernel are its fp32 result rounded once to
    nearest even (torch's cast), bit for bit: no step of the epilogue may fold a multiply
    into the conversion (one rounding of the exact product differs at fp16 ties)."""
    from ayaka.kernel.hip import fp8_scaled_mm

    _say(f"fp8_scaled_mm 16-bit outputs vs rounded fp32 m={m} n={n} k={k} rowwise={rowwise} bias={with_bias}")
    g = torch.Generator(device=gpu).manual_seed(m + n)
    a = (torch.randn(m, k, device=gpu, generator=g) * 40).clamp(-448, 448).to(FP8)
    w = (torch.randn(n, k, device=gpu, generator=g) * 40).clamp(-448, 448).to(FP8)
    sa = torch.rand(m, device=gpu, generator=g) * 0.01 + 1e-3
    sb = torch.rand(n, device=gpu, generator=g) * 0.01 + 1e-3
    if not rowwise:
        sa, sb = sa[:1].reshape(()), sb[:1].reshape(())
    bias = torch.randn(n, device=gpu, generator=g).float() if with_bias else None
    y32 = fp8_scaled_mm(a, w.t(), sa, sb, bias, out=torch.empty(m, n, dtype=torch.float32, device=gpu))
    for dt in (torch.float16, torch.bfloat16):
        y = fp8_scaled_mm(a, w.t(), sa, sb, bias, out=torch.empty(m, n, dtype=dt, device=gpu))
        assert torch.equal(y.view(torch.int16), y32.to(dt).view(torch.int16)), f"{dt} output is not the rounded fp32 result"


# 276 tiles of 256 x 256: one whole round, then a last round of 20 tiles that the pair
# kernel splits over K (three 512-K pieces each) into the workspace, ragged M and N.
TAIL_MNK = (1300, 11712, 1536)


@pytest.mark.parametrize("rowwise,out_dtype", [(True, torch.bfloat16), (False, torch.float16), (True, torch.float32)])
def test_fp8_scaled_mm_tail_split(gpu, rowwise, out_dtype):
    from ayaka.kernel.hip import _lib, fp8_scaled_mm

    m, n, k = TAIL_MNK
    _say(f"fp8_scaled_mm tail split m={m} n={n} k={k} rowwise={rowwise} out={out_dtype}")
    assert _lib.query("ayk_fp8_scaled_mm_workspace_bytes", m, n, k) == 3 * 20 * 256 * 256 * 4, "tail split expected"
    a = _fp8((m, k), seed=41, scale=40)
    w = _fp8((n, k), seed=42, scale=40)
    sa = (torch.rand(m, generator=_gen(43)) * 0.01 + 1e-3) if rowwise else torch.tensor(0.004)
    sb = (torch.rand(n, generator=_gen(44)) * 0.01 + 1e-3) if rowwise else torch.tensor(0.002)
    bias = (torch.randn(n, generator=_gen(45)) * 30).to(torch.bfloat16)
    ref = ora.fp8_scaled_mm(a, w, sa, sb, bias)
    out = torch.empty(m, n, dtype=out_dtype, device=gpu)
    fp8_scaled_mm(a.to(gpu), w.to(gpu).t(), sa.to(gpu), sb.to(gpu), bias.to(gpu), out=out)
    assert_linear_close(out, ref, "fp8_scaled_mm tail split")


def test_mxfp8_scaled_mm_tail_split(gpu):
    from ayaka.kernel.hip import _lib, mxfp8_scaled_mm

    m, n, k = TAIL_MNK
    _say(f"mxfp8_scaled_mm tail split m={m} n={n} k={k}")
    assert _lib.query("ayk_mxfp8_scaled_mm_workspace_bytes", m, n, k) == 3 * 20 * 256 * 256 * 4, "tail split expected"
    torch.manual_seed(46)
    x = torch.distributions.StudentT(3.0).sample((m, k))
    wf = torch.randn(n, k, generator=_gen(47))
    qa, ca = ora.per_token_group_quant_mxfp8(x, 32)
    qw, cw = ora.per_token_group_quant_mxfp8(wf, 32)
    bias = (torch.randn(n, generator=_gen(48)) * 10).to(torch.bfloat16)
    ref = ora.mxfp8_scaled_mm(qa, ca, qw, cw, bias)
    y = mxfp8_scaled_mm(qa.to(gpu), ca.to(gpu), qw.to(gpu), cw.to(gpu), bias.to(gpu),
                        out=torch.empty(m, n, dtype=torch.bfloat16, device=gpu))
    assert_linear_close(y, ref, "mxfp8_scaled_mm tail split")


@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_fp8_scaled_mm_big_tile_strided_out(gpu, out_dtype):
    """256x256-tile kernel: every output dtype, a padded output row stride, M/N tails."""
    from ayaka.kernel.hip import fp8_scaled_mm

    m, n, k = 520, 1284, 1280
    _say(f"fp8_scaled_mm big tile out={out_dtype}")
    a = _fp8((m, k), seed=21, scale=40)
    w = _fp8((n, k), seed=22, scale=40)
    sa = torch.rand(m, generator=_gen(1)) * 0.01 + 1e-3
    sb = torch.rand(n, generator=_gen(2)) * 0.01 + 1e-3
    bias = torch.randn(n, generator=_gen(3))
    ref = ora.fp8_scaled_mm(a, w, sa, sb, bias)
    buf = torch.full((m, n + 12), 7.0, dtype=out_dtype, device=gpu)  # row stride n + 12
    out = buf[:, :n]
    fp8_scaled_mm(a.to(gpu), w.to(gpu).t(), sa.to(gpu), sb.to(gpu), bias.to(gpu), out=out)
    assert_linear_close(out, ref, f"big tile {out_dtype}")
    assert torch.all(buf[:, n:].float() == 7.0), "wrote past the output columns"


@pytest.mark.parametrize("k", [192, 320, 1088, 640])
@pytest.mark.parametrize("rowwise,with_bias", [(True, False), (False, True), (True, True)])
def test_fp8_scaled_mm_many_tiles(gpu, k, rowwise, with_bias):
    """More 256x256 tiles (9 x 32 = 288) than compute units, so compute units run several
    tiles; K of 3, 5 and 17 stages (padded steps) and of 5 pairs of stages."""
    from ayaka.kernel.hip import fp8_scaled_mm

    m, n = 2304, 8192
    _say(f"fp8_scaled_mm many tiles m={m} n={n} k={k} rowwise={rowwise} bias={with_bias}")
    a = _fp8((m, k), seed=31, scale=40)
    w = _fp8((n, k), seed=32, scale=40)
    sa = (torch.rand(m, generator=_gen(1)) * 0.01 + 1e-3) if rowwise else torch.tensor(0.004)
    sb = (torch.rand(n, generator=_gen(2)) * 0.01 + 1e-3) if rowwise else torch.tensor(0.002)
    bias = torch.randn(n, generator=_gen(3)).to(torch.bfloat16) if with_bias else None
    ref = ora.fp8_scaled_mm(a, w, sa, sb, bias)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    fp8_scaled_mm(a.to(gpu), w.to(gpu).t(), sa.to(gpu), sb.to(gpu), None if bias is None else bias.to(gpu), out=out)
    assert_linear_close(out, ref, "many tiles bf16")
    # A second call into the same buffer (every tile is rewritten).
    out.fill_(float("nan"))
    fp8_scaled_mm(a.to(gpu), w.to(gpu).t(), sa.to(gpu), sb.to(gpu), None if bias is None else bias.to(gpu), out=out)
    assert_linear_close(out, ref, "many tiles bf16 (second call)")


def test_fp8_scaled_mm_row_major_b_and_odd_k(gpu):
    from ayaka.kernel.hip import fp8_scaled_mm

    _say("fp8_scaled_mm [K,N] b and K=40")
    a = _fp8((33, 40), seed=1, scale=10)
    w = _fp8((70, 40), seed=2, scale=10)
    b_kn = w.t().contiguous()  # row-major [K, N]
    y = fp8_scaled_mm(a.to(gpu), b_kn.to(gpu), torch.tensor(0.5, device=gpu), torch.tensor(0.25, device=gpu))
    assert_linear_close(y, ora.fp8_scaled_mm(a, w, torch.tensor(0.5), torch.tensor(0.25)), "scaled_mm odd K")


@pytest.mark.parametrize("m,n,k", [(2, 256, 256), (32, 640, 1024), (256, 384, 2048), (300, 200, 1280), (129, 1024, 7168)])
@pytest.mark.parametrize("sdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("col_major", [False, True])
def test_fp8_blockwise_mm(gpu, m, n, k, sdt, col_major):
    from ayaka.kernel.hip import fp8_blockwise_mm

    _say(f"fp8_blockwise_mm m={m} n={n} k={k} sdt={sdt} col_major={col_major}")
    kb, nb = -(-k // 128), -(-n // 128)
    a = _fp8((m, k), seed=m + 1, scale=30)
    w = _fp8((n, k), seed=n + 2, scale=30)
    # block scales spread log-uniformly over 1e-3 .. 1 exercise the per-128 rescale
    sa = torch.exp(torch.rand(m, kb, generator=_gen(4)) * -6.9).float()
    sb = torch.exp(torch.rand(nb, kb, generator=_gen(5)) * -6.9).to(sdt)
    sa_arg = sa.t().contiguous() if col_major else sa
    ref = ora.fp8_blockwise_mm(a, w, sa_arg, sb, None, col_major)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    fp8_blockwise_mm(a.to(gpu), w.to(gpu), sa_arg.to(gpu), sb.to(gpu), out=out, a_scale_col_major=col_major)
    assert_linear_close(out, ref, "blockwise_mm")


# The 256 x 256 block-scaled kernel (launches of >= 128 tiles of 256 x 256): ragged M / N
# tails, an odd number of 128-K blocks (a padded loop pair), column-major activation
# scales, 16-bit weight scales, every output dtype and the K-split form (exactly 128 tiles).
BLOCK256 = [
    (2100, 4200, 640, False, torch.float32, torch.bfloat16, True),
    (4096, 2304, 1152, True, torch.bfloat16, torch.float32, False),
    (2304, 4352, 384, False, torch.float16, torch.float16, True),
    (2048, 4096, 8192, False, torch.float32, torch.bfloat16, True),   # 128 tiles: K split 2
    (512, 2304, 7040, True, torch.float32, torch.bfloat16, True),     # 18 tiles: 6 K pieces, the last 5 blocks of 10
    (4096, 2048, 256, True, torch.float32, torch.bfloat16, False),    # two blocks, one pair
]


@pytest.mark.parametrize("m,n,k,col_major,sdt,out_dtype,with_bias", BLOCK256)
def test_fp8_blockwise_mm_256(gpu, m, n, k, col_major, sdt, out_dtype, with_bias):
    from ayaka.kernel.hip import fp8_blockwise_mm

    _say(f"fp8_blockwise_mm 256-tile m={m} n={n} k={k} col_major={col_major} sdt={sdt} out={out_dtype} bias={with_bias}")
    kb, nb = k // 128, -(-n // 128)
    a = _fp8((m, k), seed=m + 3, scale=30)
    w = _fp8((n, k), seed=n + 4, scale=30)
    # scales over eight decades, so the per-block exponent / mantissa split sees widely
    # different exponents from block to block
    sa = torch.exp(torch.rand(m, kb, generator=_gen(24)) * -18.0).float()
    sb = torch.exp(torch.rand(nb, kb, generator=_gen(25)) * -6.9).to(sdt)
    sa_arg = sa.t().contiguous() if col_major else sa
    bias = (torch.randn(n, generator=_gen(26)) * 0.01).to(torch.bfloat16) if with_bias else None
    ref = ora.fp8_blockwise_mm(a, w, sa_arg, sb, bias, col_major)
    out = torch.empty(m, n, dtype=out_dtype, device=gpu)
    fp8_blockwise_mm(a.to(gpu), w.to(gpu), sa_arg.to(gpu), sb.to(gpu), bias.to(gpu) if bias is not None else None,
                     out=out, a_scale_col_major=col_major)
    assert_linear_close(out, ref, "blockwise_mm 256-tile")


def test_fp8_blockwise_mm_256_scale_edges(gpu):
    """Zero weight-block scales add nothing (the MFMA exponent code 0 weighs a block's
    products by 2^-127), and a NaN scale poisons exactly the outputs whose sums include it,
    as in the oracle."""
    from ayaka.kernel.hip import fp8_blockwise_mm

    m, n, k = 2048, 4096, 1024
    _say(f"fp8_blockwise_mm 256-tile scale edges m={m} n={n} k={k}")
    kb, nb = k // 128, n // 128
    a = _fp8((m, k), seed=31, scale=30)
    w = _fp8((n, k), seed=32, scale=30)
    sa = torch.exp(torch.rand(m, kb, generator=_gen(33)) * -6.9).float()
    sb = torch.exp(torch.rand(nb, kb, generator=_gen(34)) * -6.9).float()
    sb[3, :] = 0.0      # weight rows 384..511 contribute nothing
    sb[5, 2] = 0.0      # one block of rows 640..767
    sa[7, 4] = float("nan")  # activation row 7: every output NaN
    ref = ora.fp8_blockwise_mm(a, w, sa, sb)
    out = torch.empty(m, n, dtype=torch.float32, device=gpu)
    fp8_blockwise_mm(a.to(gpu), w.to(gpu), sa.to(gpu), sb.to(gpu), out=out)
    y = out.cpu()
    assert torch.equal(torch.isnan(y), torch.isnan(ref))
    keep = ~torch.isnan(ref)
    assert_linear_close(y[keep], ref[keep], "blockwise_mm 256-tile edges")
    assert y[:, 384:512][keep[:, 384:512]].abs().max().item() < 1e-25


@pytest.mark.parametrize("m,n,k,col_major,sdt,with_bias", [
    (32, 1024, 4096, False, torch.float16, True),     # K split 4
    (200, 768, 8192, True, torch.bfloat16, True),     # split 8, column-major activation scales
    (7, 256, 2048, False, torch.float16, False),      # split 2, 7 rows
    (256, 2048, 7168, False, torch.float32, False),   # DeepSeek-V3 K, split 4
    (32, 7168, 18432, False, torch.bfloat16, True),   # DeepSeek-V3 (7168, 18432) at M = 32, split 16
    (16, 64, 4096, False, torch.float16, False),      # N < 128: general kernel split 4
    (40, 96, 8192, True, torch.bfloat16, True),       # N < 128, 64-row tiles: split 8
])
def test_fp8_blockwise_mm_split_k(gpu, m, n, k, col_major, sdt, with_bias):
    """Launches with too few 128 x 128 tiles split K over fp32 partials (the workspace the
    wrapper allocates from the size query) and reduce them in a fixed order. (Up to 64
    rows with fp32 weight scales take the decode-batch kernel instead: 16-bit weight scales
    here keep these on the general kernel.)"""
    from ayaka.kernel.hip import _lib, fp8_blockwise_mm

    _say(f"fp8_blockwise_mm split-K m={m} n={n} k={k} col_major={col_major} sdt={sdt} bias={with_bias}")
    assert _lib.query("ayk_fp8_blockwise_mm_workspace_bytes", m, n, k) > 0, "shape should split"
    kb, nb = k // 128, -(-n // 128)
    a = _fp8((m, k), seed=m + 11, scale=30)
    w = _fp8((n, k), seed=n + 12, scale=30)
    sa = torch.exp(torch.rand(m, kb, generator=_gen(14)) * -6.9).float()
    sb = torch.exp(torch.rand(nb, kb, generator=_gen(15)) * -6.9).to(sdt)
    sa_arg = sa.t().contiguous() if col_major else sa
    bias = (torch.randn(n, generator=_gen(16)) * 50).to(torch.bfloat16) if with_bias else None
    ref = ora.fp8_blockwise_mm(a, w, sa_arg, sb, bias, col_major)
    out = fp8_blockwise_mm(a.to(gpu), w.to(gpu), sa_arg.to(gpu), sb.to(gpu),
                           bias.to(gpu) if bias is not None else None, a_scale_col_major=col_major)
    assert not re.search(r"split=1\b", _plan()) and not _plan().startswith("skinny"), _plan()
    assert_linear_close(out, ref, "blockwise_mm split-K")


@pytest.mark.parametrize("m,n,k,col_major,with_bias", [
    (32, 18432, 7168, False, True),    # DeepSeek-V3 up at M = 32
    (32, 7168, 18432, True, False),    # DeepSeek-V3 down at M = 32, column-major activation scales
    (5, 1000, 2048, False, True),      # N not a multiple of 128: the last block's rows clamp
    (64, 300, 8192, True, True),       # two activation tiles, grid K split
    (16, 64, 4096, False, False),      # N < 128
    (40, 4096, 1280, False, True),     # K % 512 != 0
])
def test_fp8_blockwise_mm_decode_batch(gpu, m, n, k, col_major, with_bias):
    """Block-128 decode batches with fp32 scales: the weight-streaming kernel folds every
    128-K stage's partial with sa[m, kb] sb[n / 128, kb] (block amax spread 1e-3 .. 1)."""
    from ayaka.kernel.hip import fp8_blockwise_mm

    _say(f"fp8_blockwise_mm decode batch m={m} n={n} k={k} col_major={col_major} bias={with_bias}")
    kb, nb = k // 128, -(-n // 128)
    a = _fp8((m, k), seed=m + 71, scale=30)
    w = _fp8((n, k), seed=n + 72, scale=30)
    sa = torch.exp(torch.rand(m, kb, generator=_gen(74)) * -6.9).float()
    sb = torch.exp(torch.rand(nb, kb, generator=_gen(75)) * -6.9).float()
    sa_arg = sa.t().contiguous() if col_major else sa
    bias = (torch.randn(n, generator=_gen(76)) * 5).to(torch.bfloat16) if with_bias else None
    ref = ora.fp8_blockwise_mm(a, w, sa_arg, sb, bias, col_major)
    out = fp8_blockwise_mm(a.to(gpu), w.to(gpu), sa_arg.to(gpu), sb.to(gpu),
                           bias.to(gpu) if bias is not None else None, a_scale_col_major=col_major)
    assert _plan().startswith("skinny"), f"decode batch ran {_plan()!r}"
    assert_linear_close(out, ref, "blockwise_mm decode batch")


# Decode-batch plans that a case must reach, named by the library's launch record:
# (mode, M, N, K, expected plan). Rows per wavefront 32 FN, activation tiles FM, K parts
# KS, G pairs per activation chunk, CH stages per scale load, grid split. The FN = 2 /
# KS = 4 plan needs more than 160 KB of LDS with a scale ring, so only fp32 per-row /
# per-tensor scales (mode "scaled") reach it.
DECODE_PLANS = [
    ("block", 64, 18432, 7168, "skinny fn=1 fm=2 ks=1 g=2 ch=4 split=1"),  # DeepSeek-V3 up at M = 64
    ("block", 64, 7168, 18432, "skinny fn=1 fm=2 ks=1 g=2 ch=4 split=4"),  # DeepSeek-V3 down at M = 64
    ("block", 48, 4096, 2048, "skinny fn=1 fm=2 ks=2 g=2 ch=4 split=1"),
    ("block", 16, 14000, 1024, "skinny fn=1 fm=1 ks=2 g=2 ch=4 split=1"),
    ("mx", 64, 14000, 1024, "skinny fn=1 fm=2 ks=2 g=2 ch=4 split=1"),
    ("mx", 20, 13000, 1024, "skinny fn=1 fm=1 ks=2 g=2 ch=4 split=1"),
    ("scaled", 9, 14000, 1024, "skinny fn=2 fm=1 ks=4 g=2 ch=1 split=1"),  # 2-8 rows: the GEMV-shaped kernel
    ("scaled", 24, 12800, 1024, "skinny fn=2 fm=1 ks=4 g=2 ch=1 split=1"),
]


@pytest.mark.parametrize("mode,m,n,k,plan", DECODE_PLANS, ids=[f"{c[0]}-{c[1]}x{c[2]}x{c[3]}" for c in DECODE_PLANS])
def test_decode_batch_plans(gpu, mode, m, n, k, plan):
    """Each case reaches its decode-batch plan (asserted on the launch record) and
    matches the oracle: two activation tiles on the four-stage 16-byte scale path, and
    the four-K-part 64-row plan."""
    from ayaka.kernel.hip import fp8_blockwise_mm, fp8_scaled_mm, mxfp8_scaled_mm

    _say(f"decode-batch plan {mode} m={m} n={n} k={k}: {plan}")
    if mode == "block":
        kb, nb = k // 128, -(-n // 128)
        a = _fp8((m, k), seed=m + 91, scale=30)
        w = _fp8((n, k), seed=n + 92, scale=30)
        sa = torch.exp(torch.rand(m, kb, generator=_gen(93)) * -6.9).float()
        sb = torch.exp(torch.rand(nb, kb, generator=_gen(94)) * -6.9).float()
        bias = (torch.randn(n, generator=_gen(95)) * 5).to(torch.bfloat16)
        ref = ora.fp8_blockwise_mm(a, w, sa, sb, bias, False)
        out = fp8_blockwise_mm(a.to(gpu), w.to(gpu), sa.to(gpu), sb.to(gpu), bias.to(gpu))
    elif mode == "mx":
        torch.manual_seed(m + n)
        qa, ca = ora.per_token_group_quant_mxfp8(torch.distributions.StudentT(3.0).sample((m, k)), 32)
        qw, cw = ora.per_token_group_quant_mxfp8(torch.randn(n, k, generator=_gen(96)), 32)
        ref = ora.mxfp8_scaled_mm(qa, ca, qw, cw)
        out = mxfp8_scaled_mm(qa.to(gpu), ca.to(gpu), qw.to(gpu), cw.to(gpu),
                              out=torch.empty(m, n, dtype=torch.bfloat16, device=gpu))
    else:
        a = _fp8((m, k), seed=m + 97, scale=40)
        w = _fp8((n, k), seed=n + 98, scale=40)
        sa = torch.rand(m, generator=_gen(99)) * 0.01 + 1e-3
        sb = torch.rand(n, generator=_gen(100)) * 0.01 + 1e-3
        ref = ora.fp8_scaled_mm(a, w, sa, sb)
        out = fp8_scaled_mm(a.to(gpu), w.to(gpu).t(), sa.to(gpu), sb.to(gpu),
                            out=torch.empty(m, n, dtype=torch.bfloat16, device=gpu))
    assert _plan() == plan, f"expected {plan!r}, ran {_plan()!r}"
    assert_linear_close(out, ref, f"decode-batch plan {mode} {m}x{n}x{k}")


@pytest.mark.parametrize("m", [32, 64])
def test_block128_default_bf16_scales_reach_decode_batch_kernel(gpu, m):
    """A block-128 layer with the default bf16 weight-scale table (the reference's
    ``scale_format`` default) runs the decode-batch kernel at M <= 64: the method widens
    the table to fp32 once after loading. Same products as the bf16 table."""
    from torch import nn

    from ayaka.layers.linear.fp8 import FP8Config

    n, k = 4096, 7168
    _say(f"block-128 layer, default bf16 scales, m={m}")
    wf = torch.randn(n, k, generator=_gen(101)) * 0.02
    s = (wf.reshape(n // 128, 128, k // 128, 128).abs().amax(dim=(1, 3)) / 448).to(torch.bfloat16)
    w = (wf / s.float().repeat_interleave(128, 0).repeat_interleave(128, 1)).to(FP8)
    method = FP8Config.from_config({"weight_block_size": [128, 128]}).get_quant_method(None, "model.layers.0.mlp.up_proj")
    layer = nn.Module()
    method.create_weights(layer, output_partition_sizes=[n], input_size_per_partition=k, device=gpu)
    assert layer.weight_scale_inv.dtype == torch.bfloat16
    layer.weight.data.copy_(w.to(gpu))
    layer.weight_scale_inv.weight_loader(layer, layer.weight_scale_inv, s.to(gpu))
    method.process_weights_after_loading(layer)
    x = torch.randn(m, k, generator=_gen(102)).to(torch.bfloat16)
    y = method.apply(layer, x.to(gpu))
    assert _plan().startswith("skinny"), f"default block-128 layer ran {_plan()!r}"
    assert layer.weight_scale_inv.dtype == torch.bfloat16, "the parameter keeps the checkpoint dtype"
    ref = ora.fp8_linear("w8a8_block128", x, w, s, None)
    assert_linear_close(y, ref, f"default block-128 layer m={m}")
    # Writing the scale again drops the widened copy; the next apply uses the new values.
    layer.weight_scale_inv.weight_loader(layer, layer.weight_scale_inv, (s.float() * 2).to(torch.bfloat16).to(gpu))
    method.process_weights_after_loading(layer)
    y2 = method.apply(layer, x.to(gpu))
    assert_linear_close(y2, ref * 2, f"default block-128 layer m={m}, rescaled")


@pytest.mark.parametrize("m,n,k", [(1, 512, 1024), (1, 1000, 8192), (64, 256, 512), (100, 300, 1024), (512, 512, 2048), (33, 96, 96),
                                   (300, 520, 1024), (777, 1028, 2048),
                                   # 256x256 kernels: codes staged in chunks of four 128-K pairs
                                   # (K % 512 == 0; three chunks, M / N tails, 288 tiles) and the
                                   # 128-K-stage kernel for other K % 128 == 0
                                   (520, 1040, 1536), (2304, 8192, 1024), (512, 512, 640)])
def test_mxfp8_scaled_mm(gpu, m, n, k):
    from ayaka.kernel.hip import mxfp8_scaled_mm

    _say(f"mxfp8_scaled_mm m={m} n={n} k={k}")
    torch.manual_seed(m + n + k)
    x = torch.distributions.StudentT(3.0).sample((m, k))
    wf = torch.randn(n, k, generator=_gen(2))
    qa, ca = ora.per_token_group_quant_mxfp8(x, 32)
    qw, cw = ora.per_token_group_quant_mxfp8(wf, 32)
    bias = torch.randn(n, generator=_gen(3))
    ref = ora.mxfp8_scaled_mm(qa, ca, qw, cw, bias)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=gpu)
    mxfp8_scaled_mm(qa.to(gpu), ca.to(gpu), qw.to(gpu), cw.to(gpu), bias.to(gpu), out=out)
    assert_linear_close(out, ref, "mxfp8_scaled_mm")


# Kernel routes for the code-edge cases: M = 1 GEMV, general kernel, 256 x 256 pair
# kernel unsplit and split over K, and the 128-K-stage kernel (K % 512 != 0).
MX_EDGE = [(1, 512, 2048), (100, 300, 1024), (1024, 1024, 512), (512, 2048, 4096), (512, 512, 640)]


def _mx_edge_operands(m, n, k):
    torch.manual_seed(m + n + k + 7)
    x = torch.distributions.StudentT(3.0).sample((m, k))
    x[:, 32:64] = 0.0  # an all-zero activation group: the quantizer's code 0 with q = 0
    wf = torch.randn(n, k, generator=_gen(51))
    qa, ca = ora.per_token_group_quant_mxfp8(x, 32)
    qw, cw = ora.per_token_group_quant_mxfp8(wf, 32)
    assert (ca[:, 1] == 0).all()
    return qa, ca, qw, cw


@pytest.mark.parametrize("m,n,k", MX_EDGE)
def test_mxfp8_code_zero_weight_scales(gpu, m, n, k):
    """UE8M0 code 0 on nonzero weights. The reference decodes it as +0.0
    (reference/gemm.py:11-14, bits c << 23), so such a group adds nothing; the scaled
    MFMA reads it as 2^-127, so the group adds at most 32 * 448 * 448 * 2^-127 *
    2^(ca - 127) (below 1e-30 for every activation code <= 200), far under the
    tolerance floor. Every row and column carries some code-0 groups, and one weight
    row is code 0 throughout, so its outputs are the bias alone in the reference."""
    from ayaka.kernel.hip import mxfp8_scaled_mm

    _say(f"mxfp8_scaled_mm code-0 weight scales m={m} n={n} k={k}")
    qa, ca, qw, cw = _mx_edge_operands(m, n, k)
    mask = torch.rand(cw.shape, generator=_gen(52)) < 0.2
    cw = torch.where(mask, torch.zeros_like(cw), cw)
    cw[3, :] = 0
    assert (qw[3].float() != 0).any() and int(ca.max()) <= 200
    bias = torch.randn(n, generator=_gen(53))
    ref = ora.mxfp8_scaled_mm(qa, ca, qw, cw, bias)
    assert torch.equal(ref[:, 3], bias[3].expand(m)), "oracle: a code-0 row contributes exactly 0"
    out = torch.empty(m, n, dtype=torch.float32, device=gpu)
    mxfp8_scaled_mm(qa.to(gpu), ca.to(gpu), qw.to(gpu), cw.to(gpu), bias.to(gpu), out=out)
    assert_linear_close(out, ref, "mxfp8 code-0 weight scales")
    assert (out[:, 3].cpu() - bias[3]).abs().max().item() < 1e-20


@pytest.mark.parametrize("m,n,k", MX_EDGE)
def test_mxfp8_code_ff_scales_give_nan(gpu, m, n, k):
    """UE8M0 code 0xFF is NaN (reference fp8_compat e8m0 decode and reference/gemm.py:11-14):
    every output whose dot product touches a 0xFF group, weight side or activation side,
    is NaN; all other outputs are unaffected."""
    from ayaka.kernel.hip import mxfp8_scaled_mm

    _say(f"mxfp8_scaled_mm code-0xFF scales m={m} n={n} k={k}")
    qa, ca, qw, cw = _mx_edge_operands(m, n, k)
    cw[5, 2] = 0xFF
    ca[m // 2, k // 32 - 1] = 0xFF
    ref = ora.mxfp8_scaled_mm(qa, ca, qw, cw)
    out = torch.empty(m, n, dtype=torch.float32, device=gpu)
    mxfp8_scaled_mm(qa.to(gpu), ca.to(gpu), qw.to(gpu), cw.to(gpu), out=out)
    y = out.cpu()
    nan_ref = torch.isnan(ref)
    assert nan_ref[:, 5].all() and nan_ref[m // 2, :].all()
    assert torch.equal(torch.isnan(y), nan_ref), (
        f"NaN pattern differs: kernel {int(torch.isnan(y).sum())} NaNs, oracle {int(nan_ref.sum())}")
    keep = ~nan_ref
    assert_linear_close(y[keep], ref[keep], "mxfp8 0xFF: finite outputs")


@pytest.mark.parametrize("m", [4, 16, 32, 100])
@pytest.mark.parametrize("case", ["channel", "block128", "e8m0_32"])
def test_weight_only_gemm(gpu, m, case):
    from ayaka.kernel.hip import fp8_weight_only_gemm

    n, k = 640, 1024
    _say(f"fp8_weight_only_gemm m={m} case={case}")
    w = _fp8((n, k), seed=10)
    if case == "channel":
        by, bx, sdt = 1, k, "float32"
        scale = torch.rand(n, 1, generator=_gen(1)) * 0.01 + 1e-3
    elif case == "block128":
        by, bx, sdt = 128, 128, "bfloat16"
        scale = (torch.rand(n // 128, k // 128, generator=_gen(1)) * 0.01 + 1e-3).to(torch.bfloat16)
    else:
        by, bx, sdt = 1, 32, "e8m0"
        scale = torch.randint(115, 125, (n, k // 32), generator=_gen(1), dtype=torch.uint8)
    x = torch.randn(m, k, generator=_gen(2)).to(torch.bfloat16)
    y = fp8_weight_only_gemm(x.to(gpu), w.to(gpu), scale.to(gpu), -(-k // bx), by, bx, sdt)
    ref = ora.fp8_weight_only_gemm(x, w, scale, -(-k // bx), by, bx, sdt)
    assert y.dtype == torch.bfloat16
    assert_linear_close(y, ref, "weight_only_gemm")


def _weight_only_operands(n, k, case, seed=10):
    w = _fp8((n, k), seed=seed)
    if case == "channel":
        by, bx, sdt = 1, k, "float32"
        scale = torch.rand(n, 1, generator=_gen(1)) * 0.01 + 1e-3
    elif case == "channel_e8m0":
        by, bx, sdt = 1, k, "e8m0"
        scale = torch.randint(115, 125, (n, 1), generator=_gen(1), dtype=torch.uint8)
    elif case == "block128":
        by, bx, sdt = 128, 128, "bfloat16"
        scale = (torch.rand(-(-n // 128), k // 128, generator=_gen(1)) * 0.01 + 1e-3).to(torch.bfloat16)
    else:
        by, bx, sdt = 1, 32, "e8m0"
        scale = torch.randint(115, 125, (n, k // 32), generator=_gen(1), dtype=torch.uint8)
    return w, scale, by, bx, sdt


# Decode-batch launch plans: a K split of 2 and 4 (K >= 8192, few row tiles), 64-row
# tiles (M > 16, N >= 384 * 64), activation rows padded to 8 (M = 5, 9, 13, 27), row
# counts that are not a multiple of the tile, every scale dtype, fp16 activations.
@pytest.mark.parametrize("m,n,k,case,xdt", [
    (5, 600, 8192, "channel", torch.bfloat16),
    (27, 24640, 512, "block128", torch.bfloat16),
    (13, 100, 16384, "e8m0_32", torch.float16),
    (9, 200, 768, "channel_e8m0", torch.bfloat16),
    (32, 24576, 256, "channel", torch.float16),
])
def test_weight_only_gemm_decode_plans(gpu, m, n, k, case, xdt):
    from ayaka.kernel.hip import fp8_weight_only_gemm

    _say(f"fp8_weight_only_gemm decode plan m={m} n={n} k={k} case={case} x={xdt}")
    w, scale, by, bx, sdt = _weight_only_operands(n, k, case)
    x = torch.randn(m, k, generator=_gen(2)).to(xdt)
    y = fp8_weight_only_gemm(x.to(gpu), w.to(gpu), scale.to(gpu), -(-k // bx), by, bx, sdt)
    ref = ora.fp8_weight_only_gemm(x, w, scale, -(-k // bx), by, bx, sdt)
    assert y.dtype == xdt
    assert_linear_close(y, ref, "weight_only_gemm decode plan")


# Wide decode projections (N >= 24576), and narrower ones at M <= 8 with a four-way K
# split inside the workgroup, take the stream kernel: every staged activation
# row count (4, 8, 16, 32), ragged N (not a multiple of 64, nor of 16), every scale
# layout, fp16, K whose stage count leaves a remainder after the unrolled loop (3584:
# 14 stages in rounds of 6) or runs the remainder only (512: 2 stages).
@pytest.mark.parametrize("m,n,k,case,xdt", [
    (4, 24576, 4096, "channel", torch.bfloat16),
    (5, 24640, 1536, "e8m0_32", torch.bfloat16),
    (13, 24600, 2048, "block128", torch.float16),
    (32, 24576, 3584, "channel_e8m0", torch.bfloat16),
    (2, 28672, 512, "channel", torch.float16),
    (17, 24704, 2560, "block128", torch.bfloat16),
    # narrower projections at M <= 8: four K quarters of 16 rows per workgroup
    (3, 1000, 6144, "e8m0_32", torch.float16),
    (7, 3000, 2048, "block128", torch.bfloat16),
    (4, 8192, 14336, "channel", torch.bfloat16),
    # 9-16 rows over a long K: whole-K 16-row wavefronts with a grid K split (fixed-order reduce)
    (16, 4096, 14336, "channel", torch.bfloat16),
    (9, 1000, 8192, "block128", torch.float16),
    (12, 700, 12288, "e8m0_32", torch.bfloat16),
])
def test_weight_only_gemm_stream(gpu, m, n, k, case, xdt):
    from ayaka.kernel.hip import fp8_weight_only_gemm

    _say(f"fp8_weight_only_gemm stream m={m} n={n} k={k} case={case} x={xdt}")
    w, scale, by, bx, sdt = _weight_only_operands(n, k, case)
    x = torch.randn(m, k, generator=_gen(2)).to(xdt)
    y = fp8_weight_only_gemm(x.to(gpu), w.to(gpu), scale.to(gpu), -(-k // bx), by, bx, sdt)
    ref = ora.fp8_weight_only_gemm(x, w, scale, -(-k // bx), by, bx, sdt)
    assert y.dtype == xdt and y.shape == (m, n)
    assert_linear_close(y, ref, "weight_only_gemm stream")


# Narrow decode projections (K too short to split) run the row-stream kernel with 16
# weight rows per workgroup while those workgroups fit one per CU (two up to 16 rows):
# every staged activation row count (8, 16, 24, 32), ragged N, every scale layout, fp16.
# Each case asserts the plan; a longer K keeps the 32-row workgroups and its K split.
@pytest.mark.parametrize("m,n,k,case,xdt,plan", [
    (6, 300, 768, "channel", torch.bfloat16, "w8a16 rows rt=1 xj=1 split=1"),
    (10, 4096, 4096, "channel_e8m0", torch.bfloat16, "w8a16 rows rt=1 xj=2 split=1"),
    (16, 6144, 4096, "block128", torch.float16, "w8a16 rows rt=1 xj=2 split=1"),
    (20, 1000, 1024, "e8m0_32", torch.bfloat16, "w8a16 rows rt=1 xj=3 split=1"),
    (32, 4090, 2048, "block128", torch.bfloat16, "w8a16 rows rt=1 xj=4 split=1"),
    (32, 6144, 4096, "channel", torch.float16, "w8a16 rows rt=2 xj=4 split=1"),
    (32, 4096, 14336, "channel", torch.bfloat16, "w8a16 rows rt=2 xj=4 split=2"),
])
def test_weight_only_gemm_rows_plans(gpu, m, n, k, case, xdt, plan):
    from ayaka.kernel.hip import fp8_weight_only_gemm

    _say(f"fp8_weight_only_gemm rows m={m} n={n} k={k} case={case} x={xdt}")
    w, scale, by, bx, sdt = _weight_only_operands(n, k, case)
    x = torch.randn(m, k, generator=_gen(2)).to(xdt)
    y = fp8_weight_only_gemm(x.to(gpu), w.to(gpu), scale.to(gpu), -(-k // bx), by, bx, sdt)
    assert _plan() == plan
    ref = ora.fp8_weight_only_gemm(x, w, scale, -(-k // bx), by, bx, sdt)
    assert y.dtype == xdt and y.shape == (m, n)
    assert_linear_close(y, ref, "weight_only_gemm rows")


@pytest.mark.parametrize("m,n,k", [(300, 512, 1024), (4096, 768, 2048), (65, 384, 1024)])
def test_block_linear_column_major_scales_match_row_major(gpu, m, n, k):
    """Above 64 rows the block-128 linear quantizes with column-major scales; its output
    equals the row-major composition bit for bit (the same scale values, read in another
    layout, in the same K order)."""
    from ayaka.kernel.hip import fp8_block_linear, fp8_blockwise_mm, per_token_group_quant_fp8

    _say(f"fp8_block_linear column-major scales m={m} n={n} k={k}")
    x = torch.randn(m, k, generator=_gen(4)).to(torch.bfloat16).to(gpu)
    w = _fp8((n, k), seed=5).to(gpu)
    ws = (torch.rand(n // 128, k // 128, generator=_gen(6)) * 1e-3 + 1e-4).to(gpu)
    bias = torch.randn(n, generator=_gen(7)).to(torch.bfloat16).to(gpu)
    y = fp8_block_linear(x, w, ws, bias)
    q, s = per_token_group_quant_fp8(x, 128)
    ref = fp8_blockwise_mm(q, w, s, ws, bias=bias, out=torch.empty(m, n, dtype=torch.bfloat16, device=gpu))
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


# 2-8 rows of the fp32-scaled GEMM against a weight of at most 2^24 bytes take the
# GEMV-shaped kernel (VALU fmas of exact fp8 products); more rows or a larger weight keep
# the MFMA decode-batch kernel.
@pytest.mark.parametrize("m,n,k,rowwise,out_dtype,with_bias,plan", [
    (2, 4096, 4096, True, torch.bfloat16, True, "rows_gemv"),
    (3, 1001, 2048, False, torch.float16, False, "rows_gemv"),
    (4, 6144, 2048, True, torch.float32, True, "rows_gemv"),
    (2, 300, 256, True, torch.bfloat16, True, "rows_gemv"),
    (5, 3072, 1024, True, torch.bfloat16, True, "rows_gemv"),
    (8, 4096, 2048, False, torch.bfloat16, True, "rows_gemv"),
    (7, 2050, 1024, True, torch.float16, True, "rows_gemv"),
    (8, 8192, 4096, True, torch.bfloat16, True, "skinny"),
    (9, 3072, 1024, True, torch.bfloat16, True, "skinny"),
])
def test_fp8_scaled_mm_small_batch_plans(gpu, m, n, k, rowwise, out_dtype, with_bias, plan):
    from ayaka.kernel.hip import fp8_scaled_mm

    _say(f"fp8_scaled_mm small batch m={m} n={n} k={k} rowwise={rowwise} out={out_dtype}")
    a = _fp8((m, k), seed=m + 7, scale=40)
    w = _fp8((n, k), seed=n + 7, scale=40)
    sa = (torch.rand(m, generator=_gen(1)) * 0.01 + 1e-3) if rowwise else torch.tensor(0.004)
    sb = (torch.rand(n, generator=_gen(2)) * 0.01 + 1e-3) if rowwise else torch.tensor(0.002)
    bias = torch.randn(n, generator=_gen(3)).to(torch.bfloat16) if with_bias else None
    ref = ora.fp8_scaled_mm(a, w, sa, sb, bias)
    out = torch.empty(m, n, dtype=out_dtype, device=gpu)
    fp8_scaled_mm(a.to(gpu), w.to(gpu).t(), sa.to(gpu), sb.to(gpu), bias.to(gpu) if with_bias else None, out=out)
    assert _plan().startswith(plan)
    assert_linear_close(out, ref, "fp8_scaled_mm small batch")


# 2-8 rows of the rowwise linear against a small weight: per-token quantization fused
# into the GEMV-shaped kernel, bit-identical to the quantizer launch followed by the
# GEMM; a NaN row and an infinite row take the quantizer's IEEE-division path.
@pytest.mark.parametrize("m,n,k,xdt,scalar_scale,with_bias", [
    (8, 3072, 1024, torch.bfloat16, False, True),
    (2, 4096, 4096, torch.float16, True, False),
    (5, 1000, 2048, torch.float32, False, True),
    (3, 300, 256, torch.bfloat16, False, False),
    (6, 520, 8192, torch.bfloat16, True, True),  # two rows on some wavefronts, long rows
    (7, 264, 1040, torch.float16, False, False),  # a row length that is no multiple of 64 vectors
])
def test_rowwise_linear_small_fused_quant_is_bit_identical(gpu, m, n, k, xdt, scalar_scale, with_bias):
    from ayaka.kernel.hip import fp8_scaled_mm, per_token_quant_fp8
    from ayaka.kernel.hip.gemm.fp8_gemm import fp8_rowwise_linear_small

    _say(f"fp8_rowwise_linear_small m={m} n={n} k={k} x={xdt}")
    x = (torch.randn(m, k, generator=_gen(11)) * 3).to(xdt)
    x[m - 1, 5] = float("nan")
    if m > 2:
        x[1, 7] = float("inf")
    w = _fp8((n, k), seed=12, scale=40)
    ws = torch.tensor(0.003) if scalar_scale else torch.rand(n, generator=_gen(13)) * 0.01 + 1e-3
    bias = torch.randn(n, generator=_gen(14)).to(xdt) if with_bias else None
    xg, wg, sg = x.to(gpu), w.to(gpu), ws.to(gpu)
    bg = bias.to(gpu) if with_bias else None
    fused = fp8_rowwise_linear_small(xg, wg, sg, bg)
    assert _plan() == "rows_gemv quant"
    q, s = per_token_quant_fp8(xg)
    two = fp8_scaled_mm(q, wg.t(), s, sg, bg, out=torch.empty(m, n, dtype=xdt, device=gpu))
    view = torch.int32 if xdt == torch.float32 else torch.int16
    assert torch.equal(fused.view(view), two.view(view))
    # and against the oracle on the rows without a non-finite element
    ref = ora.fp8_scaled_mm(q.cpu(), w, s.cpu(), ws, bias)
    rows = [i for i in range(m) if torch.isfinite(x[i]).all()]
    assert_linear_close(fused[rows].cpu(), ref[rows], "fp8_rowwise_linear_small")


# ------------------------------------------------------------------ linear entry points
@pytest.mark.parametrize("m", [1, 8, 40])
@pytest.mark.parametrize("recipe", ["w8a8_rowwise", "w8a8_dynamic_per_tensor", "w8a8_block128"])
def test_fp8_linear_entry_points(gpu, m, recipe):
    from ayaka.kernel.hip import fp8_block_linear, fp8_pertensor_linear, fp8_rowwise_linear

    n, k = 384, 1024
    _say(f"fp8 linear recipe={recipe} m={m}")
    wf = torch.randn(n, k, generator=_gen(1)) * 0.02
    if recipe == "w8a8_block128":
        blocks = wf.reshape(n // 128, 128, k // 128, 128).abs().amax(dim=(1, 3))
        scale = blocks / 448.0
        w = (wf / scale.repeat_interleave(128, 0).repeat_interleave(128, 1)).clamp(-448, 448).to(FP8)
    elif recipe == "w8a8_rowwise":
        scale = wf.abs().amax(dim=1) / 448.0
        w = (wf / scale[:, None]).to(FP8)
    else:
        scale = (wf.abs().amax() / 448.0).reshape(())
        w = (wf / scale).to(FP8)
    x = torch.randn(2, m, k, generator=_gen(2)).to(torch.bfloat16) if m > 1 else torch.randn(1, k, generator=_gen(2)).to(torch.bfloat16)
    bias = torch.randn(n, generator=_gen(3)).to(torch.bfloat16)
    # W8A8 GEMM paths fuse the bias before the single rounding; M == 1 adds it after.
    ref = ora.fp8_linear(recipe, x, w, scale, bias, bias_in_fp32=True)
    fn = {"w8a8_rowwise": fp8_rowwise_linear, "w8a8_dynamic_per_tensor": fp8_rowwise_linear,
          "w8a8_block128": fp8_block_linear}[recipe]
    y = fn(x.to(gpu), w.to(gpu), scale.to(gpu), bias.to(gpu))
    assert y.shape == ref.shape and y.dtype == torch.bfloat16
    assert_linear_close(y, ref, recipe)
    if recipe == "w8a8_dynamic_per_tensor":
        y2 = fp8_pertensor_linear(x.to(gpu), w.to(gpu), scale.to(gpu), bias.to(gpu))
        ref2 = ora.fp8_linear("w8a16", x, w, scale.reshape(1, 1).expand(1, 1), bias, weight_block=(n, k))
        assert_linear_close(y2, ref2, "pertensor weight-only")


@pytest.mark.parametrize(
    "m,n,k,case,xdt",
    [
        (2, 600, 1152, "channel", torch.bfloat16),   # ragged N, uneven K split
        (5, 4096, 4096, "block128", torch.bfloat16),  # split 1 shape family
        (32, 96, 8192, "e8m0_32", torch.float16),     # deep split, partial last wave
        (17, 8320, 256, "channel", torch.float16),    # many wavefronts, no split
    ],
)
def test_weight_only_gemm_decode_shapes(gpu, m, n, k, case, xdt):
    """Decode batches (M <= 32) take the K-split streaming kernel."""
    from ayaka.kernel.hip import fp8_weight_only_gemm

    _say(f"fp8_weight_only_gemm decode m={m} n={n} k={k} case={case} {xdt}")
    w = _fp8((n, k), seed=11)
    if case == "channel":
        by, bx, sdt = 1, k, "float32"
        scale = torch.rand(n, 1, generator=_gen(1)) * 0.01 + 1e-3
    elif case == "block128":
        by, bx, sdt = 128, 128, "float32"
        scale = torch.rand(-(-n // 128), k // 128, generator=_gen(1)) * 0.01 + 1e-3
    else:
        by, bx, sdt = 1, 32, "e8m0"
        scale = torch.randint(115, 125, (n, k // 32), generator=_gen(1), dtype=torch.uint8)
    x = torch.randn(m, k, generator=_gen(2)).to(xdt)
    y = fp8_weight_only_gemm(x.to(gpu), w.to(gpu), scale.to(gpu), -(-k // bx), by, bx, sdt)
    ref = ora.fp8_weight_only_gemm(x, w, scale, -(-k // bx), by, bx, sdt)
    assert y.dtype == xdt and y.shape == (m, n)
    assert_linear_close(y, ref, "weight_only_gemm")


# ------------------------------------------------------------------ INT8 GEMM
def _i8(shape, seed):
    return torch.randint(-128, 128, shape, generator=_gen(seed), dtype=torch.int8)


INT8_MNK = [(8, 3072, 1024), (17, 300, 256), (200, 1000, 1040),  # general kernel (K % 64 != 0 included)
            (300, 520, 1024), (400, 300, 320), (260, 1028, 1216), (2304, 8192, 640)]  # 256x256 kernels


@pytest.mark.parametrize("m,n,k", INT8_MNK)
@pytest.mark.parametrize("with_bias", [False, True])
def test_int8_scaled_mm(gpu, m, n, k, with_bias):
    from ayaka.kernel.hip import int8_scaled_mm

    _say(f"int8_scaled_mm m={m} n={n} k={k} bias={with_bias}")
    a, w = _i8((m, k), m), _i8((n, k), n)
    sa = torch.rand(m, generator=_gen(1)) * 1e-3 + 1e-4
    sb = torch.rand(n, generator=_gen(2)) * 1e-3 + 1e-4
    bias = torch.randn(n, generator=_gen(3)).to(torch.bfloat16) if with_bias else None
    ref = ora.int8_scaled_mm(a, w, sa, sb, bias)
    args = (a.to(gpu), w.to(gpu).t(), sa.to(gpu), sb.to(gpu), None if bias is None else bias.to(gpu))
    y = int8_scaled_mm(*args)
    assert y.dtype == torch.bfloat16  # the reference's default out_dtype
    assert_linear_close(y, ref, "int8_scaled_mm bf16")
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device=gpu)
    r = int8_scaled_mm(*args, out=out)
    assert r is out
    # fp32 output: the same fp32 epilogue as the oracle up to the compiler's fused
    # multiply-add of the bias.
    torch.testing.assert_close(out.cpu(), ref, rtol=2e-6, atol=1e-6 * ref.abs().max().item())


@pytest.mark.parametrize("m,n,k", [(64, 256, 512), (512, 512, 1024), (520, 1040, 2048)])
def test_int8_scaled_mm_integer_sum_is_exact(gpu, m, n, k):
    """Unit scales, fp32 output: every int32 sum below 2^24 comes out exactly."""
    from ayaka.kernel.hip import int8_scaled_mm

    _say(f"int8_scaled_mm exact m={m} n={n} k={k}")
    a, w = _i8((m, k), 5), _i8((n, k), 6)
    exact = ora.int8_matmul_exact(a, w)
    assert exact.abs().max().item() < 2**24
    out = int8_scaled_mm(a.to(gpu), w.to(gpu).t(), torch.ones(m, device=gpu), torch.ones(n, device=gpu), out_dtype=torch.float32)
    assert torch.equal(out.cpu().to(torch.int64), exact)


@pytest.mark.parametrize("m,n,k", [(512, 768, 8192), (40, 768, 8192)])
def test_int8_scaled_mm_short_launch_is_exact(gpu, m, n, k):
    """Launches short of one round of tiles (which split K for the fp8 recipes) keep
    the INT8 GEMM unsplit: no workspace, and with full-range int8 operands (sums far
    above 2^24) the fp32 output is the exact int32 sum rounded once, as torch's
    int32 -> float32 conversion of the reference's int32 accumulator
    (gemm/int8_gemm.py:70-81)."""
    from ayaka.kernel.hip import _lib, int8_scaled_mm

    _say(f"int8_scaled_mm short launch exact m={m} n={n} k={k}")
    assert _lib.query("ayk_int8_scaled_mm_workspace_bytes", m, n, k) == 0, "INT8 must not split K"
    a = torch.randint(-128, 128, (m, k), generator=_gen(41), dtype=torch.int8)
    w = torch.randint(-128, 128, (n, k), generator=_gen(42), dtype=torch.int8)
    a[:4, : k // 2] = 127  # a few sums of order 127^2 K / 2 = 6.6e7, far beyond 2^24
    w[:4, : k // 2] = 127
    exact = ora.int8_matmul_exact(a, w)
    assert exact.abs().max().item() > 2**24, "the case must exercise sums beyond fp32's integer range"
    out = int8_scaled_mm(a.to(gpu), w.to(gpu).t(), torch.ones(m, device=gpu), torch.ones(n, device=gpu), out_dtype=torch.float32)
    assert torch.equal(out.cpu(), exact.to(torch.int32).to(torch.float32))


def test_int8_scaled_mm_row_major_b_and_contract(gpu):
    from ayaka.kernel.hip import int8_scaled_mm

    _say("int8_scaled_mm row-major b and errors")
    m, n, k = 96, 200, 256
    a, w = _i8((m, k), 8), _i8((n, k), 9)
    sa, sb = (torch.rand(m, generator=_gen(1)) + 0.5) * 1e-3, (torch.rand(n, generator=_gen(2)) + 0.5) * 1e-3
    ref = ora.int8_scaled_mm(a, w, sa, sb)  # |ref| well inside the fp16 range
    b_kn = w.t().contiguous().to(gpu)  # [K, N] row-major
    y = int8_scaled_mm(a.to(gpu), b_kn, sa.to(gpu), sb.to(gpu), out_dtype=torch.float16)
    assert y.dtype == torch.float16
    assert_linear_close(y, ref, "int8 row-major b")
    with pytest.raises(TypeError):
        int8_scaled_mm(a.to(gpu).to(torch.float8_e4m3fn), b_kn, sa.to(gpu), sb.to(gpu))
    with pytest.raises(TypeError):
        int8_scaled_mm(a.to(gpu), b_kn, sa.to(gpu).half(), sb.to(gpu))
    with pytest.raises(ValueError):
        int8_scaled_mm(a.to(gpu), b_kn, torch.tensor(1.0, device=gpu), sb.to(gpu))  # scalar scale
    with pytest.raises(ValueError):
        int8_scaled_mm(a[:, :250].contiguous().to(gpu), b_kn[:250], sa.to(gpu), sb.to(gpu))  # K % 16
    with pytest.raises(ValueError):
        int8_scaled_mm(a.to(gpu), b_kn, sa.to(gpu), sb.to(gpu), out_dtype=torch.int32)
