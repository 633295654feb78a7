"""GPU: the allocation-free decode GEMV entry point against the allocating one.

``ayk_fp8_weight_only_gemv_static`` keeps its split-K partials in a static per-device
array instead of a caller workspace. Called through the C ABI, twice in a row (the
second call smaller, so stale partials of the first would show), it must match
``ayk_fp8_weight_only_gemv`` with a torch-allocated workspace bit for bit, and both
must match the oracle.
"""

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


def _case(n, k, seed, gpu):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * 40).clamp(-448, 448).to(FP8)
    s = torch.rand(n, 1, generator=g) * 0.01 + 1e-3
    x = torch.randn(k, generator=g).to(torch.bfloat16)
    return w, s, x, w.to(gpu), s.to(gpu), x.to(gpu)


def _run(lib, name, x, w, s, n, k, out, ws=None):
    from ayaka.kernel.hip import _lib

    stream = torch.cuda.current_stream().cuda_stream
    args = [x.data_ptr(), _lib.AYK_BF16, w.data_ptr(), k, n, k, s.data_ptr(), _lib.AYK_F32, 1, 1, k, out.data_ptr()]
    if name == "ayk_fp8_weight_only_gemv":
        args += [None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel() * ws.element_size()]
    rc = getattr(lib, name)(*args, stream)
    assert rc == 0, (name, rc, lib.ayk_last_error())


# (first call, second smaller call): both split K, so the static array holds partials
PAIRS = [((512, 14336), (256, 4096)), ((3000, 8192), (40, 4096)), ((1024, 14336), (100, 2048))]


@pytest.mark.parametrize("first,second", PAIRS)
def test_static_gemv_matches_workspace_gemv(gpu, first, second):
    from ayaka.kernel.hip import _lib

    lib = _lib.load_library()
    assert lib.ayk_fp8_weight_only_gemv_static_max_bytes() == 64 * 1024
    for idx, (n, k) in enumerate((first, second)):
        _say(f"no-alloc GEMV call {idx}: N={n} K={k}")
        need = lib.ayk_fp8_weight_only_gemv_workspace_bytes(n, k)
        assert 0 < need <= lib.ayk_fp8_weight_only_gemv_static_max_bytes(), "the case must use the scratch"
        w, s, x, wd, sd, xd = _case(n, k, 7 + idx, gpu)
        ws = torch.empty(need // 4, dtype=torch.float32, device=gpu)
        out_ws = torch.empty(n, dtype=torch.bfloat16, device=gpu)
        out_static = torch.full((n,), float("nan"), dtype=torch.bfloat16, device=gpu)
        _run(lib, "ayk_fp8_weight_only_gemv", xd, wd, sd, n, k, out_ws, ws)
        _run(lib, "ayk_fp8_weight_only_gemv_static", xd, wd, sd, n, k, out_static)
        torch.cuda.synchronize()
        assert torch.equal(out_static.cpu(), out_ws.cpu()), "static scratch result differs from the workspace result"
        assert_linear_close(out_static, ora.fp8_weight_only_gemv(x, w, s, 1, 1, k, "float32"), "static gemv")


def test_static_gemv_argument_errors(gpu):
    from ayaka.kernel.hip import _lib

    lib = _lib.load_library()
    rc = lib.ayk_fp8_weight_only_gemv_static(None, _lib.AYK_F32, None, 16, 4, 16, None, _lib.AYK_F32, 1, 1, 16, None, None)
    assert rc == _lib.AYK_EINVAL and b"float16 or bfloat16" in lib.ayk_last_error()
