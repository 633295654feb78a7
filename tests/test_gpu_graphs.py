"""GPU: the operators are HIP-graph capture safe.

A decode-style sequence (quant, split-K GEMV, scaled GEMM, MX path) is captured once
and replayed several times, with eager work and synchronisations between replays;
every replay must equal the eager result bit for bit (the kernels are deterministic
and allocate nothing themselves; the K-split workspace comes from torch's graph pool).
"""

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu
FP8 = torch.float8_e4m3fn


def test_graph_replays_match_eager(gpu):
    import ayaka.kernel.hip as H

    print("graph capture / replay", flush=True)
    sys.stdout.flush()
    g = torch.Generator(device=gpu).manual_seed(0)
    x = torch.randn(4096, generator=g, device=gpu).to(torch.bfloat16)
    w = (torch.randn(4096, 4096, generator=g, device=gpu) * 30).clamp(-448, 448).to(FP8)  # split-K shape
    ws = torch.rand(4096, generator=g, device=gpu) * 1e-3
    xa = torch.randn(48, 4096, generator=g, device=gpu).to(torch.bfloat16)

    def work():
        y1 = H.fp8_weight_only_gemv(x, w, ws, 1, 1, 4096, "float32")
        q, s = H.per_token_quant_fp8(xa)
        y2 = H.fp8_scaled_mm(q, w.t(), s, ws, out=torch.empty(48, 4096, dtype=torch.bfloat16, device=gpu))
        qm, cm = H.per_token_group_quant_mxfp8(xa, 32)
        wm, cw = H.per_token_group_quant_mxfp8(w.float()[:512].to(torch.bfloat16), 32)
        y3 = H.mxfp8_scaled_mm(qm, cm, wm, cw, out=torch.empty(48, 512, dtype=torch.bfloat16, device=gpu))
        return y1, y2, y3

    eager = [t.clone() for t in work()]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        work()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            outs = work()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for replay in range(4):
        for t in outs:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for e, o in zip(eager, outs):
            assert torch.equal(e.view(torch.int16), o.view(torch.int16)), f"replay {replay} differs from eager"
        _ = work()  # eager traffic between replays
        torch.cuda.synchronize()
