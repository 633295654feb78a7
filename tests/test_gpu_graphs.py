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


def test_graph_replays_kv_cache_moe_int8_block(gpu):
    """A serving-style step: KV write of the step's tokens into fp8 pages, a
    dequantizing gather, the MoE grouped GEMM (both pointer-table flavours, device-side
    problem sizes), the INT8 GEMM, the block-128 GEMM and split-K block-128 and MXFP8
    GEMMs, captured once. Writes of the
    same tokens to the same slots are idempotent, so every replay must reproduce the
    eager caches and outputs bit for bit."""
    import ayaka.kernel.hip as H

    print("graph capture / replay: kv cache, moe, int8, block", flush=True)
    sys.stdout.flush()
    g = torch.Generator(device=gpu).manual_seed(1)
    key = torch.randn(8, 8, 128, generator=g, device=gpu).to(torch.bfloat16)
    val = torch.randn(8, 8, 128, generator=g, device=gpu).to(torch.bfloat16)
    kc = torch.zeros(16, 16, 8, 128, dtype=FP8, device=gpu)
    vc = torch.zeros_like(kc)
    slots = torch.randperm(256, generator=g, device=gpu)[:8]
    gidx = torch.randint(0, 256, (24,), generator=g, device=gpu)
    e, n, k = 4, 256, 512
    counts = torch.tensor([3, 0, 70, 9], dtype=torch.int32)
    offs = torch.cat([torch.zeros(1, dtype=torch.int64), counts.long().cumsum(0)[:-1]]).to(torch.int32).to(gpu)
    ps = torch.stack([counts, torch.full_like(counts, n), torch.full_like(counts, k)], 1).to(gpu)
    rows = int(counts.sum())
    a = (torch.randn(rows, k, generator=g, device=gpu) * 40).clamp(-448, 448).to(FP8)
    b = (torch.randn(e, n, k, generator=g, device=gpu) * 40).clamp(-448, 448).to(FP8)
    sa = torch.rand(rows, k // 128, generator=g, device=gpu) * 1e-3
    sb = torch.rand(e, n // 128, k // 128, generator=g, device=gpu) * 1e-3
    i64 = lambda: torch.zeros(e, dtype=torch.int64, device=gpu)  # noqa: E731
    tables = [i64() for _ in range(5)]
    strides = [torch.full((e,), v, dtype=torch.int64, device=gpu) for v in (k, k, n)]
    lay = [torch.zeros(e, 5, dtype=torch.int32, device=gpu) for _ in range(2)]
    wsp = torch.empty(1, dtype=torch.uint8, device=gpu)
    a8 = torch.randint(-128, 128, (40, 256), generator=g, device=gpu, dtype=torch.int8)
    w8 = torch.randint(-128, 128, (384, 256), generator=g, device=gpu, dtype=torch.int8)
    s8a, s8w = torch.rand(40, generator=g, device=gpu) * 1e-3, torch.rand(384, generator=g, device=gpu) * 1e-3
    ab = (torch.randn(200, 512, generator=g, device=gpu) * 40).clamp(-448, 448).to(FP8)
    wb = (torch.randn(256, 512, generator=g, device=gpu) * 40).clamp(-448, 448).to(FP8)
    sab = torch.rand(200, 4, generator=g, device=gpu)
    sbb = torch.rand(2, 4, generator=g, device=gpu)
    # split-K shapes: block-128 (32 rows, 4 splits) and MXFP8 (64 rows, 8 splits); their
    # partial-sum workspaces come from the graph's pool
    a_sk = (torch.randn(32, 4096, generator=g, device=gpu) * 40).clamp(-448, 448).to(FP8)
    w_sk = (torch.randn(1024, 4096, generator=g, device=gpu) * 40).clamp(-448, 448).to(FP8)
    sa_sk = torch.rand(32, 32, generator=g, device=gpu)
    sb_sk = torch.rand(8, 32, generator=g, device=gpu)
    a_mx = (torch.randn(64, 8192, generator=g, device=gpu) * 40).clamp(-448, 448).to(FP8)
    w_mx = (torch.randn(1024, 8192, generator=g, device=gpu) * 40).clamp(-448, 448).to(FP8)
    ca_mx = torch.randint(110, 125, (64, 256), generator=g, device=gpu, dtype=torch.uint8)
    cw_mx = torch.randint(110, 125, (1024, 256), generator=g, device=gpu, dtype=torch.uint8)

    def work():
        H.write_kv(key, val, kc, vc, slots, 0.5, 0.25)
        dq = torch.empty(24, 8, 128, dtype=torch.bfloat16, device=gpu)
        H.gather_cache(kc, gidx, dq, 2.0, True)
        outs = [dq]
        for swap in (False, True):
            o = torch.zeros(rows, n, dtype=torch.bfloat16, device=gpu)
            H.fp8_blockwise_scaled_grouped_mm(o, *tables, a, b, sa, sb, *strides, *lay, ps, offs, wsp, swap_ab=swap)
            outs.append(o)
        outs.append(H.int8_scaled_mm(a8, w8.t(), s8a, s8w))
        outs.append(H.fp8_blockwise_mm(ab, wb, sab, sbb))
        outs.append(H.fp8_blockwise_mm(a_sk, w_sk, sa_sk, sb_sk))
        outs.append(H.mxfp8_scaled_mm(a_mx, ca_mx, w_mx, cw_mx, out=torch.empty(64, 1024, dtype=torch.bfloat16, device=gpu)))
        return outs

    eager = [t.clone() for t in work()]
    eager_kc, eager_vc = kc.clone(), vc.clone()
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

    def bits(t):
        return t.view(torch.uint8) if t.element_size() == 1 else t.view(torch.int16)

    for replay in range(4):
        for t in outs:
            t.fill_(float("nan"))
        kc.zero_()
        vc.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(bits(kc), bits(eager_kc)) and torch.equal(bits(vc), bits(eager_vc)), f"replay {replay}: caches"
        for i, (e_, o) in enumerate(zip(eager, outs)):
            assert torch.equal(bits(e_), bits(o)), f"replay {replay}: output {i} differs from eager"
        _ = work()  # eager traffic between replays
        torch.cuda.synchronize()
