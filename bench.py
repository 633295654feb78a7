"""Benchmark of the MI355X FP8 linear path (one JSON line on stdout).

Headline (``value``): BASELINE.json configs[1] -- W8A16 rowwise decode GEMV on the
four Llama-3-8B projections (qkv 6144x4096, o 4096x4096, gate_up 28672x4096,
down 4096x14336) at M = 1. One step runs all four projections through
``ayaka::fp8_weight_only_gemv`` exactly as ``FP8W8A16LinearMethod.apply`` calls it;
``value`` is the step's algorithmic bytes (fp8 weights + fp32 row scales + bf16 x and
out) divided by its wall time, in GB/s. Inputs are resident in HBM before timing;
three independent weight/scale copies (654 MB) are rotated across steps so the
256 MB MALL cannot serve them.

Each step is replayed as a HIP graph (the four launches of one decode step), as a
serving loop runs decode; the eager per-op dispatch time is reported beside it.
``roofline`` is the dominant kernel (the gate_up GEMV, the only launch of its op):
a graph of back-to-back launches is replayed between two events on its stream and
the elapsed time divided by the launch count. ``gemm`` adds the prefill
GEMMs at M = 4096 (TFLOP/s against the 5.0 PFLOP/s dense fp8 peak) and
``cpu_baseline`` times the reference's CPU path (the oracle restatement) on a
bounded sample on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-gemm] [--no-cpu] [--copy-probe]
"""

import argparse
import itertools
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "ayaka-py_amd"), ROOT]

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
CFG2_SHAPES = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336)]
COPIES = 3


def _gemv_bytes(n: int, k: int, m: int = 1) -> int:
    return n * k + 4 * n + 2 * m * k + 2 * m * n


def _quant_rowwise(wf: torch.Tensor):
    scale = wf.abs().amax(dim=1).clamp_min(1e-12) / 448.0
    return (wf / scale[:, None]).clamp(-448, 448).to(torch.float8_e4m3fn), scale.float()


def _make_cfg2(device, seed=0):
    g = torch.Generator(device=device).manual_seed(seed)
    layers = []
    for name, n, k in CFG2_SHAPES:
        copies = []
        for _ in range(COPIES):
            wf = torch.randn(n, k, generator=g, device=device) * 0.02
            copies.append(_quant_rowwise(wf))
            del wf
        gx = torch.Generator(device=device).manual_seed(1)
        x = torch.randn(k, generator=gx, device=device)
        idx = torch.randperm(k, generator=gx, device=device)[: k // 100]
        x[idx] *= 20.0
        layers.append((name, n, k, copies, x.to(torch.bfloat16)))
    return layers


def _gemv_step(layers, step, out_bufs):
    from ayaka.kernel.hip import fp8_weight_only_gemv

    c = step % COPIES
    for (name, n, k, copies, x), out in zip(layers, out_bufs):
        w, s = copies[c]
        fp8_weight_only_gemv(x, w, s, 1, 1, k, "float32", out=out)


def _capture(fn):
    """HIP graph of ``fn`` (captured on a side stream, replayed on the current one)."""
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn()  # warm the allocator outside the capture
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            fn()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    return graph


def _time_dominant(layers, launches_per_graph=24, replays=5):
    """Per-launch time of the gate_up GEMV: a graph of back-to-back launches (rotating
    the weight copies) replayed between two events on the replay stream."""
    from ayaka.kernel.hip import fp8_weight_only_gemv

    name, n, k, copies, x = layers[2]
    out = torch.empty(n, dtype=torch.bfloat16, device=x.device)

    def launches():
        for i in range(launches_per_graph):
            w, s = copies[i % COPIES]
            fp8_weight_only_gemv(x, w, s, 1, 1, k, "float32", out=out)

    graph = _capture(launches)
    stream = torch.cuda.current_stream()
    per_launch = []
    for _ in range(replays):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        graph.replay()
        end.record(stream)
        end.synchronize()
        per_launch.append(start.elapsed_time(end) / launches_per_graph)
    per_launch.sort()
    return n, k, sum(per_launch) / len(per_launch), per_launch[len(per_launch) // 2]


def _bench_gemm(device, reps=20, warmup=5):
    """Prefill GEMMs at M = 4096 on the config shapes (supplemental M for MXFP8). Each is
    timed over `reps` launches after `warmup` untimed ones (the clocks settle over the
    first few milliseconds of matrix-core load)."""
    from ayaka.kernel.hip import fp8_blockwise_mm, fp8_scaled_mm, mxfp8_scaled_mm

    g = torch.Generator(device=device).manual_seed(0)
    m = 4096
    results = {}

    def run(label, n, k, fn, m=m):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / reps
        tflops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        results[label] = {"M": m, "N": n, "K": k, "ms": round(ms, 4), "tflops": round(tflops, 1),
                          "frac": round(tflops / FP8_PEAK_TFLOPS, 4)}

    fp8 = torch.float8_e4m3fn
    # rowwise, Qwen2-7B gate_up (Cfg3 shape, M = 4096 between its 2048 and 8192 points)
    n, k = 37888, 3584
    a = (torch.randn(m, k, generator=g, device=device) * 50).clamp(-448, 448).to(fp8)
    w = (torch.randn(n, k, generator=g, device=device) * 50).clamp(-448, 448).to(fp8)
    sa = torch.rand(m, generator=g, device=device) * 1e-3
    sb = torch.rand(n, generator=g, device=device) * 1e-3
    out = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    run("rowwise_qwen2_gate_up", n, k, lambda: fp8_scaled_mm(a, w.t(), sa, sb, out=out))
    run("per_tensor_qwen2_gate_up", n, k, lambda: fp8_scaled_mm(a, w.t(), sa[0], sb[0], out=out))
    del a, w, out
    # rowwise Qwen2 down (Cfg3) at M = 512 and 2048: few 256 x 256 tiles, so K splits.
    # Weight-bound sizes: 5 rotated weight copies (340 MB) keep every launch on HBM.
    n, k = 3584, 18944
    wds = [(torch.randn(n, k, generator=g, device=device) * 50).clamp(-448, 448).to(fp8) for _ in range(5)]
    sbd = torch.rand(n, generator=g, device=device) * 1e-3
    for m_small in (512, 2048):
        a_s = (torch.randn(m_small, k, generator=g, device=device) * 50).clamp(-448, 448).to(fp8)
        sa_s = torch.rand(m_small, generator=g, device=device) * 1e-3
        out_s = torch.empty(m_small, n, dtype=torch.bfloat16, device=device)
        cyc = itertools.cycle(wds)
        run(f"rowwise_qwen2_down_m{m_small}", n, k,
            lambda: fp8_scaled_mm(a_s, next(cyc).t(), sa_s, sbd, out=out_s), m=m_small)
    del wds, a_s, out_s
    # block-128, DeepSeek-V3 dense (Cfg4, M = 4096)
    n, k = 18432, 7168
    a = (torch.randn(m, k, generator=g, device=device) * 50).clamp(-448, 448).to(fp8)
    w = (torch.randn(n, k, generator=g, device=device) * 50).clamp(-448, 448).to(fp8)
    sa = torch.rand(m, k // 128, generator=g, device=device)
    sb = torch.rand(n // 128, k // 128, generator=g, device=device)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    run("block128_dsv3_18432x7168", n, k, lambda: fp8_blockwise_mm(a, w, sa, sb, out=out))
    # Cfg4's smaller batches: few tiles, so the K split applies (M = 32: 32-row tiles).
    # Weight-bound sizes: 3 rotated weight copies (396 MB) keep every launch on HBM.
    wbs = [w] + [(torch.randn(n, k, generator=g, device=device) * 50).clamp(-448, 448).to(fp8) for _ in range(2)]
    for m_small in (32, 256):
        a_s, sa_s = a[:m_small].contiguous(), sa[:m_small].contiguous()
        out_s = torch.empty(m_small, n, dtype=torch.bfloat16, device=device)
        cyc = itertools.cycle(wbs)
        run(f"block128_dsv3_18432x7168_m{m_small}", n, k,
            lambda: fp8_blockwise_mm(a_s, next(cyc), sa_s, sb, out=out_s), m=m_small)
    del wbs
    del a, w, out
    # MXFP8, Llama-3-70B gate_up (Cfg5 shape, supplemental M = 4096)
    n, k = 57344, 8192
    a = (torch.randn(m, k, generator=g, device=device) * 50).clamp(-448, 448).to(fp8)
    w = (torch.randn(n, k, generator=g, device=device) * 50).clamp(-448, 448).to(fp8)
    ca = torch.randint(100, 130, (m, k // 32), generator=g, device=device, dtype=torch.uint8)
    cw = torch.randint(100, 130, (n, k // 32), generator=g, device=device, dtype=torch.uint8)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    run("mxfp8_llama70b_gate_up", n, k, lambda: mxfp8_scaled_mm(a, ca, w, cw, out=out))
    del a, w, out
    # INT8 rowwise scaled GEMM, on the Qwen2 gate_up shape
    from ayaka.kernel.hip import int8_scaled_mm

    n, k = 37888, 3584
    a = torch.randint(-128, 128, (m, k), generator=g, device=device, dtype=torch.int8)
    w = torch.randint(-128, 128, (n, k), generator=g, device=device, dtype=torch.int8)
    sa = torch.rand(m, generator=g, device=device) * 1e-4
    sb = torch.rand(n, generator=g, device=device) * 1e-4
    out = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    run("int8_rowwise_qwen2_gate_up", n, k, lambda: int8_scaled_mm(a, w.t(), sa, sb, out=out))
    del a, w, out
    torch.cuda.empty_cache()
    return results


def _bench_moe(device, reps=10, warmup=3):
    """MoE FP8 block-128 grouped GEMM at the DeepSeek-V3 MoE gate_up shape: 256 experts,
    4096 tokens routed top-8 (32768 rows, per-expert counts from a seeded multinomial),
    N = 2 x 2048, K = 7168. Useful FLOPs: 2 x rows x N x K."""
    from ayaka.kernel.hip import fp8_blockwise_scaled_grouped_mm

    g = torch.Generator(device="cpu").manual_seed(0)
    experts, tokens, topk, n, k = 256, 4096, 8, 4096, 7168
    counts = torch.bincount(torch.multinomial(torch.ones(experts), tokens * topk, replacement=True, generator=g),
                            minlength=experts)
    rows = int(counts.sum())
    offsets = torch.cat([torch.zeros(1, dtype=torch.int64), counts.cumsum(0)[:-1]]).to(torch.int32)
    ps = torch.stack([counts, torch.full_like(counts, n), torch.full_like(counts, k)], 1).to(torch.int32)
    gd = torch.Generator(device=device).manual_seed(1)
    fp8 = torch.float8_e4m3fn
    a = (torch.randn(rows, k, generator=gd, device=device) * 50).clamp(-448, 448).to(fp8)
    b = torch.empty(experts, n, k, dtype=fp8, device=device)
    for e0 in range(0, experts, 32):  # in slices: a full fp32 staging tensor would be 30 GB
        b[e0:e0 + 32] = (torch.randn(32, n, k, generator=gd, device=device) * 50).clamp(-448, 448).to(fp8)
    sa = torch.rand(rows, k // 128, generator=gd, device=device) * 1e-3
    sb = torch.rand(experts, n // 128, k // 128, generator=gd, device=device) * 1e-3
    out = torch.empty(rows, n, dtype=torch.bfloat16, device=device)
    i64 = lambda: torch.empty(experts, dtype=torch.int64, device=device)  # noqa: E731
    ptrs = [i64() for _ in range(5)]
    strides = [torch.full((experts,), v, dtype=torch.int64, device=device) for v in (k, k, n)]
    lay = [torch.empty(experts, 5, dtype=torch.int32, device=device) for _ in range(2)]
    ps_d, off_d = ps.to(device), offsets.to(device)
    ws = torch.empty(1, dtype=torch.uint8, device=device)

    def run():
        fp8_blockwise_scaled_grouped_mm(out, *ptrs, a, b, sa, sb, *strides, *lay, ps_d, off_d, ws)

    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        run()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    tflops = 2.0 * rows * n * k / (ms * 1e-3) / 1e12
    result = {"experts": experts, "rows": rows, "N": n, "K": k, "max_rows_per_expert": int(counts.max()),
              "ms": round(ms, 4), "tflops": round(tflops, 1), "frac": round(tflops / FP8_PEAK_TFLOPS, 4)}
    del a, b, out
    torch.cuda.empty_cache()
    return result


def _time_rotated(fns, reps: int, warmup: int) -> float:
    """Average ms per call over `reps` calls cycling through `fns` (input copies whose
    total exceeds the 256 MB Infinity Cache, so each call streams from HBM)."""
    for i in range(warmup):
        fns[i % len(fns)]()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(reps):
        fns[i % len(fns)]()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def _hbm_entry(ms: float, nbytes: int, **extra) -> dict:
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {**extra, "us": round(ms * 1e3, 2), "bytes": nbytes, "GB/s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4)}


def _bench_kv_cache(device, reps=40, warmup=8, copies=4):
    """FP8 KV-cache write (bf16 K/V -> e4m3 pages) and dequantizing gather (e4m3 -> bf16)
    for a 16384-token prefill chunk of Llama-3-8B (8 KV heads x 128) into a 65536-slot
    cache at shuffled slots, rotating over `copies` sources and caches. Algorithmic bytes:
    write 2 planes x (2 B read + 1 B written) per element + 8 B per slot; gather 1 B read
    + 2 B written per element + 8 B per slot."""
    from ayaka.kernel.hip import gather_cache, write_kv

    g = torch.Generator(device=device).manual_seed(0)
    n, heads, dim, pages, page_size = 16384, 8, 128, 4096, 16
    width = heads * dim
    sets = []
    for _ in range(copies):
        key = torch.randn(n, heads, dim, generator=g, device=device).to(torch.bfloat16)
        value = torch.randn(n, heads, dim, generator=g, device=device).to(torch.bfloat16)
        k_cache = torch.zeros(pages, page_size, heads, dim, device=device, dtype=torch.float8_e4m3fn)
        v_cache = torch.zeros_like(k_cache)
        slots = torch.randperm(pages * page_size, generator=g, device=device)[:n]
        dest = torch.empty(n, heads, dim, device=device, dtype=torch.bfloat16)
        sets.append((key, value, k_cache, v_cache, slots, dest))
    writes = [lambda s=s: write_kv(s[0], s[1], s[2], s[3], s[4], 0.5, 0.5) for s in sets]
    gathers = [lambda s=s: gather_cache(s[2], s[4], s[5], 2.0, True) for s in sets]
    results = {
        "write_kv_bf16_to_e4m3": _hbm_entry(_time_rotated(writes, reps, warmup), 2 * n * width * 3 + 8 * n,
                                            tokens=n, width=width),
        "gather_e4m3_to_bf16": _hbm_entry(_time_rotated(gathers, reps, warmup), n * width * 3 + 8 * n,
                                          tokens=n, width=width),
    }
    del sets, writes, gathers
    torch.cuda.empty_cache()
    return results


def _bench_quant(device, reps=40, warmup=8, copies=6):
    """Activation quantizers on bf16 prefill activations (M = 4096) at the config hidden
    sizes, rotating over `copies` inputs. Algorithmic bytes: 2 B read + 1 B written per
    element, plus the scales written."""
    from ayaka.kernel.hip import (per_token_group_quant_fp8, per_token_group_quant_mxfp8, per_token_quant_fp8,
                                  static_quant_fp8)

    g = torch.Generator(device=device).manual_seed(0)
    m = 4096
    results = {}

    def inputs(k):
        return [torch.randn(m, k, generator=g, device=device).to(torch.bfloat16) for _ in range(copies)]

    xs = inputs(3584)
    results["per_token_qwen2_k3584"] = _hbm_entry(
        _time_rotated([lambda x=x: per_token_quant_fp8(x) for x in xs], reps, warmup), m * 3584 * 3 + m * 4, M=m, K=3584)
    scale = torch.full((), 0.05, device=device)
    outs = [torch.empty(m, 3584, dtype=torch.float8_e4m3fn, device=device) for _ in xs]
    results["static_qwen2_k3584"] = _hbm_entry(
        _time_rotated([lambda x=x, o=o: static_quant_fp8(x, scale, out=o) for x, o in zip(xs, outs)], reps, warmup),
        m * 3584 * 3, M=m, K=3584)
    del xs, outs
    xs = inputs(7168)
    results["group128_dsv3_k7168"] = _hbm_entry(
        _time_rotated([lambda x=x: per_token_group_quant_fp8(x, 128) for x in xs], reps, warmup),
        m * 7168 * 3 + m * 56 * 4, M=m, K=7168)
    del xs
    xs = inputs(8192)
    results["mxfp8_llama70b_k8192"] = _hbm_entry(
        _time_rotated([lambda x=x: per_token_group_quant_mxfp8(x, 32) for x in xs], reps, warmup),
        m * 8192 * 3 + m * 256, M=m, K=8192)
    del xs
    torch.cuda.empty_cache()
    return results


def _bench_decode_m(layers, reps=20):
    """W8A16 at the other Cfg2 decode batch sizes (M = 4, 16, 32): GB/s per projection
    (algorithmic bytes: fp8 weights + scales + bf16 x and out), each launch timed in a
    graph of back-to-back launches rotating the weight copies."""
    from ayaka.kernel.hip import fp8_weight_only_gemm

    out = {}
    for m in (4, 16, 32):
        row = {}
        for name, n, k, copies, x in layers:
            xm = x.reshape(1, k).repeat(m, 1).contiguous()
            y = torch.empty(m, n, dtype=torch.bfloat16, device=x.device)

            def launches():
                for i in range(reps):
                    w, s = copies[i % COPIES]
                    fp8_weight_only_gemm(xm, w, s.reshape(n, 1), 1, 1, k, "float32", out=y)

            graph = _capture(launches)
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            graph.replay()
            end.record()
            end.synchronize()
            us = start.elapsed_time(end) * 1e3 / reps
            row[name] = {"us": round(us, 2), "gbs": round(_gemv_bytes(n, k, m) / (us * 1e-6) / 1e9, 1)}
        out[f"M={m}"] = row
    return out


def _cpu_baseline():
    """The reference's CPU path (oracle restatement) on one Cfg2 M = 1 pass."""
    from oracle import fp8_oracle as ora

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)
    layers = []
    for _, n, k in CFG2_SHAPES:
        w, s = _quant_rowwise(torch.randn(n, k, generator=g) * 0.02)
        layers.append((n, k, w, s, torch.randn(1, k, generator=g).to(torch.bfloat16)))
    total_bytes = sum(_gemv_bytes(n, k) for n, k, *_ in layers)

    def one_pass():
        for n, k, w, s, x in layers:
            ora.fp8_linear("w8a16", x, w, s.reshape(n, 1), weight_block=(1, k), scale_dtype="float32")

    one_pass()  # warmup
    reps = []
    for _ in range(3):
        t0 = time.perf_counter()
        one_pass()
        reps.append(time.perf_counter() - t0)
    sec = sorted(reps)[1]
    return {"value": round(total_bytes / sec / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": "one Cfg2 M=1 pass (4 projections, 218 MB of fp8 weights), median of 3 after 1 warmup, "
            f"{sec:.2f} s per pass; oracle/fp8_oracle.fp8_linear('w8a16') on torch CPU"}


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "gemv_gate_up_traffic.md")


def _measured_traffic():
    """HBM bytes per gate_up GEMV launch from the committed counter summary (FETCH_SIZE +
    WRITE_SIZE, scaled by the copy-kernel calibration it records), or None."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip())
    except (OSError, ValueError):
        return None
    return None


def _copy_probe(device, mib=256, reps=5):
    """A plain device copy of a known size (counter calibration for the traffic figure)."""
    src = torch.ones(mib << 18, dtype=torch.float32, device=device)
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": src.numel() * 4, "copy_probe_bytes_written": dst.numel() * 4,
                      "launches": reps}), flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", action="store_true", help="only run a 256 MiB device copy (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the FP8 linear path is "
              "single-device here and multi-GPU runs are not part of this build", file=sys.stderr)
        return 2

    import ayaka.kernel.hip  # noqa: F401  (registers the ops)

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.copy_probe:
        _copy_probe(device)
        return 0
    layers = _make_cfg2(device)
    outs = [torch.empty(n, dtype=torch.bfloat16, device=device) for _, n, _, _, _ in layers]
    step_bytes = sum(_gemv_bytes(n, k) for _, n, k, _, _ in layers)

    # Eager (one Python dispatch per projection): host-bound at decode sizes.
    for i in range(args.warmup):
        _gemv_step(layers, i, outs)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        _gemv_step(layers, i, outs)
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / args.steps

    # Graph mode: each step (the four projections on one weight copy) is a HIP graph,
    # replayed back to back as a decode loop does; copies rotate every step.
    graphs = [_capture(lambda c=c: _gemv_step(layers, c, outs)) for c in range(COPIES)]
    for i in range(args.warmup):
        graphs[i % COPIES].replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        graphs[i % COPIES].replay()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    n, k, avg_ms, med_ms = _time_dominant(layers)
    achieved = _gemv_bytes(n, k) / (avg_ms * 1e-3) / 1e9
    result = {
        "metric": "FP8 linear: GEMV GB/s (% HBM peak) @M=1; GEMM TFLOP/s (% MFMA) @M=4096",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e4m3 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded N(0,0.02) weights, per-row e4m3 quant; N(0,1) activations with 1% x20 outlier channels)",
        "config": {"workload": "BASELINE configs[1]: W8A16 rowwise GEMV, Llama-3-8B decode, M=1, qkv+o+gate_up+down",
                   "shapes_NK": [[n_, k_] for _, n_, k_ in CFG2_SHAPES], "weight_copies_rotated": COPIES,
                   "launch": "one HIP graph per step (4 projections)"},
        "eager": {"ms_per_step": round(eager_ms, 5), "value": round(step_bytes / (eager_ms * 1e-3) / 1e9, 1),
                  "note": "one Python op dispatch per projection, no graph"},
        "roofline": {"bound": "hbm", "kernel": "gemv_stream_kernel (gate_up 28672x4096)", "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "avg_launch_us": round(avg_ms * 1e3, 2), "median_launch_us": round(med_ms * 1e3, 2),
                     "bytes_per_launch": _gemv_bytes(n, k), "traffic": _measured_traffic()},
    }
    result["decode_w8a16"] = _bench_decode_m(layers)
    if not args.no_gemm:
        result["gemm"] = _bench_gemm(device)
        result["moe_grouped_block128"] = _bench_moe(device)
    result["quant"] = _bench_quant(device)
    result["kv_cache"] = _bench_kv_cache(device)
    if not args.no_cpu:
        result["cpu_baseline"] = _cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
