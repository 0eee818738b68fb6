"""Benchmark of the CAM MoE hot path on one MI355X.

Default workload (benchmark config 2, "dispatch/combine at the DeepSeek-V3
one-rank shape"): T=4096 tokens, H=7168, E=256 experts, top-8, router logits
~N(0,1) plus a per-expert bias ~N(0,0.5); one step = route -> layout -> count
exchange -> fp8 1x128 dispatch -> combine of identity-expert bf16 rows, run as
the plan runs it (camhipMoePrefillDispatch + camhipMoePrefillCombine, four
launches); the reference-shaped eight-launch chain is timed beside it.
Inputs are synthetic, seeded, resident in HBM before the timed region.

Prints ONE JSON line (rank 0).  `value` is tokens/s of the whole step;
`roofline` is for the dominant kernel (the combine gather), measured with HIP
events on the launch stream over the timed steps; `cpu_baseline` times the
C oracle (oracle/cam_oracle.c, one thread) on the same workload.
"""
import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
METRIC = "MoE-layer tokens/s; dispatch+combine HBM GB/s; fp8 grouped-GEMM TFLOPS"


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "dispatch_combine_cfg2_hbm_counters.md")


def measured_traffic(kernels):
    """HBM bytes per launch of `kernels` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this
    workload (the table's scaled read + write MB columns), or None when the table is absent."""
    try:
        rows = [l.split("|") for l in open(TRAFFIC_PROFILE) if l.startswith("| `")]
    except OSError:
        return None
    total = 0.0
    for k in kernels:
        hit = [r for r in rows if k in r[1]]
        if len(hit) != 1:
            return None
        total += (float(hit[0][4]) + float(hit[0][5])) * 1e6
    return total


def dispatch_bytes(T, H, K):
    # read x once; write T*K fp8 rows, their 1x128 scales and the (rank,t,k) triples;
    # read topk ids, send_token_idx and offsets
    return T * H * 2 + T * K * H + T * K * (H // 128) * 4 + T * K * 12 + T * K * 8


def combine_bytes(T, H, K):
    # read T*K bf16 expert rows, the weights and the row map; write T bf16 rows
    return T * K * H * 2 + T * K * 4 + T * K * 12 + T * H * 2


def cpu_baseline(T, H, E, K, seed):
    import numpy as np

    from oracle import oracle as orc
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).bfloat16().view(torch.int16).numpy().view(np.uint16)
    logits = torch.randn(T, E, generator=g).numpy()
    bias = (torch.randn(E, generator=g) * 0.5).numpy()
    y = torch.randn(T * K, H, generator=g).bfloat16().view(torch.int16).numpy().view(np.uint16)
    reps, t0 = 0, time.perf_counter()
    while True:
        idx, w = orc.route(logits, bias, K)
        _, nte, _, sti = orc.dispatch_layout(idx.astype(np.int64), E, 1)
        so, _, _, _ = orc.notify_dispatch(nte)
        ex, sc, eidx = orc.dispatch(x, idx, so, sti, E, orc.QUANT_FP8)
        orc.combine(y, eidx, idx, w, E)
        reps += 1
        if time.perf_counter() - t0 > 10.0:  # a bounded ~10 s sample of CPU work
            break
    dt = (time.perf_counter() - t0) / reps
    threads = orc.num_threads()
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), model)
    except OSError:
        pass
    return {"value": T / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"full config-2 step (T={T}, H={H}, E={E}, K={K}) x{reps} on the C oracle, {threads} OpenMP "
                      f"threads over tokens (route, dispatch, combine; layout serial) of {os.cpu_count()} visible "
                      f"CPUs ({model}); {dt * 1e3:.0f} ms/step"}


def cpu_gemm_row_seconds(dt, H, I, seed, budget_s=5.0):
    """Seconds per routed row of the C oracle's GMM1+SwiGLU+GMM2 (OpenMP over rows) at one expert's
    shapes, timed on batches of rows until a bounded ~5 s sample is spent."""
    import numpy as np

    from oracle import oracle as orc
    rng = np.random.default_rng(seed)
    rows = max(orc.num_threads(), 8)
    cnt = np.array([rows], np.int64)
    if dt == "fp8":
        A = rng.integers(0, 0x7e, (rows, H), dtype=np.uint8)
        As = np.full((rows, H // 128), 0.01, np.float32)
        W1 = rng.integers(0, 0x7e, (1, 2 * I, H), dtype=np.uint8)
        W1s = np.full((1, 2 * I // 128, H // 128), 0.01, np.float32)
        W2 = rng.integers(0, 0x7e, (1, H, I), dtype=np.uint8)
        W2s = np.full((1, H // 128, I // 128), 0.01, np.float32)
        step = lambda: orc.gmm2_fp8(*orc.gmm1_swiglu_fp8(A, As, cnt, W1, W1s), cnt, W2, W2s)  # noqa: E731
    else:
        bf = lambda *sh: (torch.randn(*sh) * 0.05).bfloat16().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
        A, W1, W2 = bf(rows, H), bf(1, 2 * I, H), bf(1, H, I)
        step = lambda: orc.gmm2_bf16(orc.gmm1_swiglu_bf16(A, cnt, W1), cnt, W2)  # noqa: E731
    n, t0 = 0, time.perf_counter()
    while True:
        step()
        n += rows
        if time.perf_counter() - t0 > budget_s:
            break
    return (time.perf_counter() - t0) / n, n


def cpu_decode_baseline(x, logits, w1, s1, w2, s2, K, L, budget_s=10.0):
    """The C oracle's whole decode step on the config-5 inputs themselves: route over all experts, layout and
    count exchange over the L local experts, fp8 dispatch, GMM1 + SwiGLU + fp8 requant, GMM2, combine;
    repeated for a bounded ~10 s sample."""
    import numpy as np

    from oracle import oracle as orc
    T = x.shape[0]
    xb = x.cpu().view(torch.int16).numpy().view(np.uint16)
    lg = logits.cpu().numpy()
    u8 = lambda t: t.cpu().contiguous().view(torch.uint8).numpy()  # noqa: E731
    hw1, hw2, hs1, hs2 = u8(w1), u8(w2), s1.cpu().numpy(), s2.cpu().numpy()
    reps, t0 = 0, time.perf_counter()
    while True:
        idx, w = orc.route(lg, None, K)
        rid = np.where(idx < L, idx, -1).astype(np.int32)
        _, nte, _, sti = orc.dispatch_layout(rid.astype(np.int64), L, 1)
        so, _, _, _ = orc.notify_dispatch(nte)
        ex, xs, eidx = orc.dispatch(xb, rid, so, sti, L, orc.QUANT_FP8)
        cnt = nte.astype(np.int64)
        hq, hs = orc.gmm1_swiglu_fp8(ex, xs, cnt, hw1, hs1)
        y = orc.gmm2_fp8(hq, hs, cnt, hw2, hs2)
        orc.combine(y, eidx, rid, w, L)
        reps += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = (time.perf_counter() - t0) / reps
    threads = orc.num_threads()
    return {"value": dt * 1e6, "unit": "us per step (lower is better)", "tokens_per_s": T / dt, "cores": threads,
            "kind": "port",
            "sample": f"the config-5 step on the same inputs x{reps} through the C oracle (route, layout, fp8 "
                      f"dispatch, GMM1+SwiGLU, GMM2, combine; {int(cnt.sum())} local rows), {threads} OpenMP "
                      f"threads; {dt * 1e3:.1f} ms/step"}


def cpu_layer_full(x, logits, bias, w1, s1, w2, s2, K, L, budget_s=8.0):
    """The C oracle's whole fp8 layer on the layer's own inputs: route (with the expert bias) over all experts,
    layout and count exchange over the L local experts, fp8 dispatch, GMM1 + SwiGLU + fp8 requant, GMM2,
    combine; whole layers repeated until ~budget_s (at least one)."""
    import numpy as np

    from oracle import oracle as orc
    T = x.shape[0]
    xb = x.cpu().view(torch.int16).numpy().view(np.uint16)
    lg = logits.cpu().numpy()
    bs = None if bias is None else bias.cpu().numpy()
    u8 = lambda t: t.cpu().contiguous().view(torch.uint8).numpy()  # noqa: E731
    hw1, hw2, hs1, hs2 = u8(w1), u8(w2), s1.cpu().numpy(), s2.cpu().numpy()
    reps, t0 = 0, time.perf_counter()
    while True:
        idx, w = orc.route(lg, bs, K)
        rid = np.where(idx < L, idx, -1).astype(np.int32)
        _, nte, _, sti = orc.dispatch_layout(rid.astype(np.int64), L, 1)
        so, _, _, _ = orc.notify_dispatch(nte)
        ex, xs, eidx = orc.dispatch(xb, rid, so, sti, L, orc.QUANT_FP8)
        cnt = nte.astype(np.int64)
        hq, hs = orc.gmm1_swiglu_fp8(ex, xs, cnt, hw1, hs1)
        y = orc.gmm2_fp8(hq, hs, cnt, hw2, hs2)
        orc.combine(y, eidx, rid, w, L)
        reps += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = (time.perf_counter() - t0) / reps
    threads = orc.num_threads()
    return {"value": T / dt, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{reps} whole layer(s) on the same inputs through the C oracle (route with the expert bias, "
                      f"layout, fp8 dispatch, GMM1+SwiGLU, GMM2, combine; {int(cnt.sum())} local rows), {threads} "
                      f"OpenMP threads; {dt:.2f} s per layer"}


def cpu_layer_baseline(cfg_cpu, dt, T, H, I, M, seed):
    """CPU oracle time of one layer too long to run whole (config 3: ~80 s per layer): a ~5 s sample of rows
    through the oracle's expert GEMMs scaled to M, plus cfg_cpu's measured bookkeeping step when given (None
    for config 3, whose bookkeeping is < 1% of its GEMMs)."""
    from oracle import oracle as orc
    per_row, n = cpu_gemm_row_seconds(dt, H, I, seed)
    step = (T / cfg_cpu["value"]) if cfg_cpu else 0.0
    t = step + M * per_row
    return {"value": T / t, "unit": "tokens/s", "cores": orc.num_threads(), "kind": "port",
            "sample": f"{n} rows of the C oracle's {dt} GMM1+SwiGLU+GMM2 at H={H}, I={I} "
                      f"({per_row * 1e3:.2f} ms/row, OpenMP over rows) x M={M}"
                      + (f" + the measured config-2 step ({step * 1e3:.0f} ms)" if cfg_cpu else "")
                      + f": {t:.1f} s per layer"}


BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0
INT8_PEAK_TOPS = 5000.0  # dense int8 MFMA, POP/s


def graph_time(fn, n, warmup, stream):
    """ms per call of fn (a sequence of launches, no host synchronisation), over exactly n timed calls: fn is
    captured `reps` times back to back in one HIP graph (reps = the largest of 10, 5, 2, 1 that divides n; a
    model's forward pass would hold the layer in a larger graph, not replay one graph per layer), after two eager
    runs on a side stream; the graph is replayed for the warmup, then n / reps times between two HIP events on
    `stream`."""
    reps = next(r for r in (10, 5, 2, 1) if n % r == 0)
    side = torch.cuda.Stream(device=stream.device)
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        fn()
        fn()
    stream.wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for _ in range(reps):
            fn()
    stream.wait_stream(side)
    with torch.cuda.stream(stream):
        for _ in range(max(3, warmup // reps)):
            graph.replay()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(n // reps):
            graph.replay()
        b.record(stream)
    torch.cuda.synchronize()
    del graph
    return a.elapsed_time(b) / n


def cold_time(fn, n, stream, flush_bytes=512 << 20):
    """(median ms with cold caches, median ms without a flush) of fn over n single-step graph replays, each
    timed by its own pair of HIP events.  The cold runs read a 512 MiB buffer outside the timed region first
    (the reference's timing method flushes the L2 and the 256 MB MALL between timed runs; reading leaves only
    clean lines, so no write-back of the flush lands in the timed step)."""
    flush = torch.ones(flush_bytes // 4, dtype=torch.int32, device=stream.device)
    sink = torch.empty((), dtype=torch.int64, device=stream.device)
    side = torch.cuda.Stream(device=stream.device)
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        fn()
        fn()
    stream.wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        fn()
    stream.wait_stream(side)
    out = []
    for cold in (True, False):
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        with torch.cuda.stream(stream):
            graph.replay()
            for a, b in ev:
                if cold:
                    torch.sum(flush, dim=0, out=sink)
                a.record(stream)
                graph.replay()
                b.record(stream)
        torch.cuda.synchronize()
        t = sorted(a.elapsed_time(b) for a, b in ev)
        out.append(t[len(t) // 2])
    del graph, flush
    return out[0], out[1]


def zipf_bias(E, s, seed):
    """log-popularity bias: expert popularity ~ 1/rank^s over a seeded permutation of the ids"""
    g = torch.Generator().manual_seed(seed + 17)
    rank = torch.empty(E)
    rank[torch.randperm(E, generator=g)] = torch.arange(1, E + 1, dtype=torch.float32)
    return -s * torch.log(rank)


def make_weights(L, H, I, dtype, dev, seed):
    """W1 [L, 2I, H], W2 [L, H, I] ~ N(0, 0.02); fp8: 128x128 block-quantised e4m3fn + fp32 scales;
    int8: per-output-channel symmetric int8 + fp32 scales [L, n] (the reference's fused-op weights)."""
    g = torch.Generator(device=dev).manual_seed(seed + 5)

    def one(shape):
        w = torch.randn(shape, device=dev, generator=g, dtype=torch.float32) * 0.02
        if dtype == "bf16":
            return w.bfloat16(), None
        if dtype == "int8":
            sc = w.abs().amax(dim=2).clamp(min=1e-6) / 127.0
            q = torch.round(w / sc[:, :, None]).clamp(-127, 127).to(torch.int8)
            del w
            return q, sc.contiguous()
        Ln, n, k = shape
        wv = w.view(Ln, n // 128, 128, k // 128, 128)
        amax = wv.abs().amax(dim=(2, 4)).clamp(min=1e-6)
        sc = amax / 448.0
        q = (wv / sc[:, :, None, :, None]).to(torch.float8_e4m3fn).view(Ln, n, k)
        del wv, w
        return q, sc.contiguous()

    w1, s1 = one((L, 2 * I, H))
    w2, s2 = one((L, H, I))
    return w1, s1, w2, s2


def run_layer(name, T, H, E, K, L, I, dtype, steps, warmup, seed, bias_kind, cpu=False):
    """Full layer (route, layout, dispatch, GMM1+SwiGLU, GMM2, combine) on one rank's L local experts.  cpu
    (fp8 only): also time the C oracle's whole layer on the same inputs (cpu_layer_full)."""
    from umdk_amd.plan import MoeLayerPlan
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).bfloat16().to(dev)
    logits = torch.randn(T, E, generator=g).to(dev)
    bias = zipf_bias(E, 1.1, seed).to(dev) if bias_kind == "zipf" else None
    w1, s1, w2, s2 = make_weights(L, H, I, dtype, dev, seed)
    plan = MoeLayerPlan(T, H, E, K, L, I, dtype=dtype, device=dev)
    stream = torch.cuda.current_stream(dev)

    def step():
        plan.dispatch_step(logits, x, bias)
        plan.experts(w1, s1, w2, s2)
        plan.combine_step(plan.y)

    # HIP-graph replays (see graph_time): the whole layer, then the experts call (both GEMMs: one chained
    # launch where the kernel exists) and each GEMM launch alone on the layer's data
    ms = graph_time(step, steps, warmup, stream)
    gx = graph_time(lambda: plan.experts(w1, s1, w2, s2), steps, warmup, stream)
    g1 = graph_time(lambda: plan.gmm1(w1, s1), steps, warmup, stream)
    g2 = graph_time(lambda: plan.gmm2(w2, s2), steps, warmup, stream)
    counts = plan.recv_tokens_per_expert[:L].cpu()
    M = int(counts.sum())
    touched = int((counts > 0).sum())
    esz = 1 if dtype in ("fp8", "int8") else 2
    f1, f2 = 2.0 * M * H * 2 * I, 2.0 * M * I * H
    wb1, wb2 = touched * 2 * I * H * esz, touched * H * I * esz
    peak = {"fp8": FP8_PEAK_TFLOPS, "int8": INT8_PEAK_TOPS}.get(dtype, BF16_PEAK_TFLOPS)
    # roofline time per GEMM: max(FLOP/peak, weight+activation bytes/HBM peak)
    ab1 = M * H * esz + M * I * esz + wb1
    ab2 = M * I * esz + M * H * 2 + wb2
    roof = max(f1 / (peak * 1e12), ab1 / (HBM_PEAK_GBPS * 1e9)) + max(f2 / (peak * 1e12), ab2 / (HBM_PEAK_GBPS * 1e9))
    tflops = (f1 + f2) / (gx * 1e-3) / 1e12
    cpu_res = cpu_layer_full(x, logits, bias, w1, s1, w2, s2, K, L) if cpu and dtype == "fp8" else None
    del w1, w2
    res = {"workload": name, "tokens": T, "hidden": H, "experts_routed": E, "local_experts": L, "topk": K,
            "intermediate": I, "dtype": dtype, "local_rows_M": M, "experts_touched": touched,
            "ms_per_step": ms, "tokens_per_s": T / (ms * 1e-3),
            "experts_ms": gx, "gmm1_ms": g1, "gmm2_ms": g2, "gemm_tflops": tflops,
            "gemm_frac_of_mfma_peak": tflops / peak, "gemm_roofline_frac": roof / (gx * 1e-3),
            "gemm_bound": "mfma" if (f1 + f2) / (peak * 1e12) > (ab1 + ab2) / (HBM_PEAK_GBPS * 1e9) else "hbm"}
    if cpu_res:
        res["cpu_baseline"] = cpu_res
    return res


def measured_peaks():
    """Practical ceilings of this GPU, for reading the roofline fractions: a STREAM-style device copy and a
    read-only reduction over 2 GiB (HBM), and the vendor GEMM library on large square-ish GEMMs (MFMA):
    bf16 through torch.mm, fp8 e4m3 with per-tensor scales through torch._scaled_mm."""
    dev = torch.device("cuda:0")

    def timed(fn, it=10):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(it):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / it * 1e-3

    n = 1 << 29  # 2 GiB of fp32
    src = torch.empty(n, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    t_copy = timed(lambda: dst.copy_(src))
    t_sum = timed(lambda: src.sum())
    del src, dst
    M = N = K = 8192
    a16 = torch.randn(M, K, device=dev, dtype=torch.bfloat16)
    b16 = torch.randn(N, K, device=dev, dtype=torch.bfloat16)
    t_bf16 = timed(lambda: a16 @ b16.t())
    a8, b8 = a16.to(torch.float8_e4m3fn), b16.to(torch.float8_e4m3fn)
    one = torch.tensor(1.0, device=dev)
    t_fp8 = timed(lambda: torch._scaled_mm(a8, b8.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16))
    del a16, b16, a8, b8
    torch.cuda.empty_cache()
    flop = 2.0 * M * N * K
    return {"copy_TBps": 2 * 4 * n / t_copy / 1e12, "read_TBps": 4 * n / t_sum / 1e12,
            "bf16_mm_TFLOPS": flop / t_bf16 / 1e12, "fp8_scaled_mm_TFLOPS": flop / t_fp8 / 1e12,
            "note": "2 GiB fp32 copy (read + write bytes) and fp32 sum over 2 GiB; 8192^3 GEMMs via the vendor library"}


def gemm_sweep(steps, warmup, seed, ms=(4096, 8192, 16384, 32768, 65536), dt="fp8"):
    """fp8 (or int8 W8A8) GMM1+GMM2 at DeepSeek-V3 expert shapes (32 experts, H=7168, I=2048) for
    growing M."""
    from umdk_amd import ops
    dev = torch.device("cuda:0")
    H, I, L = 7168, 2048, 32
    w1, s1, w2, s2 = make_weights(L, H, I, dt, dev, seed)
    oq = 3 if dt == "fp8" else 2
    out = []
    for M in ms:
        gl = torch.full((L,), M // L, dtype=torch.int64, device=dev)
        if dt == "fp8":
            xq = (torch.randn(M, H, device=dev) * 0.5).to(torch.float8_e4m3fn)
            xs = torch.full((M, H // 128), 0.01, device=dev)
        else:
            xq = torch.randint(-127, 128, (M, H), dtype=torch.int8, device=dev)
            xs = torch.full((M,), 0.01, device=dev)
        for _ in range(warmup):
            h, hs = ops.grouped_matmul_swiglu(xq, xs, gl, w1, s1, oq)
            ops.grouped_matmul(h, hs, gl, w2, s2)
        torch.cuda.synchronize()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        e[0].record()
        for _ in range(steps):
            h, hs = ops.grouped_matmul_swiglu(xq, xs, gl, w1, s1, oq)
        e[1].record()
        for _ in range(steps):
            ops.grouped_matmul(h, hs, gl, w2, s2)
        e[2].record()
        torch.cuda.synchronize()
        t1 = e[0].elapsed_time(e[1]) / steps
        t2 = e[1].elapsed_time(e[2]) / steps
        f1, f2 = 2.0 * M * H * 2 * I, 2.0 * M * I * H
        out.append({"M": M, "gmm1_ms": t1, "gmm1_tflops": f1 / t1 / 1e9, "gmm2_ms": t2, "gmm2_tflops": f2 / t2 / 1e9,
                    "frac_of_peak": (f1 + f2) / (t1 + t2) / 1e9 / (FP8_PEAK_TFLOPS if dt == "fp8" else INT8_PEAK_TOPS)})
    return out


def run_decode(steps, seed, dtype="fp8", cpu=False):
    """Config 5: decode step (T=128, H=7168, route over 256 experts, 32 local experts, I=2048, fp8)
    = route + fused_deep_moe captured in one HIP graph; p50/p99 of single-replay times.  dtype "int8"
    runs the same step with the reference's int8 W8A8 weights (per-channel scales)."""
    import numpy as np

    from umdk_amd import _lib
    T, H, E, K, L, I = 128, 7168, 256, 8, 32, 2048
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).bfloat16().to(dev)
    logits = torch.randn(T, E, generator=g).to(dev)
    w1, s1, w2, s2 = make_weights(L, H, I, dtype, dev, seed)
    ids = torch.empty(T, K, dtype=torch.int32, device=dev)
    wts = torch.empty(T, K, dtype=torch.float32, device=dev)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    share = torch.empty(T, H, dtype=torch.bfloat16, device=dev)
    etn = torch.empty(L, dtype=torch.int64, device=dev)
    fargs = (x.data_ptr(), ids.data_ptr(), w1.data_ptr(), s1.data_ptr(), w2.data_ptr(), s2.data_ptr(),
             wts.data_ptr(), None, None, None, None, None, None, None, T, H, K, 2 * I, 0, 3 if dtype == "fp8" else 2,
             1, 0, L, 0, 0,
             out.data_ptr(), share.data_ptr(), etn.data_ptr())
    ws = torch.empty(_lib.workspace_size("camhipFusedDeepMoe", *fargs), dtype=torch.uint8, device=dev)

    def step():
        # routing over all 256 experts; ids of the 224 non-local experts are not routed on this rank
        _lib.launch("camhipMoeRoute", logits.data_ptr(), None, T, E, K, ids.data_ptr(), wts.data_ptr(), None,
                    device=dev)
        _lib.launch("camhipFusedDeepMoe", *fargs, workspace=ws, device=dev)

    st = torch.cuda.Stream(device=dev)
    st.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(st):
        for _ in range(3):
            step()
    torch.cuda.current_stream(dev).wait_stream(st)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(20):
        graph.replay()
    torch.cuda.synchronize()
    times = []
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in evs:
        a.record()
        graph.replay()
        b.record()
    torch.cuda.synchronize()
    single = np.array([a.elapsed_time(b) * 1e3 for a, b in evs])
    del graph
    # per layer inside a model's graph: LAYERS consecutive steps captured in one graph (as a decode forward pass
    # holds every layer in one graph), each replay timed; per-layer time = replay time / LAYERS
    LAYERS = 10
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(LAYERS):
            step()
    for _ in range(5):
        graph.replay()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(max(steps // LAYERS, 1))]
    for a, b in evs:
        a.record()
        graph.replay()
        b.record()
    torch.cuda.synchronize()
    times = np.array([a.elapsed_time(b) * 1e3 / LAYERS for a, b in evs])
    del graph
    counts = etn.cpu()
    touched = int((counts > 0).sum())
    wbytes = touched * 3 * H * I   # 1-byte W1 (2I x H) + W2 (H x I) of touched experts
    p50 = float(np.percentile(times, 50))
    cpu_base = cpu_decode_baseline(x, logits, w1, s1, w2, s2, K, L) if cpu and dtype == "fp8" else None
    res = {"workload": f"config5: decode step, route + fused_deep_moe in one HIP graph, {dtype}", "tokens": T,
            "hidden": H, "experts_routed": E, "local_experts": L, "topk": K, "intermediate": I,
            "layer_steps": len(evs) * LAYERS, "timing": f"{len(evs)} replays of a graph of {LAYERS} consecutive "
            "steps; p50/p99 over the replays of replay time / 10",
            "p50_us": p50, "p99_us": float(np.percentile(times, 99)), "mean_us": float(times.mean()),
            "one_step_per_replay": {"replays": steps, "p50_us": float(np.percentile(single, 50)),
                                    "p99_us": float(np.percentile(single, 99)),
                                    "note": "one step per graph replay: adds the replay's launch overhead"},
            "local_rows": int(counts.sum()), "experts_touched": touched,
            "weight_bytes_touched": wbytes, "weight_GBps_at_p50": wbytes / (p50 * 1e-6) / 1e9,
            "hbm_roofline_frac": (wbytes / (HBM_PEAK_GBPS * 1e9)) / (p50 * 1e-6)}
    if cpu_base:
        res["cpu_baseline"] = cpu_base
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--config", default="default", choices=["default", "2", "3", "4", "4i8", "5", "5i8", "sweep", "sweepi8", "peaks", "all"],
                    help="default: the config-2 headline line plus brief config 3/4/5 results; 2: config 2 only; "
                         "3/4/5: only that config; 5i8: config 5 with int8 W8A8 weights; peaks: measured copy/read bandwidth and vendor GEMM rates; sweep: fp8 grouped-GEMM M-sweep; sweepi8: the same with int8 W8A8; all: default + sweep")
    ap.add_argument("--sweep-m", type=int, default=0, help="--config sweep: only this M")
    ap.add_argument("--calib-copy", action="store_true",
                    help="only run 20 device copies of 1 GiB (known bytes) to calibrate HBM counters")
    args = ap.parse_args()
    if args.calib_copy:
        a = torch.empty(1 << 30, dtype=torch.uint8, device="cuda:0")
        b = torch.empty_like(a)
        for _ in range(20):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"calib_copy_bytes_each": 1 << 30, "copies": 20}))
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (one EP rank, no collectives); --gpus {args.gpus} "
              "is not supported", file=sys.stderr)
        sys.exit(2)

    import umdk_amd  # noqa: F401
    from umdk_amd.plan import MoePrefillPlan

    cfg3 = lambda st, wu: run_layer("config3: Mixtral-8x7B grouped SwiGLU FFN, bf16", 8192, 4096, 8, 2, 8, 14336,
                                    "bf16", st, wu, args.seed, None)
    cfg4 = lambda st, wu, dt="fp8", cpu=False: run_layer(
        f"config4: DeepSeek-V3 one-rank layer (32 of 256 experts, Zipf 1.1), {dt}", 4096, 7168, 256, 8, 32, 2048,
        dt, st, wu, args.seed, "zipf", cpu)
    if args.config == "peaks":
        print(json.dumps({"config": "peaks", "result": measured_peaks()}))
        return
    if args.config in ("3", "4", "4i8", "5", "5i8", "sweep", "sweepi8"):
        r = {"3": lambda: cfg3(args.steps, args.warmup), "4": lambda: cfg4(args.steps, args.warmup, cpu=not args.no_cpu),
             "4i8": lambda: cfg4(args.steps, args.warmup, "int8"),
             "5": lambda: run_decode(max(args.steps, 1000), args.seed, cpu=not args.no_cpu),
             "5i8": lambda: run_decode(max(args.steps, 1000), args.seed, "int8"),
             "sweep": lambda: gemm_sweep(args.steps, args.warmup, args.seed,
                                         (args.sweep_m,) if args.sweep_m else (4096, 8192, 16384, 32768, 65536)),
             "sweepi8": lambda: gemm_sweep(args.steps, args.warmup, args.seed,
                                           (args.sweep_m,) if args.sweep_m else (4096, 8192, 16384, 32768, 65536),
                                           "int8"),
             }[args.config]()
        print(json.dumps({"config": args.config, "result": r}))
        return

    T, H, E, K = 4096, 7168, 256, 8
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(args.seed)
    x = torch.randn(T, H, generator=g).bfloat16().to(dev)
    logits = torch.randn(T, E, generator=g).to(dev)
    bias = (torch.randn(E, generator=g) * 0.5).to(dev)
    y = torch.randn(T * K, H, generator=g).bfloat16().to(dev)   # identity-expert outputs, dispatch order
    plan = MoePrefillPlan(T, H, E, K, quant_mode=3, device=dev)
    stream = torch.cuda.current_stream(dev)

    # Every timing below replays a HIP graph of the work: eager launches through the Python binding cost more
    # host time per step than the GPU needs, which would leave the GPU idle between launches.
    def step():
        # the step as the plan runs it: route + layout + count exchange + dispatch in three launches
        # (camhipMoePrefillDispatch), then the combine gather on the dispatch's row map
        plan.dispatch_step(logits, x, bias)
        plan.combine_step(y)

    def step_ops():
        # the same step through the reference-shaped calls (eight launches)
        plan.route(logits, bias)
        plan.layout()
        plan.dispatch(x)
        plan.combine(y)

    n = args.steps
    ms = graph_time(step, n, args.warmup, stream)
    rows = int(plan.recv_count[-1].item())
    assert rows == T * K
    ds_ms = graph_time(lambda: plan.dispatch_step(logits, x, bias), n, args.warmup, stream)
    c_ms = graph_time(lambda: plan.combine_step(y), n, args.warmup, stream)
    ms_ops = graph_time(step_ops, n, args.warmup, stream)
    d_ms = graph_time(lambda: plan.dispatch(x), n, args.warmup, stream)      # the dispatch launch alone
    cold_ms, single_ms = cold_time(step, 20, stream)
    c_ops_ms = graph_time(lambda: plan.combine(y), n, args.warmup, stream)   # scatter + gather
    db, cb = dispatch_bytes(T, H, K), combine_bytes(T, H, K)
    comb_gbps = cb / (c_ms * 1e-3) / 1e9
    disp_gbps = db / (d_ms * 1e-3) / 1e9
    dc_gbps = (db + cb) / ((d_ms + c_ms) * 1e-3) / 1e9

    result = {
        "metric": METRIC,
        "value": T / (ms * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": n,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3+bf16",
        "data": "synthetic (seeded torch.Generator; N(0,1) activations and logits, N(0,0.5) expert bias)",
        "config": {"workload": "config2: DSV3 one-rank dispatch+combine (route, layout, fp8 1x128 dispatch, "
                               "identity experts, bf16 combine)", "tokens": T, "hidden": H, "experts": E,
                   "topk": K, "parallelism": "ep1 (one GPU, no collectives)"},
        "roofline": {"bound": "hbm", "achieved": comb_gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": comb_gbps / HBM_PEAK_GBPS,
                     "traffic": measured_traffic(["combine_gather_kernel"]),
                     "traffic_source": "profiles/dispatch_combine_cfg2_hbm_counters.md (rocprofv3 FETCH_SIZE x2.0 + "
                                       "WRITE_SIZE x1.0, same workload)",
                     "kernel": "combine gather (the step's combine launch)", "algorithmic_bytes": cb},
        "step_launches": "camhipMoePrefillDispatch (route+histogram, scan+count exchange, dispatch) + "
                         "camhipMoePrefillCombine (gather)",
        "dispatch_step_ms": ds_ms,
        "cold_caches": {"ms_per_step_median": cold_ms, "tokens_per_s": T / (cold_ms * 1e-3),
                        "same_without_flush_ms": single_ms,
                        "method": "one step per graph replay, 20 replays, each after reading 512 MiB (L2 and MALL "
                                  "flushed), per-replay HIP events, median; the same replays without the flush "
                                  "beside it"},
        "dispatch": {"ms": d_ms, "GBps": disp_gbps, "frac": disp_gbps / HBM_PEAK_GBPS, "algorithmic_bytes": db,
                     "timed_in": "the reference-op chain (the dispatch launch alone)"},
        "combine": {"ms": c_ms, "GBps": comb_gbps, "frac": comb_gbps / HBM_PEAK_GBPS},
        "dispatch_combine_GBps": dc_gbps,
        "dispatch_combine_frac": dc_gbps / HBM_PEAK_GBPS,
        "reference_op_chain": {"ms_per_step": ms_ops, "tokens_per_s": T / (ms_ops * 1e-3), "dispatch_ms": d_ms,
                               "combine_ms": c_ops_ms,
                               "calls": "camhipMoeRoute, camhipDispatchLayout, camhipNotifyDispatch, "
                                        "camhipMoeDispatchNormal, camhipMoeCombineNormal (8 launches)"},
    }
    del plan, x, y
    torch.cuda.empty_cache()
    if args.config in ("default", "all"):
        # the decode step first: its weight stream is measured on weights allocated before the larger
        # configurations have cycled memory through the caching allocator, as a server allocates them at start-up
        result["config5"] = run_decode(1000, args.seed, cpu=not args.no_cpu)
        torch.cuda.empty_cache()
        result["config5_int8"] = run_decode(1000, args.seed, "int8")
        torch.cuda.empty_cache()
        result["config3"] = cfg3(10, 3)
        torch.cuda.empty_cache()
        result["config4"] = cfg4(20, 5, cpu=not args.no_cpu)
        result["config4_int8"] = cfg4(20, 5, "int8")
        torch.cuda.empty_cache()
    if args.config in ("default", "all"):
        result["measured_peaks"] = measured_peaks()
        torch.cuda.empty_cache()
    if args.config == "all":
        result["fp8_gemm_sweep"] = gemm_sweep(10, 3, args.seed)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(T, H, E, K, args.seed)
        if args.config in ("default", "all"):
            c3 = result["config3"]
            c3["cpu_baseline"] = cpu_layer_baseline(None, "bf16", 8192, 4096, 14336, c3["local_rows_M"], args.seed)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
