"""Benchmark of the CAM MoE hot path on one MI355X.

Default workload ("dispatch/combine at the DeepSeek-V3
one-rank shape"): T=4096 tokens, H=7168, E=256 experts, top-8, router logits
~N(0,1) plus a per-expert bias ~N(0,0.5); one step = route -> layout -> count
exchange -> fp8 1x128 dispatch -> combine of identity-expert bf16 rows.
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
        if time.perf_counter() - t0 > 10.0 or reps >= 3:
            break
    dt = (time.perf_counter() - t0) / reps
    return {"value": T / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"full config-2 step (T={T}, H={H}, E={E}, K={K}) x{reps} on the C oracle, 1 thread; "
                      f"{dt * 1e3:.0f} ms/step"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
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

    T, H, E, K = 4096, 7168, 256, 8
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(args.seed)
    x = torch.randn(T, H, generator=g).bfloat16().to(dev)
    logits = torch.randn(T, E, generator=g).to(dev)
    bias = (torch.randn(E, generator=g) * 0.5).to(dev)
    y = torch.randn(T * K, H, generator=g).bfloat16().to(dev)   # identity-expert outputs, dispatch order
    plan = MoePrefillPlan(T, H, E, K, quant_mode=3, device=dev)
    stream = torch.cuda.current_stream(dev)

    n = args.steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(n)]

    def step(i=None):
        plan.route(logits, bias)
        plan.layout()
        if i is not None:
            ev[i][0].record(stream)
        plan.dispatch(x)
        if i is not None:
            ev[i][1].record(stream)
        plan.combine(y)
        if i is not None:
            ev[i][2].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    t_start.record(stream)
    for i in range(n):
        step(i)
    t_end.record(stream)
    torch.cuda.synchronize()
    ms = t_start.elapsed_time(t_end) / n
    d_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / n
    c_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / n
    db, cb = dispatch_bytes(T, H, K), combine_bytes(T, H, K)
    comb_gbps = cb / (c_ms * 1e-3) / 1e9
    disp_gbps = db / (d_ms * 1e-3) / 1e9
    dc_gbps = (db + cb) / ((d_ms + c_ms) * 1e-3) / 1e9
    rows = int(plan.total_recv.item())
    assert rows == T * K

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
                     "frac": comb_gbps / HBM_PEAK_GBPS, "traffic": None, "kernel": "combine (scatter+gather)",
                     "algorithmic_bytes": cb},
        "dispatch": {"ms": d_ms, "GBps": disp_gbps, "frac": disp_gbps / HBM_PEAK_GBPS, "algorithmic_bytes": db},
        "combine": {"ms": c_ms, "GBps": comb_gbps, "frac": comb_gbps / HBM_PEAK_GBPS},
        "dispatch_combine_GBps": dc_gbps,
        "dispatch_combine_frac": dc_gbps / HBM_PEAK_GBPS,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(T, H, E, K, args.seed)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
