"""Per-tile timeline of the grouped GEMMs of one expert layer (a diagnostic, not part of the op surface).

    python -m umdk_amd.build --timeline         # the instrumented library (-DCAM_GMM_TIMELINE)
    python -m umdk_amd.timeline --config 4      # run from the repository root, on a GPU

Runs bench.py's layer (config 4: DeepSeek-V3 rank, 32 of 256 experts, Zipf 1.1 popularity, fp8; config 5: the
decode step's 128 tokens) once through the prefill step, then each GEMM launch once more with the instrumented
library, and prints per tile class the tile count and durations, the span of the launch against its CU time
over 256 CUs, and the gaps a block spends between tile classes.  Every block of the instrumented kernels stamps
the 100 MHz constant clock at each tile's start and end; camhipDebugGmmTimeline copies the records out.
"""
import argparse
import ctypes
import os
import sys

import numpy as np

from . import _lib
from .build import TIMELINE_LIB

SLOTS, BLOCKS = 128, 1024  # records per block, blocks recorded (gmm.hip: G_TL_SLOTS, G_TL_BLOCKS)


def _records(lib):
    buf = np.zeros((BLOCKS * SLOTS, 3), dtype=np.uint64)
    n = lib.camhipDebugGmmTimeline(buf.ctypes.data, buf.nbytes)
    if n <= 0:
        raise RuntimeError("camhipDebugGmmTimeline failed")
    r = buf[buf[:, 1] != 0]
    info = r[:, 0]
    t0 = r[:, 1].astype(np.int64)
    t1 = r[:, 2].astype(np.int64)
    base = t0.min()
    return dict(block=(info >> 48).astype(int), bm=((info >> 36) & 0xFFF).astype(int),
                expert=((info >> 20) & 0xFFF).astype(int), start=(t0 - base) / 100.0, end=(t1 - base) / 100.0)


def summarise(name, rec, event_us, cus=256):
    s, f, bm, blk = rec["start"], rec["end"], rec["bm"], rec["block"]
    busy = float((f - s).sum())
    print(f"{name}: HIP-event {event_us:.1f} us, {len(s)} tiles, span {f.max():.1f} us, CU time {busy:.0f} us "
          f"= {busy / cus:.1f} us over {cus} CUs")
    for c in sorted(set(bm.tolist()), reverse=True):
        m = bm == c
        d = f[m] - s[m]
        print(f"  {c:3d}-row tiles: {int(m.sum()):5d}, {d.mean():.1f} us each ({d.min():.1f}-{d.max():.1f}), "
              f"started {s[m].min():.1f}-{s[m].max():.1f}, ended {f[m].min():.1f}-{f[m].max():.1f}")
    gaps, ends = [], []
    for b in np.unique(blk):
        m = blk == b
        o = np.argsort(s[m])
        ss, ff, cc = s[m][o], f[m][o], bm[m][o]
        ends.append(ff.max())
        gaps += [ss[i] - ff[i - 1] for i in range(1, len(ss)) if cc[i] != cc[i - 1]]
    ends = np.array(ends)
    print(f"  blocks {len(ends)}: last tile ends {ends.min():.1f} (min) / {np.median(ends):.1f} (median) / "
          f"{ends.max():.1f} (max) us")
    if gaps:
        print(f"  between tile classes: {len(gaps)} switches, {np.mean(gaps):.1f} us each ({np.min(gaps):.1f}-"
              f"{np.max(gaps):.1f})")


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--config", choices=["4", "5"], default="4")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--lib", default=TIMELINE_LIB, help="the instrumented libcamhip.so")
    args = ap.parse_args(argv)
    if not os.path.exists(args.lib):
        raise SystemExit(f"{args.lib} is not built: python -m umdk_amd.build --timeline")
    _lib.LIB_PATH = args.lib  # before the first call loads a library
    import torch
    sys.path.insert(0, os.getcwd())
    import bench
    from .plan import MoeLayerPlan

    dev = torch.device("cuda:0")
    T = 4096 if args.config == "4" else 128
    H, E, K, L, I = 7168, 256, 8, 32, 2048
    g = torch.Generator().manual_seed(args.seed)
    x = torch.randn(T, H, generator=g).bfloat16().to(dev)
    logits = torch.randn(T, E, generator=g).to(dev)
    bias = bench.zipf_bias(E, 1.1, args.seed).to(dev) if args.config == "4" else None
    w1, s1, w2, s2 = bench.make_weights(L, H, I, "fp8", dev, args.seed)
    plan = MoeLayerPlan(T, H, E, K, L, I, dtype="fp8", device=dev)
    plan.dispatch_step(logits, x, bias)
    torch.cuda.synchronize()
    counts = plan.recv_tokens_per_expert[:L].cpu().tolist()
    print(f"config {args.config}, seed {args.seed}: rows per local expert {counts}")
    lib = _lib.lib()
    lib.camhipDebugGmmTimeline.restype = ctypes.c_int
    lib.camhipDebugGmmTimeline.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    for name, fn in (("GMM1 + SwiGLU", lambda: plan.gmm1(w1, s1)), ("GMM2", lambda: plan.gmm2(w2, s2))):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        _records(lib)  # clears the warm-up launches' records
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        summarise(name, _records(lib), a.elapsed_time(b) * 1e3)


if __name__ == "__main__":
    main()
