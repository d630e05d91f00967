"""Benchmark of the Q8_0 matmul path on one MI355X.

Default workload: the Q8_0 decode GEMV (W ~ N(0, 0.02) from seed 0, x ~ N(0,1),
both Q8_0) at 6144x2048 and 2048x6144, streamed over >= 64 rotated weight
copies so the working set (> 850 MB) exceeds the 256 MB Infinity Cache.
Prints one JSON line.  --gpus above 1 is refused: this build runs on one GPU.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "voxcpm-cpp_amd"))

HBM_PEAK_GBS = 8000.0


def q8_bytes(n, k):
    return n * k // 32 * 34


def gemv_bytes(n, k):
    # weights + quantized activation (K int8 + K/32 fp16) + fp32 output
    return q8_bytes(n, k) + k + k // 32 * 2 + 4 * n


def time_gemv(ctx, torch, vxm, N, K, copies, steps, warmup):
    import numpy as np

    w32 = vxm.host_randn(0, N * K, 0.0, 0.02).reshape(N, K)
    x = vxm.host_randn(0, K, 0.0, 1.0, offset=N * K).reshape(1, K)
    wq = vxm.host_quantize_q8_0(w32)
    ws = [ctx.upload_q8_0(wq, N, K) for _ in range(copies)]
    xd = torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")
    xq, xs = ctx.quantize_q8_0(xd, vxm.QUANT_X86)
    y = torch.empty((1, N), dtype=torch.float32, device="cuda:0")
    ctx.sync()
    L = vxm.lib()
    h = ctx.h
    args = [(w.h, vxm._ptr(xq), vxm._ptr(xs), vxm._ptr(y)) for w in ws]
    for _ in range(warmup):
        for a in args:
            L.vxm_mul_mat_q8_0_q8_0(h, a[0], a[1], a[2], 1, a[3])
    ctx.sync()
    st = ctx.torch_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(steps):
        for a in args:
            L.vxm_mul_mat_q8_0_q8_0(h, a[0], a[1], a[2], 1, a[3])
    e1.record(st)
    e1.synchronize()
    ms = e0.elapsed_time(e1)
    launches = steps * len(args)
    us = ms * 1000.0 / launches
    for w in ws:
        w.free()
    return us


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--copies", type=int, default=64)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import vxm

    ctx = vxm.Context(0)
    res = {}
    for (N, K) in ((6144, 2048), (2048, 6144)):
        us = time_gemv(ctx, torch, vxm, N, K, args.copies, args.steps, args.warmup)
        gbs = gemv_bytes(N, K) / (us * 1e-6) / 1e9
        res[f"{N}x{K}"] = {"us": us, "GBs": gbs, "hbm_frac": gbs / HBM_PEAK_GBS}
        print(f"# gemv {N}x{K}: {us:.3f} us/launch, {gbs:.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM)",
              file=sys.stderr, flush=True)
    ctx.close()
    main_key = "6144x2048"
    out = {
        "metric": "Q8_0 decode GEMV GB/s (% HBM peak) + us per 28-layer decode step, 1 GPU",
        "value": res[main_key]["GBs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res[main_key]["us"] / 1000.0,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "Q8_0 decode GEMV 6144x2048, 64 rotated weight copies"},
        "gemv": res,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
