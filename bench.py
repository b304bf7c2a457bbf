"""Benchmark of the MI355X Qwen3.5 GGUF hot path.

Workloads:
  gemv   BASELINE config 2: dequant-GEMV sweep (Q8_0/Q4_K, M in {1,4,16,32}),
         bf16 activations with the RMSNorm prologue; weights rotate across
         distinct buffers totalling > 2x the 256 MB Infinity Cache so every
         launch streams from HBM.  Timed with HIP events on the launch stream.

The default workload is the one BASELINE.json's metric is quoted on.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(kind, N, K, M):
    bpe = 34 / 32 if kind == 8 else 144 / 256
    return N * K * bpe + M * K * 2 + M * N * 4


def register_copies(kern, kind, N, K, rng):
    """Distinct device copies totalling > 2.2x the Infinity Cache."""
    from zerogravity_amd import synth
    w = synth.random_matrix(rng, kind, N, K)
    copies = int(min(512, max(2, np.ceil(2.2 * MALL_BYTES / w.nbytes))))
    return [kern.register(4242, f"bench.{kind}.{N}.{K}.{i}", kind, K, N, w) for i in range(copies)]


def bench_gemv(kern, torch, handles, kind, N, K, M, steps, warmup, rng):
    from zerogravity_amd import _lib as L
    from zerogravity_amd import synth
    copies = len(handles)
    xf, xb = synth.bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    gamma = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    x_d = torch.from_numpy(xb.view(np.int16)).cuda()
    g_d = torch.from_numpy(gamma).cuda()
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    assert s.cuda_stream != 0, "launch and event stream must be a real stream"
    lib, ctx = L.lib(), kern.ctx
    nbytes = lib.zg_act_prepared_bytes(handles[0].h, M)
    prep = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    ctx.check(lib.zg_act_prepare_device(ctx.h, handles[0].h, x_d.data_ptr(), L.BF16, M, g_d.data_ptr(), 1e-6,
                                        prep.data_ptr(), nbytes, s.cuda_stream))

    def launch(i):
        h = handles[i % copies]
        ctx.check(lib.zg_gemv_prepared_device(ctx.h, h.h, M, prep.data_ptr(), y.data_ptr(), s.cuda_stream))

    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for i in range(steps):
        launch(i)
    e1.record(s)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    byts = gemv_bytes(kind, N, K, M)
    return us, byts / us / 1e3  # GB/s


def cpu_gemv_baseline(kind, N, K, seconds=10.0):
    """Oracle GEMV (OpenMP over rows, all host cores) on a bounded row sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import zg_oracle as O
    from zerogravity_amd import synth
    rng = np.random.default_rng(1)
    rows = min(N, 32768)
    w = synth.random_matrix(rng, kind, rows, K)
    x = rng.standard_normal(K).astype(np.float32)
    threads = os.cpu_count() or 1
    O.matvec(kind, w.reshape(-1), rows, K, x, threads)
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds:
        O.matvec(kind, w.reshape(-1), rows, K, x, threads)
        n += 1
    dt = (time.perf_counter() - t0) / n
    byts = rows * K * (34 / 32 if kind == 8 else 144 / 256) + K * 4 + rows * 4
    return byts / dt / 1e9, threads, f"{rows}x{K} rows of the {N}x{K} matrix, {n} passes"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="gemv", choices=["gemv"])
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(data-parallel sharding is described in DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch
    from zerogravity_amd import regions as R
    kern = R.HipMatVecKernel(0)
    torch.cuda.set_stream(torch.cuda.Stream())  # default priority, non-null
    rng = np.random.default_rng(2026)
    results = []
    shapes = [(3584, 1024), (1024, 3584), (6144, 2048), (2048, 6144), (151936, 2048)]
    for kind in (12, 8):
        for (N, K) in shapes:
            handles = register_copies(kern, kind, N, K, rng)
            for M in (1, 4, 16, 32):
                us, gbs = bench_gemv(kern, torch, handles, kind, N, K, M, args.steps, args.warmup, rng)
                name = "Q4_K" if kind == 12 else "Q8_0"
                log(f"gemv {name} N={N:6d} K={K:5d} M={M:2d}: {us:9.2f} us  {gbs:8.1f} GB/s  "
                    f"({gbs / HBM_PEAK_GBS:.1%} of HBM)")
                results.append(dict(kind=name, N=N, K=K, M=M, us=us, gbs=gbs))
            del handles
            kern.release_source(4242)
    head = next(r for r in results if r["kind"] == "Q4_K" and r["N"] == 151936 and r["M"] == 1)
    line = {
        "metric": "dequant-GEMV achieved HBM GB/s (Q4_K 151936x2048, M=1, RMSNorm-prepared bf16 activation)",
        "value": round(head["gbs"], 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": head["us"] / 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k x f32", "data": "synthetic (seeded random GGUF blocks)",
        "config": {"workload": "BASELINE config 2: GEMV sweep", "sweep": results},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 4), "traffic": None},
    }
    if not args.no_cpu:
        v, cores, sample = cpu_gemv_baseline(12, 151936, 2048, args.cpu_seconds)
        line["cpu_baseline"] = {"value": round(v, 2), "unit": "GB/s", "cores": cores, "kind": "port",
                                "sample": sample}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
