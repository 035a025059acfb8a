"""Benchmark of the MI355X GPT-2 INT8 hot path (BASELINE.json metric:
"GPT-2 INT8 decode tokens/sec at b=1/b=32; W8A16 GEMV achieved HBM GB/s").

Modes
  gemv (default until the runtime lands): BASELINE configs[1] W8A16 linear at
       decode sizes, M in {1, 8} x (768->3072, 3072->768), fused bias+GELU.  A
       "step" is one pass of the four GEMV shapes over one rotation of >= 600 MB
       of distinct weight sets (more than the 256 MB Infinity Cache), timed with
       HIP events on the launch stream.
Prints one JSON line (the driver's contract) with a `roofline` object for the
dominant kernel and a `cpu_baseline` object (rank 0, N=1).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 640 << 20


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--mode", default="gemv", choices=["gemv"])
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    return p.parse_args()


def gemv_bytes(m, k, n):
    # A fp16, q int8, scales fp32, bias fp16, y fp16
    return 2 * m * k + k * n + 4 * n + 2 * n + 2 * m * n


def run_gemv(args):
    import torch
    from tinyinfer_amd.native_ops import NativeOps
    ops = NativeOps()
    lib = ops.lib
    fn = lib.ti_amd_gemm_i8_fused
    fn.argtypes = [C.c_void_p] * 6 + [C.c_int] * 4 + [C.c_size_t, C.c_int]
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    shapes = [(1, 768, 3072), (1, 3072, 768), (8, 768, 3072), (8, 3072, 768)]
    g = torch.Generator(device=dev)
    g.manual_seed(20261101)
    wbytes = 768 * 3072
    nsets = max(1, ROTATE_BYTES // wbytes)
    q = torch.randint(-127, 128, (nsets, 768 * 3072), dtype=torch.int8, device=dev, generator=g)
    scales = (torch.rand((nsets, 3072), device=dev, generator=g) * 9e-3 + 1e-3).half().float()
    bias = (torch.randn((nsets, 3072), device=dev, generator=g) * 0.02).half()
    a = torch.randn((8, 3072), device=dev, generator=g).half()
    y = torch.empty((8, 3072), device=dev, dtype=torch.float16)

    def launch(m, k, n, i):
        st = fn(a.data_ptr(), q[i].data_ptr(), scales[i].data_ptr(), bias[i].data_ptr(), y.data_ptr(), None,
                m, n, k, 1, stream.cuda_stream, 0)
        if st:
            raise RuntimeError(lib.ti_v2_last_error().decode())

    def step():
        for (m, k, n) in shapes:
            for i in range(nsets):
                launch(m, k, n, i)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    per_shape = {}
    for (m, k, n) in shapes:
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        for _ in range(max(1, args.steps // 4)):
            for i in range(nsets):
                launch(m, k, n, i)
        ev1.record(stream)
        torch.cuda.synchronize()
        launches = max(1, args.steps // 4) * nsets
        us = ev0.elapsed_time(ev1) * 1e3 / launches
        per_shape[f"M{m}_K{k}_N{n}"] = {"us_per_launch": us, "GBps": gemv_bytes(m, k, n) / us / 1e3}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    total_bytes = args.steps * nsets * sum(gemv_bytes(*s) for s in shapes)
    value = total_bytes / elapsed / 1e9
    dom = per_shape["M1_K3072_N768"]
    return {
        "metric": "W8A16 GEMV achieved HBM GB/s (GPT-2 INT8 decode tokens/sec pending the runtime)",
        "value": value, "unit": "GB/s", "ms_per_step": elapsed / args.steps * 1e3,
        "dtype": "int8xfp16->fp32acc",
        "config": {"workload": "configs[1] W8A16 GEMV M in {1,8} x (768->3072, 3072->768), fused bias+GELU, "
                               f"{nsets} rotating weight sets ({nsets * wbytes >> 20} MiB)"},
        "gemv": per_shape,
        "roofline": {"bound": "hbm", "kernel": "skinny_kernel<int8,MT=1> M=1 K=3072 N=768",
                     "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dom["GBps"] / HBM_PEAK_GBS, "traffic": None},
    }


def cpu_baseline_gemv(seconds):
    """The reference's CPU FP32 matmul_blocked (restated in the oracle) over
    dequantized weights at M=1, K=3072, N=768, timed on this host's cores."""
    import oracle
    rng = np.random.default_rng(1)
    k, n = 3072, 768
    w = oracle.f16_bits_to_f32(oracle.dequantize(rng.integers(-127, 128, (k, n)).astype(np.int8),
                                                 rng.uniform(1e-3, 1e-2, n).astype(np.float32)))
    a = rng.standard_normal((1, k)).astype(np.float32)
    oracle.matmul_blocked(a, w)
    calls, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.matmul_blocked(a, w)
        calls += 1
    dt = (time.perf_counter() - t0) / calls
    return {"value": gemv_bytes(1, k, n) / dt / 1e9, "unit": "GB/s", "cores": oracle.num_threads(),
            "kind": "port",
            "sample": f"{calls} calls of matmul_blocked (reference kernels/src/cpu/matmul.cpp) at M=1 K=3072 "
                      f"N=768 over dequantized fp32 weights, {seconds:.0f} s"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no "
              "multi-GPU path", file=sys.stderr)
        sys.exit(2)
    res = run_gemv(args)
    res["cpu_baseline"] = cpu_baseline_gemv(args.cpu_seconds)
    line = {"metric": res.pop("metric"), "value": res.pop("value"), "unit": res.pop("unit"), "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": res.pop("ms_per_step"),
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": res.pop("dtype"),
            "data": "synthetic", "config": res.pop("config")}
    line.update(res)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
