"""Benchmark of the MI355X GPT-2 INT8 hot path.

BASELINE.json metric: "GPT-2 INT8 decode tokens/sec at b=1/b=32; W8A16 GEMV
achieved HBM GB/s".

* value: GPT-2 small INT8 (random-init N(0,0.02), seed 42) greedy decode
  tokens/s at batch 32 through libtinyinfer_llm's ti_llm_greedy_batch: 32
  seeded prompt ids per request, 64 new tokens, rate B*(new-1)/(t_last-t_first)
  as reference llm/evaluate.py:195 defines it.  One "step" is one such greedy
  batch; batch 1 is reported beside it.
* roofline: the W8A16 GEMV (skinny MFMA kernel, M=1, K=3072 -> N=768, fused
  bias+GELU) replayed back-to-back from a HIP graph over >= 600 MiB of distinct
  weight sets (beyond the 256 MiB Infinity Cache), timed with HIP events on the
  launch stream; algorithmic bytes per launch 2MK + KN + 4N + 2N + 2MN.
* cpu_baseline: the CPU restatement of the reference runtime (oracle/) decoding
  the same batch-32 workload for a bounded number of steps on this host.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 640 << 20
PROMPT, NEW = 32, 64


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--cpu-seconds", type=float, default=15.0)
    p.add_argument("--skip-cpu", action="store_true")
    return p.parse_args()


def gemv_bytes(m, k, n):
    return 2 * m * k + k * n + 4 * n + 2 * n + 2 * m * n


def artifact_path():
    from tinyinfer_amd.artifact import GPT2_SMALL, write_synthetic
    d = Path(tempfile.gettempdir()) / "tinyinfer_amd_gpt2_small_seed42"
    m = d / "manifest.json"
    if not m.exists():
        write_synthetic(d, GPT2_SMALL, seed=42)
    return m


def prompts(batch):
    rng = np.random.default_rng(42)
    return [rng.integers(0, 50257, PROMPT).tolist() for _ in range(batch)]


def decode_rate(res, batch):
    t_first = min(res["ttft_ms"])
    t_last = max(res["total_ms"])
    return batch * (NEW - 1) / ((t_last - t_first) / 1e3), t_last


def run_decode(model, batch, steps, warmup):
    ps = prompts(batch)
    for _ in range(warmup):
        model.reset_all()
        model.greedy(ps, NEW)
    rates, totals, ttfts = [], [], []
    t0 = time.perf_counter()
    for _ in range(steps):
        model.reset_all()
        res = model.greedy(ps, NEW)
        r, t_last = decode_rate(res, batch)
        rates.append(r)
        totals.append(t_last)
        ttfts.append(min(res["ttft_ms"]))
    elapsed = time.perf_counter() - t0
    return {"tokens_per_s": float(np.median(rates)), "samples": rates, "ms_per_step": elapsed / steps * 1e3,
            "ttft_ms_p50": float(np.median(ttfts)), "total_ms_p50": float(np.median(totals)),
            "tokens": res["tokens"]}


def run_gemv_roofline(reps=5):
    import torch
    from tinyinfer_amd.native_ops import NativeOps
    ops = NativeOps()
    fn = ops.lib.ti_amd_gemm_i8_fused
    fn.argtypes = [C.c_void_p] * 6 + [C.c_int] * 4 + [C.c_size_t, C.c_int]
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(20261101)
    out = {}
    stream = torch.cuda.Stream()
    for (m, k, n) in ((1, 3072, 768), (1, 768, 3072), (8, 3072, 768), (8, 768, 3072)):
        nsets = max(1, ROTATE_BYTES // (k * n))
        q = torch.randint(-127, 128, (nsets, k * n), dtype=torch.int8, device=dev, generator=g)
        scales = (torch.rand((nsets, n), device=dev, generator=g) * 9e-3 + 1e-3).half().float()
        bias = (torch.randn((nsets, n), device=dev, generator=g) * 0.02).half()
        a = torch.randn((m, k), device=dev, generator=g).half()
        y = torch.empty((m, n), device=dev, dtype=torch.float16)

        def launch(i):
            st = fn(a.data_ptr(), q[i].data_ptr(), scales[i].data_ptr(), bias[i].data_ptr(), y.data_ptr(), None,
                    m, n, k, 1, stream.cuda_stream, 0)
            if st:
                raise RuntimeError(ops.lib.ti_v2_last_error().decode())

        with torch.cuda.stream(stream):
            launch(0)  # creates the library's split-K scratch for this stream
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(nsets):
                launch(i)
        with torch.cuda.stream(stream):
            graph.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                graph.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * nsets)
        out[f"M{m}_K{k}_N{n}"] = {"us_per_launch": us, "GBps": gemv_bytes(m, k, n) / us / 1e3,
                                  "weight_sets": int(nsets), "rotated_MiB": int(nsets * k * n >> 20)}
        del graph, q, scales, bias
        torch.cuda.empty_cache()
    return out


def cpu_baseline_decode(manifest, seconds):
    """The oracle's CPU GPT-2 (restating reference llm/src/runtime.cu) on the batch-32
    workload: one prefill of 32 x 32 tokens, then single-token steps until the time
    budget is spent; tokens/s over the decode steps."""
    import oracle
    from tinyinfer_amd.artifact import load_tensors
    man, tensors = load_tensors(manifest)
    cpu = oracle.Gpt2(tensors, man["architecture"], slots=32, capacity=PROMPT + NEW)
    ps = prompts(32)
    _, nxt = cpu.forward(list(range(32)), ps, logits=False)
    steps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds and steps < NEW - 1:
        _, nxt = cpu.forward(list(range(32)), [[int(t)] for t in nxt], logits=False)
        steps += 1
    dt = time.perf_counter() - t0
    cpu.close()
    return {"value": 32 * steps / dt, "unit": "tokens/s", "cores": oracle.num_threads(), "kind": "port",
            "sample": f"GPT-2 small INT8 batch 32: prefill of 32x32 tokens then {steps} decode steps "
                      f"({dt:.1f} s) through the oracle's C++/OpenMP restatement of reference llm/src/runtime.cu"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)
    import torch
    from tinyinfer_amd import LLM_LIB, require
    from tinyinfer_amd.runtime import NativeModel
    manifest = artifact_path()
    with NativeModel(require(LLM_LIB), manifest, max_batch=32, cache_slots=32, capacity=PROMPT + NEW) as model:
        torch.cuda.synchronize()
        b1 = run_decode(model, 1, max(2, args.steps // 2), 1)
        torch.cuda.synchronize()
        b32 = run_decode(model, 32, args.steps, args.warmup)
        torch.cuda.synchronize()
    gemv = run_gemv_roofline()
    dom = gemv["M1_K3072_N768"]
    line = {
        "metric": "GPT-2 INT8 decode tokens/sec (b=32; b=1 in decode_b1); W8A16 GEMV achieved HBM GB/s in roofline",
        "value": b32["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": b32["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8 weights x fp16 activations, fp32 accumulate",
        "data": "synthetic (random-init N(0,0.02) GPT-2 small, seed 42; seeded prompt ids)",
        "config": {"workload": f"configs[0] GPT-2 small INT8 greedy, batch 32, prompt {PROMPT}, {NEW} new tokens",
                   "global_batch": 32, "seq_len": PROMPT + NEW, "parallelism": "single GPU"},
        "decode_b32": {k: v for k, v in b32.items() if k != "tokens"},
        "decode_b1": {k: v for k, v in b1.items() if k != "tokens"},
        "gemv": gemv,
        "roofline": {"bound": "hbm", "kernel": "skinny_kernel<int8,MT=1> + split-K epilogue, M=1 K=3072 N=768",
                     "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": dom["GBps"] / HBM_PEAK_GBS, "traffic": None},
    }
    if not args.skip_cpu:
        line["cpu_baseline"] = cpu_baseline_decode(manifest, args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
