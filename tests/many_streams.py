"""A fresh process whose first library calls run on eight streams at once:
every split plan that finishes in its launch through the library's
per-hardware-queue pool (row-major GEMV, skinny and tiled GEMMs, the packed K-split
GEMV, the split panel GEMM, split-key decode attention, split-key causal
prefill attention), and the packed row-block GEMV beside them, is
enqueued on every stream with no synchronisation between them, three times
over, and each result must equal, bit for bit, the same call made alone on
one stream afterwards.  Streams map onto the hardware queues round-robin, so
calls overlap across queues (each queue claims its own pool slot, some of them
at the same moment) while calls on one queue run in order.

Run by tests/test_pool_many_streams_gpu.py as `python tests/many_streams.py`;
prints one JSON line and exits 0 when every check passes.
"""
import ctypes
import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from tinyinfer_amd import BACKEND_LIB  # noqa: E402

P, I = ctypes.c_void_p, ctypes.c_int
STREAMS = 8


def f16(a):
    return np.asarray(a, np.float16).view(np.uint16)


def gpu(a, dtype=None):
    x = torch.from_numpy(np.ascontiguousarray(a))
    return (x.view(dtype) if dtype is not None else x).cuda()


def main():
    assert torch.cuda.is_available()
    lib = ctypes.CDLL(str(BACKEND_LIB))
    lib.ti_v2_last_error.restype = ctypes.c_char_p
    lib.ti_v2_gemm_ex_i8.argtypes = [P] * 6 + [I] * 5 + [ctypes.c_size_t, I]
    lib.ti_amd_packed_w8_bytes.restype = ctypes.c_int64
    lib.ti_amd_packed_w8_bytes.argtypes = [I, I]
    lib.ti_amd_pack_w8.argtypes = [P, I, I, P, ctypes.c_size_t, I]
    lib.ti_amd_gemm_w8p_fused.argtypes = [P] * 6 + [I] * 4 + [ctypes.c_size_t, I]
    lib.ti_v2_attention_f16.argtypes = [P] * 7 + [I] * 7 + [ctypes.c_size_t, I]

    cases = []
    for kind, m, k, n in (("rowmajor", 1, 768, 3072), ("rowmajor", 8, 3072, 768), ("rowmajor", 24, 3072, 768),
                          ("rowmajor", 64, 768, 3072),
                          ("rowmajor", 512, 3072, 768), ("packed", 32, 3072, 768), ("packed", 64, 3072, 768),
                          ("packed", 512, 3072, 768)):
        rng = np.random.default_rng(m * 7 + k + n)
        a = f16(rng.standard_normal((m, k)) * 0.25)
        q, s = oracle.quantize(f16(rng.standard_normal((k, n)) * 0.25))
        bias = f16(rng.standard_normal(n) * 0.1)
        c = dict(kind=kind, m=m, k=k, n=n, a=gpu(a, torch.float16), q=gpu(q), s=gpu(s), bias=gpu(bias, torch.float16))
        if kind == "packed":
            # Packed once on the current stream before any other call.
            c["pk"] = torch.empty(lib.ti_amd_packed_w8_bytes(k, n), dtype=torch.uint8, device="cuda")
            assert lib.ti_amd_pack_w8(c["q"].data_ptr(), k, n, c["pk"].data_ptr(),
                                      torch.cuda.current_stream().cuda_stream, 0) == 0
        cases.append(c)
    rng = np.random.default_rng(4242)
    B, H, D = 8, 12, 64
    L = rng.integers(600, 1025, B)
    K = int(L.max())
    attn = dict(q=gpu(f16(rng.standard_normal((B, H, 1, D)) / 8), torch.float16),
                k=gpu(f16(rng.standard_normal((B, H, K, D)) / 8), torch.float16),
                v=gpu(f16(rng.standard_normal((B, H, K, D)) / 8), torch.float16),
                meta=[gpu(np.asarray(x, np.int32)) for x in ([1] * B, L, L - 1)])
    # Causal prefill over few query tiles: heavy tiles split their keys over
    # two workgroups merged through the prefill pool.
    PB, PH, PN = 1, 4, 1024
    pre = dict(q=gpu(f16(rng.standard_normal((PB, PH, PN, D)) * 0.5), torch.float16),
               k=gpu(f16(rng.standard_normal((PB, PH, PN, D)) * 0.5), torch.float16),
               v=gpu(f16(rng.standard_normal((PB, PH, PN, D))), torch.float16),
               ql=gpu(np.full(PB, PN, np.int32)), off=gpu(np.zeros(PB, np.int32)))
    torch.cuda.synchronize()

    def run_prefill(st):
        out = torch.empty((PB, PH, PN, D), dtype=torch.float16, device="cuda")
        r = lib.ti_v2_attention_f16(pre["q"].data_ptr(), pre["k"].data_ptr(), pre["v"].data_ptr(), out.data_ptr(),
                                    pre["ql"].data_ptr(), pre["ql"].data_ptr(), pre["off"].data_ptr(), PB, PH, PN, PN,
                                    D, 1, 0, st, 0)
        assert r == 0, lib.ti_v2_last_error()
        return out

    def run(c, st):
        y = torch.empty((c["m"], c["n"]), dtype=torch.float16, device="cuda")
        if c["kind"] == "rowmajor":
            r = lib.ti_v2_gemm_ex_i8(c["a"].data_ptr(), c["q"].data_ptr(), c["s"].data_ptr(), c["bias"].data_ptr(),
                                     y.data_ptr(), None, c["m"], c["n"], c["k"], 0, 0, st, 0)
        else:
            r = lib.ti_amd_gemm_w8p_fused(c["a"].data_ptr(), c["pk"].data_ptr(), c["s"].data_ptr(),
                                          c["bias"].data_ptr(), y.data_ptr(), None, c["m"], c["n"], c["k"], 1, st, 0)
        assert r == 0, lib.ti_v2_last_error()
        return y

    def run_attn(st):
        out = torch.empty((B, H, 1, D), dtype=torch.float16, device="cuda")
        r = lib.ti_v2_attention_f16(attn["q"].data_ptr(), attn["k"].data_ptr(), attn["v"].data_ptr(), out.data_ptr(),
                                    attn["meta"][0].data_ptr(), attn["meta"][1].data_ptr(),
                                    attn["meta"][2].data_ptr(), B, H, 1, K, D, 1, 0, st, 0)
        assert r == 0, lib.ti_v2_last_error()
        return out

    print(f"[streams] {len(cases)} GEMMs, split decode and prefill attention on {STREAMS} streams at once, 3 rounds",
          flush=True)
    streams = [torch.cuda.Stream() for _ in range(STREAMS)]
    got = []
    for rnd in range(3):
        outs = []
        for i, sm in enumerate(streams):
            with torch.cuda.stream(sm):
                # Each stream walks the cases from a different start.
                order = cases[i % len(cases):] + cases[:i % len(cases)]
                res = {id(c): run(c, sm.cuda_stream) for c in order}
                outs.append([res[id(c)] for c in cases] + [run_attn(sm.cuda_stream), run_prefill(sm.cuda_stream)])
        torch.cuda.synchronize()
        got.extend(outs)

    print("[streams] the same calls alone on one stream", flush=True)
    st = torch.cuda.current_stream().cuda_stream
    want = [run(c, st) for c in cases] + [run_attn(st), run_prefill(st)]
    torch.cuda.synchronize()
    bad = []
    for r, outs in enumerate(got):
        for j, (o, w) in enumerate(zip(outs, want)):
            if not torch.equal(o.view(torch.int16), w.view(torch.int16)):
                bad.append((r, j))
    assert not bad, f"results that differ from the lone call (stream round, case): {bad[:10]}"
    assert all(torch.isfinite(w.float()).all() for w in want)
    print(json.dumps({"ok": True, "streams": STREAMS, "calls": len(got) * len(want)}), flush=True)


if __name__ == "__main__":
    main()
