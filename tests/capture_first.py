"""A fresh process whose first calls into libtinyinfer_backend.so happen under
HIP graph capture (torch.cuda.graph on its own capture stream): the W8A16
GEMM through NativeOps.gemm_int8 at M in {1, 8, 64, 512} x both configs[1]
shapes, configs 0 (fused) and 6 (caller workspace); ti_amd_pack_w8 then
ti_amd_gemm_w8p_fused (bias + GELU) over the packed weights at shapes that
take each packed kernel (M=1 part-block GEMV, M=16 / 32 K-split GEMV, M=64
row-block GEMV, M=512 split panel GEMM); and
ti_v2_attention_f16 at the configs[3] shape (B=32, H=12, D=64, ragged
U[128,1024]).  Neither may
allocate (the reference ABI's contract, backend/include/tinyinfer_backend_v2.h:13),
so capture must succeed with no call made before it.

Then: every replay (with eager torch work and synchronisations between them,
and one replay running beside eager calls of the same operations on another
stream) equals the first replay bit for bit; eager calls give the same bits;
and the results match the CPU oracle (linear rtol 1e-2 / atol 2e-2;
configs[3] attention within 1e-4 absolute, its signal scale).

Run by tests/test_capture_first_gpu.py as `python tests/capture_first.py`;
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
from tinyinfer_amd.native_ops import NativeOps  # noqa: E402


def f16(a):
    return np.asarray(a, np.float16).view(np.uint16)


def gpu(a, dtype=None):
    x = torch.from_numpy(np.ascontiguousarray(a))
    return (x.view(dtype) if dtype is not None else x).cuda()


def say(*args):
    print("[capture]", *args, flush=True)


def main():
    assert torch.cuda.is_available()
    ops = NativeOps()  # loads the library and reads its version and catalog (host calls only)
    lib = ops.lib
    attn = lib.ti_v2_attention_f16

    gemms = []
    for m in (1, 8, 64, 512):
        for n, k in ((3072, 768), (768, 3072)):
            for config in (0, 6):
                rng = np.random.default_rng(1000 * m + n + k + config)
                a = f16(rng.standard_normal((m, k)) * 0.25)
                w = f16(rng.standard_normal((k, n)) * 0.25)
                bias = f16(rng.standard_normal(n) * 0.1)
                q, s = oracle.quantize(w)
                out32 = config == 6  # the workspace configs also check the fp32 output
                gemms.append(dict(m=m, n=n, k=k, config=config, out32=out32, a=a, q=q, s=s, bias=bias,
                                  dev=(gpu(a, torch.float16), gpu(q), gpu(s), gpu(bias, torch.float16))))

    lib.ti_amd_packed_w8_bytes.restype = ctypes.c_int64
    lib.ti_amd_packed_w8_bytes.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.ti_amd_pack_w8.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t,
                                   ctypes.c_int]
    lib.ti_amd_gemm_w8p_fused.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 4 + [ctypes.c_size_t, ctypes.c_int]
    packed = []
    for m, k, n in ((1, 3072, 768), (16, 3072, 768), (32, 3072, 768), (64, 3072, 768), (64, 768, 3072),
                    (512, 3072, 768)):
        rng = np.random.default_rng(7000 + m + k)
        a = f16(rng.standard_normal((m, k)) * 0.25)
        w = f16(rng.standard_normal((k, n)) * 0.25)
        bias = f16(rng.standard_normal(n) * 0.1)
        q, s = oracle.quantize(w)
        nbytes = lib.ti_amd_packed_w8_bytes(k, n)
        packed.append(dict(m=m, n=n, k=k, a=a, q=q, s=s, bias=bias,
                           dev=(gpu(a, torch.float16), gpu(q), gpu(s), gpu(bias, torch.float16)),
                           pk=[torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(2)]))

    rng = np.random.default_rng(20261101)
    B, H, D = 32, 12, 64
    L = rng.integers(128, 1025, B)
    K = int(L.max())
    aq = f16(rng.standard_normal((B, H, 1, D)) / 8)
    ak = f16(rng.standard_normal((B, H, K, D)) / 8)
    av = f16(rng.standard_normal((B, H, K, D)) / 8)
    meta = [gpu(np.asarray(x, np.int32)) for x in ([1] * B, L, L - 1)]
    tq, tk, tv = gpu(aq, torch.float16), gpu(ak, torch.float16), gpu(av, torch.float16)
    torch.cuda.synchronize()

    def gemm_call(c):
        a, q, s, bias = c["dev"]
        return ops.gemm_int8(a, q, s, bias=bias, config=c["config"],
                             output_dtype=torch.float32 if c["out32"] else None)

    def packed_call(c, which):
        # Pack (a kernel on the stream), then the GEMM over the packed copy.
        a, q, s, bias = c["dev"]
        pk = c["pk"][which]
        st = torch.cuda.current_stream().cuda_stream
        assert lib.ti_amd_pack_w8(q.data_ptr(), c["k"], c["n"], pk.data_ptr(), st, 0) == 0, lib.ti_v2_last_error()
        y = torch.empty((c["m"], c["n"]), dtype=torch.float16, device="cuda")
        assert lib.ti_amd_gemm_w8p_fused(a.data_ptr(), pk.data_ptr(), s.data_ptr(), bias.data_ptr(), y.data_ptr(),
                                         None, c["m"], c["n"], c["k"], 1, st, 0) == 0, lib.ti_v2_last_error()
        return y

    def attn_call(out):
        st = attn(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), out.data_ptr(), meta[0].data_ptr(),
                  meta[1].data_ptr(), meta[2].data_ptr(), B, H, 1, K, D, 1, 0,
                  torch.cuda.current_stream().cuda_stream, 0)
        assert st == 0, lib.ti_v2_last_error()

    say("capturing", len(gemms), "GEMMs,", len(packed), "packed GEMMs and the configs[3] attention as the "
        "process's first library calls")
    graph = torch.cuda.CUDAGraph()
    attn_out = torch.empty((B, H, 1, D), dtype=torch.float16, device="cuda")
    with torch.cuda.graph(graph):
        outs = [gemm_call(c) for c in gemms] + [packed_call(c, 0) for c in packed]
        attn_call(attn_out)
    outs.append(attn_out)

    say("replays")
    graph.replay()
    torch.cuda.synchronize()
    first = [o.clone() for o in outs]
    scratch = torch.randn(1 << 20, device="cuda")
    for r in range(3):
        scratch.mul_(1.0001)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            assert torch.equal(o.view(torch.int8), first[i].view(torch.int8)), f"replay {r}: output {i} changed"

    say("replay beside eager calls on another stream")
    side = torch.cuda.Stream()
    for r in range(3):
        with torch.cuda.stream(side):
            eager = [gemm_call(c) for c in gemms] + [packed_call(c, 1) for c in packed]
            eager_attn = torch.empty_like(attn_out)
            attn_call(eager_attn)
        graph.replay()
        torch.cuda.synchronize()
        eager.append(eager_attn)
        for i, (o, e) in enumerate(zip(outs, eager)):
            assert torch.equal(o.view(torch.int8), first[i].view(torch.int8)), f"concurrent replay {r}: output {i}"
            assert torch.equal(e.view(torch.int8), first[i].view(torch.int8)), f"eager call {r}: output {i}"

    say("oracle")
    worst = {}
    for c, o in zip(gemms, first):
        ref = oracle.linear(c["a"], q=c["q"], scales=c["s"], bias_bits=c["bias"],
                            out_dtype="f32" if c["out32"] else "f16")
        ref = ref.astype(np.float64) if c["out32"] else ref.view(np.float16).astype(np.float64)
        got = o.cpu().numpy().astype(np.float64)
        err = np.abs(got - ref)
        assert np.all(np.isfinite(got)) and np.all(err <= 2e-2 + 1e-2 * np.abs(ref)), (c["m"], c["n"], err.max())
        worst[f"M{c['m']}_{c['k']}to{c['n']}_cfg{c['config']}"] = float(err.max())
    worst_packed = {}
    for c, o in zip(packed, first[len(gemms):]):
        ref = oracle.linear(c["a"], q=c["q"], scales=c["s"], bias_bits=c["bias"], gelu=True)
        ref = ref.view(np.float16).astype(np.float64)
        got = o.cpu().numpy().astype(np.float64)
        err = np.abs(got - ref)
        assert np.all(np.isfinite(got)) and np.all(err <= 2e-2 + 1e-2 * np.abs(ref)), (c["m"], c["n"], err.max())
        worst_packed[f"M{c['m']}_{c['k']}to{c['n']}_gelu"] = float(err.max())
    got = first[-1].cpu().numpy().view(np.uint16).view(np.float16).astype(np.float64)
    ref = oracle.attention_f16(aq, ak, av, [1] * B, L, L - 1, True).view(np.float16).astype(np.float64)
    aerr = float(np.abs(got - ref).max())
    assert aerr <= 1e-4, aerr
    print(json.dumps({"ok": True, "gemm_max_err": worst, "packed_max_err": worst_packed, "attention_max_err": aerr}),
          flush=True)


if __name__ == "__main__":
    main()
