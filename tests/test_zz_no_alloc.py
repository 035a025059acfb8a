"""GPU check of ti_amd_gemm_ex_i8_noalloc against ti_v2_gemm_ex_i8 through the
C ABI: identical bits on two calls in a row, the second smaller than the first,
and within the linear tolerance (rtol 1e-2 / atol 2e-2) of the CPU oracle; and
the no-allocation call captured into a graph on a fresh stream (a hipMalloc
there would fail the capture), its replays bit-identical to the eager call.
Both entry points keep split-K partials in the calling hardware queue's slot
of the library's static pool and finish them in the same launch."""
import ctypes as C

import numpy as np
import pytest

import oracle
from tinyinfer_amd import BACKEND_LIB

pytestmark = pytest.mark.gpu

P, I = C.c_void_p, C.c_int
ARGS = [P, P, P, P, P, P, I, I, I, I, I, C.c_size_t, I]


def _lib():
    lib = C.CDLL(str(BACKEND_LIB))
    for name in ("ti_v2_gemm_ex_i8", "ti_amd_gemm_ex_i8_noalloc"):
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = ARGS, I
    lib.ti_v2_last_error.restype = C.c_char_p
    return lib


def _case(m, n, k, seed):
    rng = np.random.default_rng(seed)
    a = np.asarray(rng.standard_normal((m, k)) * 0.25, np.float16).view(np.uint16)
    w = np.asarray(rng.standard_normal((k, n)) * 0.25, np.float16).view(np.uint16)
    bias = np.asarray(rng.standard_normal(n) * 0.1, np.float16).view(np.uint16)
    q, s = oracle.quantize(w)
    return a, q, s, bias


def _run(lib, name, dev, m, n, k, dtype, config):
    import torch
    a, q, s, bias = dev
    y = torch.empty((m, n), dtype=torch.float32 if dtype else torch.float16, device="cuda")
    ws = torch.empty((m, n), dtype=torch.float32, device="cuda") if config >= 6 else None
    stream = torch.cuda.current_stream().cuda_stream
    st = getattr(lib, name)(a.data_ptr(), q.data_ptr(), s.data_ptr(), bias.data_ptr(), y.data_ptr(),
                            None if ws is None else ws.data_ptr(), m, n, k, dtype, config, stream, 0)
    assert st == 0, (name, st, lib.ti_v2_last_error())
    torch.cuda.synchronize()
    return y.cpu().numpy()


# (M, N, K, dtype, config) pairs: the second call of each pair is smaller and
# reuses the array the first one filled.  Every shape here splits K.
PAIRS = [
    ((64, 768, 3072, 0, 0), (1, 768, 768, 0, 0)),       # 22-way split tiled, then 12-way split row GEMV
    ((32, 3072, 768, 1, 7), (8, 2304, 768, 0, 2)),      # workspace epilogue + fp32 out, then fused fp16
]


@pytest.mark.parametrize("pair", PAIRS, ids=lambda p: f"{p[0][:3]}->{p[1][:3]}")
def test_noalloc_gemm_equals_allocating_entry(pair):
    import torch
    lib = _lib()
    for i, (m, n, k, dtype, config) in enumerate(pair):
        print(f"[case] noalloc call {i}: M={m} N={n} K={k} dtype={dtype} config={config}", flush=True)
        a, q, s, bias = _case(m, n, k, seed=17 + 101 * i + m)
        dev = (torch.from_numpy(a).view(torch.float16).cuda(), torch.from_numpy(q).cuda(),
               torch.from_numpy(s).cuda(), torch.from_numpy(bias).view(torch.float16).cuda())
        got = _run(lib, "ti_amd_gemm_ex_i8_noalloc", dev, m, n, k, dtype, config)
        want = _run(lib, "ti_v2_gemm_ex_i8", dev, m, n, k, dtype, config)
        assert got.tobytes() == want.tobytes(), f"call {i}: no-allocation result differs from ti_v2_gemm_ex_i8"
        ref = oracle.linear(a, q=q, scales=s, bias_bits=bias, out_dtype="f32" if dtype else "f16")
        ref = ref.astype(np.float64) if dtype else ref.view(np.float16).astype(np.float64)
        err = np.abs(got.astype(np.float64) - ref)
        assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref)), f"call {i}: max err {err.max()}"


def test_noalloc_gemm_validates_before_enqueue():
    import torch
    lib = _lib()
    print("[case] noalloc validation: misaligned scales, bad config", flush=True)
    a = torch.zeros((1, 64), dtype=torch.float16, device="cuda")
    q = torch.zeros((64, 64), dtype=torch.int8, device="cuda")
    s = torch.ones(65, dtype=torch.float32, device="cuda")
    y = torch.full((1, 64), 7.0, dtype=torch.float16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    fn = lib.ti_amd_gemm_ex_i8_noalloc
    assert fn(a.data_ptr(), q.data_ptr(), s.data_ptr() + 2, None, y.data_ptr(), None, 1, 64, 64, 0, 0, stream, 0) == 1
    assert fn(a.data_ptr(), q.data_ptr(), s.data_ptr(), None, y.data_ptr(), None, 1, 64, 64, 0, 12, stream, 0) == 3
    assert fn(a.data_ptr(), q.data_ptr(), s.data_ptr(), None, y.data_ptr(), None, 1, 64, 64, 0, 7, stream, 0) == 1
    torch.cuda.synchronize()
    assert torch.all(y == 7.0).item()


def test_noalloc_gemm_captured_on_fresh_stream():
    import torch
    lib = _lib()
    m, n, k = 8, 768, 3072  # a split-K plan: partials go to the queue pool slot
    print(f"[case] noalloc under capture on a fresh stream: M={m} N={n} K={k}", flush=True)
    a, q, s, bias = _case(m, n, k, seed=5)
    dev = (torch.from_numpy(a).view(torch.float16).cuda(), torch.from_numpy(q).cuda(),
           torch.from_numpy(s).cuda(), torch.from_numpy(bias).view(torch.float16).cuda())
    want = _run(lib, "ti_amd_gemm_ex_i8_noalloc", dev, m, n, k, 0, 0)
    y = torch.empty((m, n), dtype=torch.float16, device="cuda")
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        st = lib.ti_amd_gemm_ex_i8_noalloc(dev[0].data_ptr(), dev[1].data_ptr(), dev[2].data_ptr(),
                                           dev[3].data_ptr(), y.data_ptr(), None, m, n, k, 0, 0,
                                           torch.cuda.current_stream().cuda_stream, 0)
    assert st == 0, lib.ti_v2_last_error()
    for r in range(3):
        y.fill_(0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert y.cpu().numpy().tobytes() == want.tobytes(), f"replay {r} differs from the eager call"
