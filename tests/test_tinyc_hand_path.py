"""tinyc's "hand" dispatch against the legacy FP32 ABI: a C++ caller with the
shape of tinyc's generated code (reference tinyc/codegen_cpp.py:102-132,
tinyc/runtime/tinyc_runtime.hpp:11-14: ti_cpu_gemm(a, b, tmp, m, k, n) into a
temporary, bias epilogue, ti_cpu_layernorm, ti_cpu_softmax) compiled against
include/tinyinfer_backend.h and linked to libtinyinfer_backend.so; its CUDA
twin (tinyc/codegen_cuda.py:50-65) through ti_cuda_* on the GPU; and the three
FP32 GEMM variants of ikernels.cuda_bench_matmul (reference
kernels/src/cuda/bench_api.cu:43-51).  Tolerances from the reference's tests
(kernels/tests/test_cpu.cpp, test_cuda.cpp): GEMM 1e-5*K + 1e-5, LayerNorm
1e-4 (CPU) / 1e-3 (GPU), softmax 1e-5."""
import ctypes as C
import subprocess

import numpy as np
import pytest

from tests.conftest import ROOT

M, K, N = 33, 65, 70  # ragged, as the reference's shapes (65x257x300 style)


def _inputs(seed):
    rng = np.random.default_rng(seed)
    x = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    w = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    bias, g, b = (rng.uniform(-1, 1, N).astype(np.float32) for _ in range(3))
    return x, w, bias, g, b


def _expected(x, w, bias, g, b):
    lin = x.astype(np.float64) @ w + bias
    mu = lin.mean(1, keepdims=True)
    ln = (lin - mu) / np.sqrt(((lin - mu) ** 2).mean(1, keepdims=True) + 1e-5) * g + b
    e = np.exp(ln - ln.max(1, keepdims=True))
    return lin, ln, e / e.sum(1, keepdims=True)


def _run(binary, tmp_path, seed):
    args = _inputs(seed)
    src, dst = tmp_path / "in.bin", tmp_path / "out.bin"
    np.concatenate([a.ravel() for a in args]).astype(np.float32).tofile(src)
    subprocess.run([str(binary), str(M), str(K), str(N), str(src), str(dst)], check=True, timeout=60)
    out = np.fromfile(dst, np.float32).reshape(3, M, N)
    return out, _expected(*args)


def test_tinyc_hand_caller_cpu(tmp_path):
    from tests.tinyc_caller.build import build_cpu
    binary = build_cpu(tmp_path)
    (lin, ln, sm), (want_lin, want_ln, want_sm) = _run(binary, tmp_path, 1)
    assert np.allclose(lin, want_lin, atol=1e-5 * K + 1e-5)
    assert np.allclose(ln, want_ln, atol=1e-4)
    assert np.allclose(sm, want_sm, atol=1e-5)


@pytest.mark.gpu
def test_tinyc_hand_caller_gpu(tmp_path):
    binary = ROOT / "tests" / "tinyc_caller" / "hand_gpu"
    assert binary.is_file(), "tests/tinyc_caller/hand_gpu is built by __graft_entry__.build()"
    print("[case] tinyc hand caller on ti_cuda_*", flush=True)
    (lin, ln, sm), (want_lin, want_ln, want_sm) = _run(binary, tmp_path, 2)
    assert np.allclose(lin, want_lin, atol=1e-5 * K + 1e-5)
    assert np.allclose(ln, want_ln, atol=1e-3)
    assert np.allclose(sm, want_sm, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("variant", [0, 1, 2])
def test_fp32_gemm_variants(variant):
    import torch
    from tinyinfer_amd import BACKEND_LIB
    lib = C.CDLL(str(BACKEND_LIB))
    fn = lib.ti_amd_legacy_gemm_f32_variant
    fn.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_size_t, C.c_int]
    rng = np.random.default_rng(variant)
    for m, n, k in ((1, 1, 1), (7, 13, 5), (65, 257, 300), (128, 96, 513)):
        print(f"[case] fp32 gemm variant {variant} {m}x{n}x{k}", flush=True)
        a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
        da, db = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
        assert fn(variant, da.data_ptr(), db.data_ptr(), y.data_ptr(), m, n, k,
                  torch.cuda.current_stream().cuda_stream, 0) == 0
        torch.cuda.synchronize()
        assert np.allclose(y.cpu().numpy(), a.astype(np.float64) @ b, atol=1e-5 * k + 1e-5)
    import tinyinfer_amd.ikernels as ik
    assert ik.cuda_bench_matmul(variant, 256, 256, 256, iters=3) > 0
    with pytest.raises(ValueError):
        ik.cuda_bench_matmul(3, 16, 16, 16)
