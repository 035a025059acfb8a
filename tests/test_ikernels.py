"""The pybind11 `ikernels` module against reference kernels/tests/test_python.py:13-47
(tolerances from there) and its GPU benchmark hooks."""
import numpy as np
import pytest

ik = pytest.importorskip("tinyinfer_amd.ikernels")


def test_module_surface():
    for name in ("openmp_threads", "matmul", "softmax", "layernorm", "cuda_device_available",
                 "cuda_bench_matmul", "cuda_bench_softmax", "cuda_bench_layernorm"):
        assert callable(getattr(ik, name))
    assert ik.has_cuda is True and ik.openmp_threads() >= 1


@pytest.mark.parametrize("blocked", [True, False])
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (7, 13, 5), (65, 300, 257)])
def test_matmul(m, k, n, blocked):
    rng = np.random.default_rng(m + k + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    np.testing.assert_allclose(ik.matmul(a, b, blocked=blocked), a.astype(np.float64) @ b, atol=1e-4 * k)


@pytest.mark.parametrize("fused", [True, False])
def test_softmax_and_layernorm(fused):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((17, 129)).astype(np.float32) * 3
    e = np.exp(x - x.max(1, keepdims=True))
    np.testing.assert_allclose(ik.softmax(x, fused=fused), e / e.sum(1, keepdims=True), rtol=1e-6, atol=1e-4)
    g = rng.standard_normal(129).astype(np.float32)
    b = rng.standard_normal(129).astype(np.float32)
    xd = x.astype(np.float64)
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-5) * g + b
    np.testing.assert_allclose(ik.layernorm(x, g, b, fused=fused), ref, rtol=1e-4, atol=1e-4)


def test_shape_errors_raise_value_error():
    a = np.ones((2, 3), np.float32)
    with pytest.raises(ValueError):
        ik.matmul(a, a)
    with pytest.raises(ValueError):
        ik.softmax(np.ones(3, np.float32))
    with pytest.raises(ValueError):
        ik.layernorm(a, np.ones(2, np.float32), np.ones(3, np.float32))


@pytest.mark.gpu
def test_gpu_bench_hooks():
    assert ik.cuda_device_available()
    assert ik.cuda_bench_softmax(1024, 1024, iters=5) > 0
    assert ik.cuda_bench_layernorm(1024, 1024, iters=5) > 0
    assert ik.cuda_bench_matmul(2, 256, 256, 256, iters=3) > 0
