// pybind11 module `ikernels` (installed next to libtinyinfer_backend.so, which
// tinyc locates through ikernels.__file__).  Same functions, arguments and
// errors as reference kernels/python/bindings.cpp:52-70:
//   openmp_threads(); matmul(A, B, blocked=True); softmax(x, fused=True);
//   layernorm(x, gamma, beta, eps=1e-5, fused=True)   -- FP32 NumPy on the host
//   has_cuda (True: this build has the gfx950 GPU path); cuda_device_available();
//   cuda_bench_matmul(variant, M, N, K, iters=20), cuda_bench_softmax(rows, cols,
//   iters=50), cuda_bench_layernorm(rows, cols, iters=50) -> mean ms per launch
//   from HIP events around `iters` back-to-back launches after 3 warmups.
// Host ops call the library's ti_cpu_* entry points (blocked / fused) or a
// plain loop (the unblocked variants); shape errors raise ValueError.
#include <hip/hip_runtime.h>
#include <omp.h>
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>

#include <cmath>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/tinyinfer_backend.h"
#include "kernels.hpp"

namespace py = pybind11;
using Arr = py::array_t<float, py::array::c_style | py::array::forcecast>;

namespace {

void need2d(const Arr& a, const char* name) {
  if (a.ndim() != 2) throw std::invalid_argument(std::string(name) + " must be 2-D");
}

Arr matmul(Arr A, Arr B, bool blocked) {
  need2d(A, "A");
  need2d(B, "B");
  const int m = int(A.shape(0)), k = int(A.shape(1)), n = int(B.shape(1));
  if (B.shape(0) != k) throw std::invalid_argument("inner dimensions differ");
  Arr C({m, n});
  {
    py::gil_scoped_release nogil;
    if (blocked) {
      ti_cpu_gemm(A.data(), B.data(), C.mutable_data(), m, k, n);
    } else {
      const float *a = A.data(), *b = B.data();
      float* c = C.mutable_data();
      for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j) {
          float s = 0.f;
          for (int kk = 0; kk < k; ++kk) s += a[size_t(i) * k + kk] * b[size_t(kk) * n + j];
          c[size_t(i) * n + j] = s;
        }
    }
  }
  return C;
}

Arr softmax(Arr x, bool fused) {
  need2d(x, "x");
  const int rows = int(x.shape(0)), cols = int(x.shape(1));
  Arr y({rows, cols});
  {
    py::gil_scoped_release nogil;
    if (fused) {
      ti_cpu_softmax(x.data(), y.mutable_data(), rows, cols);
    } else {
      const float* xp = x.data();
      float* yp = y.mutable_data();
      for (int r = 0; r < rows; ++r) {
        float mx = -INFINITY, s = 0.f;
        for (int c = 0; c < cols; ++c) mx = std::fmax(mx, xp[size_t(r) * cols + c]);
        for (int c = 0; c < cols; ++c) s += (yp[size_t(r) * cols + c] = std::exp(xp[size_t(r) * cols + c] - mx));
        for (int c = 0; c < cols; ++c) yp[size_t(r) * cols + c] /= s;
      }
    }
  }
  return y;
}

Arr layernorm(Arr x, Arr g, Arr b, float eps, bool fused) {
  need2d(x, "x");
  const int rows = int(x.shape(0)), cols = int(x.shape(1));
  if (g.size() != cols || b.size() != cols) throw std::invalid_argument("gamma/beta size");
  Arr y({rows, cols});
  {
    py::gil_scoped_release nogil;
    if (fused) {
      ti_cpu_layernorm(x.data(), g.data(), b.data(), y.mutable_data(), rows, cols, eps);
    } else {
      const float *xp = x.data(), *gp = g.data(), *bp = b.data();
      float* yp = y.mutable_data();
      for (int r = 0; r < rows; ++r) {
        double mean = 0, var = 0;
        for (int c = 0; c < cols; ++c) mean += xp[size_t(r) * cols + c];
        mean /= cols;
        for (int c = 0; c < cols; ++c) var += (xp[size_t(r) * cols + c] - mean) * (xp[size_t(r) * cols + c] - mean);
        const double inv = 1.0 / std::sqrt(var / cols + eps);
        for (int c = 0; c < cols; ++c)
          yp[size_t(r) * cols + c] = float((xp[size_t(r) * cols + c] - mean) * inv) * gp[c] + bp[c];
      }
    }
  }
  return y;
}

void hip_check(hipError_t e) {
  if (e != hipSuccess) throw std::runtime_error(hipGetErrorString(e));
}

bool device_available() {
  int n = 0;
  return hipGetDeviceCount(&n) == hipSuccess && n > 0;
}

struct DeviceBuffer {
  float* p = nullptr;
  DeviceBuffer(size_t n, unsigned seed) {
    std::vector<float> h(n);
    std::mt19937 rng(seed);
    std::uniform_real_distribution<float> d(-1.f, 1.f);
    for (auto& v : h) v = d(rng);
    hip_check(hipMalloc(&p, n * sizeof(float)));
    hip_check(hipMemcpy(p, h.data(), n * sizeof(float), hipMemcpyHostToDevice));
  }
  ~DeviceBuffer() { (void)hipFree(p); }
};

template <class F>
double time_ms(F&& launch, int iters) {
  if (iters < 1) throw std::invalid_argument("iters must be positive");
  for (int i = 0; i < 3; ++i) hip_check(launch());
  hipEvent_t a, b;
  hip_check(hipEventCreate(&a));
  hip_check(hipEventCreate(&b));
  hip_check(hipEventRecord(a, nullptr));
  for (int i = 0; i < iters; ++i) hip_check(launch());
  hip_check(hipEventRecord(b, nullptr));
  hip_check(hipEventSynchronize(b));
  float ms = 0.f;
  hip_check(hipEventElapsedTime(&ms, a, b));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  return double(ms) / iters;
}

double bench_matmul(int variant, int m, int n, int k, int iters) {
  if (variant < 0 || variant > 2) throw std::invalid_argument("variant must be 0, 1 or 2");
  DeviceBuffer A(size_t(m) * k, 1), B(size_t(k) * n, 2), C(size_t(m) * n, 3);
  return time_ms([&] { return tia::legacy_gemm_f32_variant(variant, A.p, B.p, C.p, m, n, k, nullptr); }, iters);
}
double bench_softmax(int rows, int cols, int iters) {
  DeviceBuffer x(size_t(rows) * cols, 3), y(size_t(rows) * cols, 4);
  return time_ms([&] { return tia::softmax_f32(x.p, y.p, rows, cols, nullptr); }, iters);
}
double bench_layernorm(int rows, int cols, int iters) {
  DeviceBuffer x(size_t(rows) * cols, 4), g(cols, 5), b(cols, 6), y(size_t(rows) * cols, 7);
  return time_ms([&] { return tia::layernorm_f32(x.p, g.p, b.p, y.p, rows, cols, 1e-5f, nullptr); }, iters);
}

}  // namespace

PYBIND11_MODULE(ikernels, m) {
  m.doc() = "tinyinfer MI355X (gfx950) backend: host FP32 ops and GPU benchmark hooks";
  m.def("openmp_threads", [] { return omp_get_max_threads(); });
  m.def("matmul", &matmul, py::arg("A"), py::arg("B"), py::arg("blocked") = true);
  m.def("softmax", &softmax, py::arg("x"), py::arg("fused") = true);
  m.def("layernorm", &layernorm, py::arg("x"), py::arg("gamma"), py::arg("beta"), py::arg("eps") = 1e-5f,
        py::arg("fused") = true);
  m.attr("has_cuda") = true;
  m.def("cuda_device_available", &device_available);
  m.def("cuda_bench_matmul", &bench_matmul, py::arg("variant"), py::arg("M"), py::arg("N"), py::arg("K"),
        py::arg("iters") = 20,
        "HIP-event ms per launch of FP32 GEMM variant 0 (naive), 1 (LDS-tiled) or 2 (register-tiled)");
  m.def("cuda_bench_softmax", &bench_softmax, py::arg("rows"), py::arg("cols"), py::arg("iters") = 50);
  m.def("cuda_bench_layernorm", &bench_layernorm, py::arg("rows"), py::arg("cols"), py::arg("iters") = 50);
}
