// C entry points over the reference's CPU kernels (declared in the reference's
// own kernels/include/ik/cpu_kernels.hpp) so tests can reach them through
// ctypes.  The reference's host codec already exports C symbols (ti_host_*).
#include "ik/cpu_kernels.hpp"

extern "C" {
void ref_matmul_blocked(const float* a, const float* b, float* c, int m, int n, int k) {
  ik::cpu::matmul_blocked(a, b, c, m, n, k);
}
void ref_softmax_fused(const float* x, float* y, int r, int c) { ik::cpu::softmax_fused(x, y, r, c); }
void ref_softmax_naive(const float* x, float* y, int r, int c) { ik::cpu::softmax_naive(x, y, r, c); }
void ref_layernorm_fused(const float* x, const float* g, const float* b, float* y, int r, int c, float e) {
  ik::cpu::layernorm_fused(x, g, b, y, r, c, e);
}
void ref_layernorm_naive(const float* x, const float* g, const float* b, float* y, int r, int c, float e) {
  ik::cpu::layernorm_naive(x, g, b, y, r, c, e);
}
}
