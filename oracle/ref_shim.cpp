// ref_shim.cpp -- C-ABI binding over the reference's own kernels/cpu library.
//
// TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile together with the
// reference's kernels/cpu/cpu_reference.cpp, straight from /root/reference,
// into oracle/_ref/libpkref.so, so tests can call the reference's launch_*_cpu
// (kernels/cpu/cpu_reference.h:37-154) with ctypes and pin the C restatement in
// oracle.c bit for bit.  Nothing here is product code.
#include "cpu_reference.h"

namespace pkc = polykernel::cpu;

extern "C" {
void ref_rmsnorm(const uint16_t *in, const uint16_t *w, uint16_t *out, int64_t rows,
                 int64_t cols, float eps) {
  pkc::launch_rmsnorm_cpu(in, w, out, rows, cols, eps);
}
void ref_gelu(const uint16_t *in, uint16_t *out, int64_t n) { pkc::launch_gelu_cpu(in, out, n); }
void ref_matmul(const uint16_t *a, const uint16_t *b, uint16_t *c, int64_t M, int64_t N,
                int64_t K) {
  pkc::launch_matmul_cpu(a, b, c, M, N, K);
}
void ref_fused_rmsnorm_matmul(const uint16_t *x, const uint16_t *w, uint16_t *out, int64_t M,
                              int64_t N, int64_t K, float eps) {
  pkc::launch_fused_rmsnorm_matmul_cpu(x, w, out, M, N, K, eps);
}
void ref_fused_matmul_bias_gelu(const uint16_t *a, const uint16_t *b, const uint16_t *bias,
                                uint16_t *out, int64_t M, int64_t N, int64_t K) {
  pkc::launch_fused_matmul_bias_gelu_cpu(a, b, bias, out, M, N, K);
}
void ref_softmax(const uint16_t *in, uint16_t *out, int64_t rows, int64_t cols) {
  pkc::launch_softmax_cpu(in, out, rows, cols);
}
uint16_t ref_f32_to_bf16(float f) { return pkc::float_to_bf16(f); }
}
