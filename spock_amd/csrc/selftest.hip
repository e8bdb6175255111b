// selftest.hip -- diagnostics: evaluates the device scalar numerics over an
// array so tests can compare them bit for bit with the CPU restatement.
#include "capi_common.hpp"
#include "numerics.hpp"

namespace {

__global__ void numerics_kernel(const float* __restrict__ x, int n, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  out[0 * (size_t)n + i] = spk::expf_det(v);
  out[1 * (size_t)n + i] = spk::logf_det(v);
  out[2 * (size_t)n + i] = spk::rsqrt_det(v);
  out[3 * (size_t)n + i] = spk::silu_det(v);
  out[4 * (size_t)n + i] = spk::h2f(spk::f2h(v));
  out[5 * (size_t)n + i] = __uint_as_float((uint32_t)spk::f2h_trunc(v));
}

}  // namespace

extern "C" int spk_selftest_numerics(const float* x, int32_t n, float* out, spk_stream_t stream) {
  if (!x || !out) return spk::fail(SPK_ERR_NULL, "spk_selftest_numerics: NULL pointer");
  if (n <= 0) return spk::fail(SPK_ERR_SHAPE, "spk_selftest_numerics: n %d", n);
  hipLaunchKernelGGL(numerics_kernel, dim3((n + 255) / 256), dim3(256), 0, spk::to_hip(stream), x, n, out);
  return spk::check_launch("spk_selftest_numerics");
}
