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

// ---------------------------------------------------------------------------
// Measured ceilings for the roofline denominators (reported beside the
// datasheet peaks): dense fp32 MFMA issue and a read-only HBM stream.
// ---------------------------------------------------------------------------
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Every wavefront runs 8 independent v_mfma_f32_16x16x4_f32 chains of `iters`
// steps (2 * 16 * 16 * 4 FLOP per instruction).
__global__ __launch_bounds__(256) void mfma_peak_kernel(int iters, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  float a = 1.0f + 1e-7f * (float)lane, b = 1.0f - 1e-7f * (float)lane;
  v4f acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < 8; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

// Grid-stride 16-byte reads of the whole buffer, non-temporal (NT) or plain
// cached loads.  Each thread's XOR of what it read is stored only if it equals
// a fixed constant, so the reads cannot be dropped and (almost) nothing is
// written.
template <bool NT>
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, long long n16,
                                                          uint32_t* __restrict__ out) {
  uint32_t acc = 0;
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += 4 * stride) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long long j = min(i + u * stride, n16 - 1);
      v[u] = NT ? __builtin_nontemporal_load(p + j) : p[j];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) out[blockIdx.x] = acc;
}

}  // namespace

extern "C" int spk_selftest_mfma_peak(int32_t blocks, int32_t iters, float* out, spk_stream_t stream) {
  if (!out) return spk::fail(SPK_ERR_NULL, "spk_selftest_mfma_peak: NULL out");
  if (blocks <= 0 || iters <= 0) return spk::fail(SPK_ERR_SHAPE, "spk_selftest_mfma_peak: blocks %d iters %d", blocks, iters);
  hipLaunchKernelGGL(mfma_peak_kernel, dim3(blocks), dim3(256), 0, spk::to_hip(stream), iters, out);
  return spk::check_launch("spk_selftest_mfma_peak");
}

extern "C" int spk_selftest_stream_read(const void* p, size_t bytes, int32_t blocks, int32_t cached,
                                        uint32_t* out, spk_stream_t stream) {
  if (!p || !out) return spk::fail(SPK_ERR_NULL, "spk_selftest_stream_read: NULL pointer");
  if (bytes < 16 || bytes % 16 || blocks <= 0 || !spk::aligned(p, 16))
    return spk::fail(SPK_ERR_SHAPE, "spk_selftest_stream_read: bytes %zu blocks %d (16-byte multiple and alignment)",
                     bytes, blocks);
  const u32x4* src = static_cast<const u32x4*>(p);
  if (cached)
    hipLaunchKernelGGL(stream_read_kernel<false>, dim3(blocks), dim3(256), 0, spk::to_hip(stream), src,
                       (long long)(bytes / 16), out);
  else
    hipLaunchKernelGGL(stream_read_kernel<true>, dim3(blocks), dim3(256), 0, spk::to_hip(stream), src,
                       (long long)(bytes / 16), out);
  return spk::check_launch("spk_selftest_stream_read");
}
