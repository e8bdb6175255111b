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

// 16-byte reads of the whole buffer, non-temporal (NT) or plain cached
// loads, four per thread per round.  STRIDE: the grid walks the whole buffer
// in steps of grid x 256 x 16 bytes; otherwise workgroup b reads its own
// contiguous share.  Measured on MI355X: over 2 GiB, contiguous shares reach
// 6.8-7.1 TB/s with non-temporal loads against 6.0-6.9 TB/s for the
// grid-stride walk (cached loads 5.5-6.5); for reads of a few MB in one
// launch the grid-stride walk is the faster one.  Each thread's XOR of what
// it read is stored only if it equals a fixed constant, so the reads cannot
// be dropped and (almost) nothing is written.
template <bool NT, bool STRIDE>
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ p, long long n16,
                                                          uint32_t* __restrict__ out) {
  long long lo, hi, step, lane_step;
  if (STRIDE) {
    lo = 0;
    hi = n16;
    lane_step = (long long)gridDim.x * blockDim.x;
    step = 4 * lane_step;
  } else {
    const long long per = (n16 + gridDim.x - 1) / gridDim.x;
    lo = (long long)blockIdx.x * per;
    hi = min(lo + per, n16);
    lane_step = 256;
    step = 4 * 256;
  }
  const long long first = STRIDE ? (long long)blockIdx.x * blockDim.x + threadIdx.x : lo + threadIdx.x;
  uint32_t acc = 0;
  for (long long i = first; i < hi; i += step) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long long j = min(i + u * lane_step, hi - 1);
      v[u] = NT ? __builtin_nontemporal_load(p + j) : p[j];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9e3779b9u) out[blockIdx.x] = acc;
}

// XCC (XCD) id of each workgroup: hardware register HW_REG_XCC_ID (20),
// bits 3:0.
__global__ __launch_bounds__(64) void xcc_id_kernel(int32_t* __restrict__ out) {
  if (threadIdx.x == 0) out[blockIdx.x] = (int32_t)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15);
}

}  // namespace

extern "C" int spk_selftest_xcc_ids(int32_t blocks, int32_t* out, spk_stream_t stream) {
  if (!out) return spk::fail(SPK_ERR_NULL, "spk_selftest_xcc_ids: NULL out");
  if (blocks <= 0) return spk::fail(SPK_ERR_SHAPE, "spk_selftest_xcc_ids: blocks %d", blocks);
  hipLaunchKernelGGL(xcc_id_kernel, dim3(blocks), dim3(64), 0, spk::to_hip(stream), out);
  return spk::check_launch("spk_selftest_xcc_ids");
}

extern "C" int spk_selftest_mfma_peak(int32_t blocks, int32_t iters, float* out, spk_stream_t stream) {
  if (!out) return spk::fail(SPK_ERR_NULL, "spk_selftest_mfma_peak: NULL out");
  if (blocks <= 0 || iters <= 0) return spk::fail(SPK_ERR_SHAPE, "spk_selftest_mfma_peak: blocks %d iters %d", blocks, iters);
  hipLaunchKernelGGL(mfma_peak_kernel, dim3(blocks), dim3(256), 0, spk::to_hip(stream), iters, out);
  return spk::check_launch("spk_selftest_mfma_peak");
}

extern "C" int spk_selftest_stream_read(const void* p, size_t bytes, int32_t blocks, int32_t mode,
                                        uint32_t* out, spk_stream_t stream) {
  if (!p || !out) return spk::fail(SPK_ERR_NULL, "spk_selftest_stream_read: NULL pointer");
  if (bytes < 16 || bytes % 16 || blocks <= 0 || !spk::aligned(p, 16) || mode < 0 || mode > 3)
    return spk::fail(SPK_ERR_SHAPE, "spk_selftest_stream_read: bytes %zu blocks %d mode %d (16-byte multiple and alignment)",
                     bytes, blocks, mode);
  const u32x4* src = static_cast<const u32x4*>(p);
  const long long n16 = (long long)(bytes / 16);
  hipStream_t s = spk::to_hip(stream);
  switch (mode) {
    case 0: hipLaunchKernelGGL((stream_read_kernel<true, false>), dim3(blocks), dim3(256), 0, s, src, n16, out); break;
    case 1: hipLaunchKernelGGL((stream_read_kernel<false, false>), dim3(blocks), dim3(256), 0, s, src, n16, out); break;
    case 2: hipLaunchKernelGGL((stream_read_kernel<true, true>), dim3(blocks), dim3(256), 0, s, src, n16, out); break;
    default: hipLaunchKernelGGL((stream_read_kernel<false, true>), dim3(blocks), dim3(256), 0, s, src, n16, out); break;
  }
  return spk::check_launch("spk_selftest_stream_read");
}
