// dn_prefill.hip -- the DeltaNet layer's work around the chunk rule for a
// whole prompt: causal depthwise conv (k = 4) + SiLU + L2 of the Q/K heads
// over T tokens, g/beta per token, and the gated RMSNorm of the chunk output.
//
// Per token these are exactly the decode shaders' operations
// (deltanet_conv_l2_qk.comp:41-111, deltanet_recurrent_gbeta_norm_gate.comp:
// 102-116 and :182-224, in the order decode.hip evaluates them), so a prompt
// token and a decoded token at the same place get the same bits; only the
// recurrence itself is replaced by the chunk rule (spk_chunk_prefill).  The
// conv runs token-parallel: the output of token t needs the raw inputs
// t-3..t, taken from the conv state for t < 3.
#include "capi_common.hpp"
#include "numerics.hpp"

namespace {

constexpr int kConvDim = 6144;
constexpr int kHeads = 16;
constexpr int kDim = 128;

// grid (48 channel blocks of 128, T tokens); one wave: lane owns channels
// lane and lane + 64 of the block.  Block < 16: Q head, < 32: K head, else V.
__global__ __launch_bounds__(64) void dn_prefill_conv_kernel(const uint16_t* __restrict__ qkv, long long ld,
                                                             const uint16_t* __restrict__ conv_state,
                                                             const uint16_t* __restrict__ conv_w, int T,
                                                             uint16_t* __restrict__ q_hm,
                                                             uint16_t* __restrict__ k_hm,
                                                             uint16_t* __restrict__ v_hm) {
  const int blk = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  float y[2];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int ch = blk * kDim + lane + 64 * half;
    const uint2 wv = *reinterpret_cast<const uint2*>(conv_w + ch * 4);
    const float w[4] = {spk::h2f(wv.x & 0xffffu), spk::h2f(wv.x >> 16), spk::h2f(wv.y & 0xffffu),
                        spk::h2f(wv.y >> 16)};
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // window x_{t-3..t}, taps in order 0..3
      const int j = t - 3 + i;
      const uint16_t x = j >= 0 ? qkv[(long long)j * ld + ch] : conv_state[ch * 4 + (j + 4)];
      sum = sum + spk::h2f(x) * w[i];
    }
    y[half] = spk::h2f(spk::f2h(spk::silu_det(sum)));
  }
  if (blk < 2 * kHeads) {  // L2 of the Q / K head block: 128-wide tree, eps inside the sqrt
    float v = y[0] * y[0] + y[1] * y[1];
    v = spk::tree64_to_lane0(v);
    const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));  // lane 0 broadcast, no LDS
    const float inv = spk::rsqrt_det(tot + 1e-6f);
    y[0] = y[0] * inv;
    y[1] = y[1] * inv;
  }
  const int h = blk % kHeads;
  uint16_t* dst = blk < kHeads ? q_hm : (blk < 2 * kHeads ? k_hm : v_hm);
  uint16_t* row = dst + ((long long)h * T + t) * kDim;
  row[lane] = spk::f2h(y[0]);
  row[lane + 64] = spk::f2h(y[1]);
}

// Conv state after the prompt: the last 4 raw inputs per channel.
__global__ void dn_prefill_conv_state_kernel(const uint16_t* __restrict__ qkv, long long ld,
                                             uint16_t* __restrict__ conv_state, int T) {
  const int ch = blockIdx.x * blockDim.x + threadIdx.x;
  if (ch >= kConvDim) return;
  uint16_t nv[4];
  const uint2 old = *reinterpret_cast<const uint2*>(conv_state + ch * 4);
  const uint16_t ov[4] = {(uint16_t)(old.x & 0xffffu), (uint16_t)(old.x >> 16), (uint16_t)(old.y & 0xffffu),
                          (uint16_t)(old.y >> 16)};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int j = T - 4 + i;
    nv[i] = j >= 0 ? qkv[(long long)j * ld + ch] : ov[j + 4];
  }
  *reinterpret_cast<uint2*>(conv_state + ch * 4) =
      make_uint2((uint32_t)nv[0] | ((uint32_t)nv[1] << 16), (uint32_t)nv[2] | ((uint32_t)nv[3] << 16));
}

// g = -exp(A_log) * softplus(a + dt_bias), beta = sigmoid(b); head-major [16][T].
__global__ void dn_prefill_gbeta_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                        long long ld, const float* __restrict__ alb, int layer, int T,
                                        float* __restrict__ g, float* __restrict__ beta) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T * kHeads) return;
  const int t = i / kHeads, h = i % kHeads;
  const float av = spk::h2f(a[(long long)t * ld + h]);
  const float bv = spk::h2f(b[(long long)t * ld + h]);
  const float a_log = alb[(layer * kHeads + h) * 2];
  const float dt_bias = alb[(layer * kHeads + h) * 2 + 1];
  const float sp = spk::logf_det(1.0f + spk::expf_det(av + dt_bias));
  g[h * T + t] = -spk::expf_det(a_log) * sp;
  beta[h * T + t] = 1.0f / (1.0f + spk::expf_det(-bv));
}

// Gated RMSNorm of one 128-wide head row held by one wave (lane l: elements
// l and l + 64): the squares' tree (s[l] + s[l+64], then strides 32..1),
// r = 1/sqrt(sum/128 + eps), out = fp16(fp16(w * (o*r)) * SiLU(z)).
__device__ __forceinline__ void norm_gate_row(float oa, float ob, const uint16_t* __restrict__ zr,
                                              const float* __restrict__ norm_w, float eps,
                                              uint16_t* __restrict__ orow, int lane) {
  float v = oa * oa + ob * ob;
  v = spk::tree64_to_lane0(v);
  const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));  // lane 0 broadcast, no LDS
  const float r = spk::rsqrt_det(tot / 128.0f + eps);
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int j = lane + 64 * half;
    const float normed = (half ? ob : oa) * r;
    const float weighted = spk::h2f(spk::f2h(norm_w[j] * normed));
    orow[j] = spk::f2h(weighted * spk::silu_det(spk::h2f(zr[j])));
  }
}

// Gated RMSNorm of the fp32 chunk output: grid (16 heads, T); one wave.
__global__ __launch_bounds__(64) void dn_norm_gate_kernel(const float* __restrict__ core, long long head_stride,
                                                          const uint16_t* __restrict__ z, long long zld,
                                                          const float* __restrict__ norm_w, float eps,
                                                          uint16_t* __restrict__ out, long long old) {
  const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  const float* o = core + ((long long)h * head_stride + t) * kDim;
  norm_gate_row(o[lane], o[lane + 64], z + (long long)t * zld + h * kDim, norm_w, eps,
                out + (long long)t * old + h * kDim, lane);
}

// deltanet_norm_gate.comp:80-105 on fp16 rows, in place: grid (heads); one
// wave.  The shader's 256-lane tree first adds 128 zero partials (exact), so
// its sum is the 128-wide tree above.
__global__ __launch_bounds__(64) void dn_norm_gate_f16_kernel(uint16_t* __restrict__ io,
                                                              const uint16_t* __restrict__ z,
                                                              const float* __restrict__ norm_w, float eps) {
  const int h = blockIdx.x, lane = threadIdx.x;
  uint16_t* row = io + (long long)h * kDim;
  const float oa = spk::h2f(row[lane]), ob = spk::h2f(row[lane + 64]);
  norm_gate_row(oa, ob, z + (long long)h * kDim, norm_w, eps, row, lane);
}

}  // namespace

extern "C" int spk_deltanet_prefill_conv(const uint16_t* qkv, int64_t ld, uint16_t* conv_state,
                                         const uint16_t* conv_weight, int32_t tokens, uint16_t* q_hm,
                                         uint16_t* k_hm, uint16_t* v_hm, spk_stream_t stream) {
  if (!qkv || !conv_state || !conv_weight || !q_hm || !k_hm || !v_hm)
    return spk::fail(SPK_ERR_NULL, "spk_deltanet_prefill_conv: NULL pointer");
  if (tokens <= 0 || ld < kConvDim)
    return spk::fail(SPK_ERR_SHAPE, "spk_deltanet_prefill_conv: tokens %d ld %lld", tokens, (long long)ld);
  if (!spk::aligned(conv_state, 8) || !spk::aligned(conv_weight, 8))
    return spk::fail(SPK_ERR_ALIGN, "spk_deltanet_prefill_conv: conv buffers must be 8-byte aligned");
  hipStream_t s = spk::to_hip(stream);
  hipLaunchKernelGGL(dn_prefill_conv_kernel, dim3(kConvDim / kDim, tokens), dim3(64), 0, s, qkv, (long long)ld,
                     conv_state, conv_weight, tokens, q_hm, k_hm, v_hm);
  int rc = spk::check_launch("spk_deltanet_prefill_conv");
  if (rc) return rc;
  hipLaunchKernelGGL(dn_prefill_conv_state_kernel, dim3(kConvDim / 256), dim3(256), 0, s, qkv, (long long)ld,
                     conv_state, tokens);
  return spk::check_launch("spk_deltanet_prefill_conv (state)");
}

extern "C" int spk_deltanet_prefill_gbeta(const uint16_t* a, const uint16_t* b, int64_t ld,
                                          const float* a_log_bias, int32_t layer_idx, int32_t tokens, float* g,
                                          float* beta, spk_stream_t stream) {
  if (!a || !b || !a_log_bias || !g || !beta) return spk::fail(SPK_ERR_NULL, "spk_deltanet_prefill_gbeta: NULL pointer");
  if (tokens <= 0 || ld < kHeads || layer_idx < 0)
    return spk::fail(SPK_ERR_SHAPE, "spk_deltanet_prefill_gbeta: tokens %d ld %lld layer %d", tokens, (long long)ld,
                     layer_idx);
  const int n = tokens * kHeads;
  hipLaunchKernelGGL(dn_prefill_gbeta_kernel, dim3((n + 255) / 256), dim3(256), 0, spk::to_hip(stream), a, b,
                     (long long)ld, a_log_bias, layer_idx, tokens, g, beta);
  return spk::check_launch("spk_deltanet_prefill_gbeta");
}

extern "C" int spk_deltanet_norm_gate(const float* core, int64_t core_head_stride, const uint16_t* z, int64_t z_ld,
                                      const float* norm_weight, float eps, int32_t tokens, uint16_t* out,
                                      int64_t out_ld, spk_stream_t stream) {
  if (!core || !z || !norm_weight || !out) return spk::fail(SPK_ERR_NULL, "spk_deltanet_norm_gate: NULL pointer");
  if (tokens <= 0 || core_head_stride < tokens || z_ld < kHeads * kDim || out_ld < kHeads * kDim)
    return spk::fail(SPK_ERR_SHAPE, "spk_deltanet_norm_gate: tokens %d head stride %lld", tokens,
                     (long long)core_head_stride);
  hipLaunchKernelGGL(dn_norm_gate_kernel, dim3(kHeads, tokens), dim3(64), 0, spk::to_hip(stream), core,
                     (long long)core_head_stride, z, (long long)z_ld, norm_weight, eps != 0.0f ? eps : 1e-6f, out,
                     (long long)out_ld);
  return spk::check_launch("spk_deltanet_norm_gate");
}

extern "C" int spk_deltanet_norm_gate_f16(uint16_t* io, const uint16_t* z, const float* norm_weight,
                                          int32_t num_heads, int32_t head_dim, float eps, spk_stream_t stream) {
  if (!io || !z || !norm_weight) return spk::fail(SPK_ERR_NULL, "spk_deltanet_norm_gate_f16: NULL pointer");
  if (num_heads <= 0 || head_dim != kDim)
    return spk::fail(SPK_ERR_SHAPE, "spk_deltanet_norm_gate_f16: num_heads %d head_dim %d (head_dim must be %d)",
                     num_heads, head_dim, kDim);
  hipLaunchKernelGGL(dn_norm_gate_f16_kernel, dim3(num_heads), dim3(64), 0, spk::to_hip(stream), io, z, norm_weight,
                     eps);
  return spk::check_launch("spk_deltanet_norm_gate_f16");
}
