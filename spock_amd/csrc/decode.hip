// decode.hip -- DeltaNet recurrent decode step for B independent sequences.
//
// One workgroup of 4, 8 or 16 wavefronts per (head, sequence): the launch
// picks the width from the batch (16 wavefronts when a handful of heads must
// carry the whole launch, 4 when thousands of workgroups fill the chip).  The
// step itself (conv, L2, g/beta, recurrence, norm-gate; its reduction orders)
// is spk_dn::dn_step in dn_step.hpp.
#include <stdlib.h>

#include "capi_common.hpp"
#include "numerics.hpp"
#include "dn_step.hpp"

namespace {

using spk_dn::DecodeParams;
using spk_dn::make_params;

template <bool CONV, bool REC, bool GB_TAIL, bool NORM_GATE, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void dn_decode_kernel(DecodeParams p) {
  spk_dn::dn_step<CONV, REC, GB_TAIL, NORM_GATE, WAVES>(p, blockIdx.x, blockIdx.y);
}

int validate(const SpkDecodeArgs* a, bool conv, bool rec, bool gb_inline, bool norm_gate) {
  if (!a) return spk::fail(SPK_ERR_NULL, "decode: args is NULL");
  if (a->batch < 0) return spk::fail(SPK_ERR_SHAPE, "decode: batch %d < 0", a->batch);
  if (a->num_heads <= 0 || a->num_heads > 64)
    return spk::fail(SPK_ERR_SHAPE, "decode: num_heads %d unsupported", a->num_heads);
  const long long conv_dim = 3LL * a->num_heads * 128;
  if (!a->qkv) return spk::fail(SPK_ERR_NULL, "decode: qkv is NULL");
  if (a->batch > 1 && a->qkv_stride < conv_dim)
    return spk::fail(SPK_ERR_SHAPE, "decode: qkv_stride %lld < conv_dim %lld", (long long)a->qkv_stride, conv_dim);
  if (conv) {
    if (!a->conv_state || !a->conv_weight) return spk::fail(SPK_ERR_NULL, "decode: conv_state/conv_weight NULL");
    if (!spk::aligned(a->conv_state, 8) || !spk::aligned(a->conv_weight, 8) || (a->conv_state_stride % 4) != 0)
      return spk::fail(SPK_ERR_ALIGN, "decode: conv_state/conv_weight must be 8-byte aligned, stride %% 4 == 0");
    if (a->batch > 1 && a->conv_state_stride < conv_dim * 4)
      return spk::fail(SPK_ERR_SHAPE, "decode: conv_state_stride too small");
  }
  if (rec) {
    if (!a->state) return spk::fail(SPK_ERR_NULL, "decode: state is NULL");
    if (!spk::aligned(a->state, 16) || (a->state_stride % 4) != 0)
      return spk::fail(SPK_ERR_ALIGN, "decode: state must be 16-byte aligned with state_stride %% 4 == 0");
    const long long need = (long long)a->num_heads * 128 * 128 + (gb_inline ? 0 : 2LL * a->num_heads);
    if (a->batch > 1 && a->state_stride < need)
      return spk::fail(SPK_ERR_SHAPE, "decode: state_stride %lld < %lld", (long long)a->state_stride, need);
    if (gb_inline) {
      if (!a->a || !a->b || !a->a_log_bias) return spk::fail(SPK_ERR_NULL, "decode: a/b/a_log_bias NULL");
      if (a->layer_idx < 0) return spk::fail(SPK_ERR_ARG, "decode: layer_idx < 0");
      if (a->batch > 1 && a->ab_stride < a->num_heads) return spk::fail(SPK_ERR_SHAPE, "decode: ab_stride too small");
    }
    if (norm_gate) {
      if (!a->z || !a->norm_weight) return spk::fail(SPK_ERR_NULL, "decode: z/norm_weight NULL");
      if (a->batch > 1 && a->z_stride < a->num_heads * 128) return spk::fail(SPK_ERR_SHAPE, "decode: z_stride too small");
    }
  }
  return SPK_OK;
}

// Wavefronts per workgroup by the number of workgroups the launch has:
// overridable with SPK_DECODE_WAVES=4|8|16 (measurement only).  Measured (us
// per launch, B = 1 / 16 / 64 / 256 with 16 heads): 16 wavefronts 4.5 / 8.25
// / 29.2 / 99, 8: 4.55 / 8.37 / 25.5 / 86.7, 4: 5.1 / 9.4 / 25.6 / 87.3.  The
// reduction order does not depend on the count, so results are identical.
int decode_waves(int workgroups) {
  static const int forced = [] {
    const char* e = getenv("SPK_DECODE_WAVES");
    const int v = e ? atoi(e) : 0;
    return (v == 4 || v == 8 || v == 16) ? v : 0;
  }();
  if (forced) return forced;
  if (workgroups <= 256) return 16;
  if (workgroups <= 512) return 8;
  return 4;
}

template <bool CONV, bool REC, bool GB_TAIL, bool NORM_GATE>
int launch(const SpkDecodeArgs* a, spk_stream_t stream, const char* name) {
  const int rc = validate(a, CONV, REC, REC && !GB_TAIL, REC && NORM_GATE);
  if (rc) return rc;
  if (a->batch == 0) return SPK_OK;
  dim3 grid(a->num_heads, a->batch);
  const int waves = decode_waves(a->num_heads * a->batch);
  hipStream_t s = spk::to_hip(stream);
  if (waves == 16)
    hipLaunchKernelGGL((dn_decode_kernel<CONV, REC, GB_TAIL, NORM_GATE, 16>), grid, dim3(1024), 0, s,
                       make_params(a));
  else if (waves == 8)
    hipLaunchKernelGGL((dn_decode_kernel<CONV, REC, GB_TAIL, NORM_GATE, 8>), grid, dim3(512), 0, s,
                       make_params(a));
  else
    hipLaunchKernelGGL((dn_decode_kernel<CONV, REC, GB_TAIL, NORM_GATE, 4>), grid, dim3(256), 0, s,
                       make_params(a));
  return spk::check_launch(name);
}

}  // namespace

extern "C" int spk_deltanet_decode_step(const SpkDecodeArgs* a, spk_stream_t stream) {
  return launch<true, true, false, true>(a, stream, "spk_deltanet_decode_step");
}
extern "C" int spk_deltanet_conv_l2_qk(const SpkDecodeArgs* a, spk_stream_t stream) {
  return launch<true, false, false, false>(a, stream, "spk_deltanet_conv_l2_qk");
}
extern "C" int spk_deltanet_recurrent_gbeta_norm_gate(const SpkDecodeArgs* a, spk_stream_t stream) {
  return launch<false, true, false, true>(a, stream, "spk_deltanet_recurrent_gbeta_norm_gate");
}
extern "C" int spk_deltanet_recurrent(const SpkDecodeArgs* a, spk_stream_t stream) {
  return launch<false, true, true, false>(a, stream, "spk_deltanet_recurrent");
}
