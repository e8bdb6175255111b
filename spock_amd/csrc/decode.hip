// decode.hip -- DeltaNet recurrent decode step for B independent sequences.
//
// One workgroup of 4, 8 or 16 wavefronts per (head, sequence): the launch
// picks the width and the state-load kind from the batch (16 wavefronts and
// plain loads when a handful of heads must carry the whole launch, 4
// wavefronts and non-temporal loads when thousands of workgroups fill the
// chip).  The step itself (conv, L2, g/beta, recurrence, norm-gate; its
// reduction orders) is spk_dn::dn_step in dn_step.hpp.
#include <stdlib.h>

#include "capi_common.hpp"
#include "numerics.hpp"
#include "dn_step.hpp"

namespace {

using spk_dn::DecodeParams;
using spk_dn::make_params;

template <bool CONV, bool REC, bool GB_TAIL, bool NORM_GATE, int WAVES, bool NT_STATE>
__global__ __launch_bounds__(WAVES * 64) void dn_decode_kernel(DecodeParams p) {
  spk_dn::dn_step<CONV, REC, GB_TAIL, NORM_GATE, WAVES, false, NT_STATE>(p, blockIdx.x, blockIdx.y);
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

// Launch shape by the number of workgroups (heads x sequences): 16
// wavefronts up to 256 workgroups, 4 above; non-temporal state loads from
// 256 workgroups on.  The wavefront count is overridable with
// SPK_DECODE_WAVES=4|8|16 (measurement only).  Measured (us per launch,
// graph-timed over rotated copies, one box, B = 1 / 4 / 16 / 32 / 64 / 128 /
// 256 with 16 heads):
//   plain loads, 16 wavefronts  4.62 / 5.17 / 8.21 / 14.37 / 28.42 / 46.88 / 87.62
//   plain loads,  8 wavefronts  4.71 / 5.25 / 8.38 / 14.16 / 25.08 / 42.33 / 81.32
//   plain loads,  4 wavefronts  5.32 / 5.88 / 9.43 / 14.33 / 25.10 / 42.67 / 81.87
//   non-temporal, 16 wavefronts 4.94 / 5.75 / 8.00 / 13.56 / 25.48 / 44.19 / 84.54
//   non-temporal,  8 wavefronts 4.95 / 5.72 / 8.18 / 14.29 / 23.60 / 42.42 / 81.07
//   non-temporal,  4 wavefronts 5.71 / 6.59 / 9.21 / 13.51 / 23.76 / 42.91 / 81.22
// The reduction order depends on neither, so results are identical.
struct DecodeShape {
  int waves;
  bool nt_state;
};

DecodeShape decode_shape(int workgroups) {
  static const int forced = [] {
    const char* e = getenv("SPK_DECODE_WAVES");
    const int v = e ? atoi(e) : 0;
    return (v == 4 || v == 8 || v == 16) ? v : 0;
  }();
  const bool nt = workgroups >= 256;
  if (forced) return {forced, nt};
  return {workgroups <= 256 ? 16 : 4, nt};
}

template <bool CONV, bool REC, bool GB_TAIL, bool NORM_GATE, bool NT>
void launch_shape(int waves, dim3 grid, hipStream_t s, const DecodeParams& p) {
  if (waves == 16)
    hipLaunchKernelGGL((dn_decode_kernel<CONV, REC, GB_TAIL, NORM_GATE, 16, NT>), grid, dim3(1024), 0, s, p);
  else if (waves == 8)
    hipLaunchKernelGGL((dn_decode_kernel<CONV, REC, GB_TAIL, NORM_GATE, 8, NT>), grid, dim3(512), 0, s, p);
  else
    hipLaunchKernelGGL((dn_decode_kernel<CONV, REC, GB_TAIL, NORM_GATE, 4, NT>), grid, dim3(256), 0, s, p);
}

template <bool CONV, bool REC, bool GB_TAIL, bool NORM_GATE>
int launch(const SpkDecodeArgs* a, spk_stream_t stream, const char* name) {
  const int rc = validate(a, CONV, REC, REC && !GB_TAIL, REC && NORM_GATE);
  if (rc) return rc;
  if (a->batch == 0) return SPK_OK;
  dim3 grid(a->num_heads, a->batch);
  const DecodeShape sh = decode_shape(a->num_heads * a->batch);
  hipStream_t s = spk::to_hip(stream);
  if (sh.nt_state)
    launch_shape<CONV, REC, GB_TAIL, NORM_GATE, true>(sh.waves, grid, s, make_params(a));
  else
    launch_shape<CONV, REC, GB_TAIL, NORM_GATE, false>(sh.waves, grid, s, make_params(a));
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
