// dn_step.hpp -- one (head, sequence) DeltaNet recurrent decode step on one
// workgroup of WAVES wavefronts: the body of decode.hip's dn_decode_kernel,
// shared with the projection launch that runs the step of each head in its
// last-arriving workgroup (model.hip).
//
// One workgroup performs, with one read and one write of the head's 64 KiB
// fp32 state:
//   deltanet_conv_l2_qk.comp:41-111              conv-state shift, depthwise
//       conv (k=4) + SiLU, fp16 store, L2 of the Q and K head blocks;
//   deltanet_recurrent_gbeta_norm_gate.comp:91-225  g/beta, decay, kv=S^T k,
//       delta, rank-1 update, o=S^T q, RMSNorm, fp16(w*n)*SiLU(z).
// The state stream is the cost (2 x 64 KiB per head): each lane owns
// 16 / (WAVES / 4) consecutive rows x 4 columns, loaded as float4
// (global_load_dwordx4, row segments of 512 B per 32 lanes).  Every global
// load is issued at the start, so no phase after the conv waits on a memory
// round trip of its own.  g/beta (a chain of exp/log) is evaluated by the
// fourth wavefront while the first three run the conv.
//
// Reduction orders (fixed, and restated by the CPU oracle):
//   conv taps summed i = 0..3; L2 / RMS sums use the shaders' 128-wide tree
//   (s[l] += s[l+64], then 32..1: lane-local add, then wave shuffles);
//   S^T x per column: 32 row groups of 4 rows, fma-accumulated from 0 in row
//   order, then combined by a balanced pairwise tree (adjacent pairs first).
#pragma once

#include "capi_common.hpp"
#include "numerics.hpp"

namespace spk_dn {

struct DecodeParams {
  int nh;
  int layer;
  float q_scale;
  float eps;
  uint16_t* qkv;
  long long qkv_stride;
  uint16_t* conv_state;
  long long conv_stride;
  const uint16_t* conv_w;
  const uint16_t* a;
  const uint16_t* b;
  long long ab_stride;
  const float* alb;
  float* state;
  long long state_stride;
  const uint16_t* z;
  long long z_stride;
  const float* norm_w;
};

// Balanced pairwise tree over 32 partials in LDS column `col` of s_part
// (adjacent pairs first: level 1 sums (0,1), (2,3), ...).
__device__ __forceinline__ float tree32(const float (*part)[128], int col) {
  float v[32];
#pragma unroll
  for (int r = 0; r < 32; ++r) v[r] = part[r][col];
#pragma unroll
  for (int n = 32; n > 1; n >>= 1)
#pragma unroll
    for (int i = 0; i < n / 2; ++i) v[i] = v[2 * i] + v[2 * i + 1];
  return v[0];
}

// A value the compiler cannot see through (an empty asm that defines a
// VGPR): the starting value of an operand that only some waves load.
__device__ __forceinline__ uint32_t opaque_u32() {
  uint32_t v;
  asm volatile("" : "=v"(v));
  return v;
}

// CONV: run the conv/L2 phase.  REC: run the recurrence.  GB_TAIL: g/beta from
// the state tail (deltanet_recurrent.comp) instead of a/b/A_log/dt_bias.
// NORM_GATE: RMSNorm-gate the output (else fp16 of the raw output).
// AB_IN: the step's a and b inputs (fp16 bits) are the arguments a_in and
// b_in instead of p.a / p.b.  NT_STATE: read the state with non-temporal
// loads (faster once hundreds of workgroups stream states, slower for a few).
template <bool CONV, bool REC, bool GB_TAIL, bool NORM_GATE, int WAVES, bool AB_IN = false,
          bool NT_STATE = false>
__device__ __forceinline__ void dn_step(const DecodeParams& p, int h, int seq, uint16_t a_in = 0,
                                        uint16_t b_in = 0) {
  // G row groups of 4 rows per lane: 32 row groups over WAVES*2 lanes per column
  constexpr int G = 32 / (WAVES * 2);
  constexpr int M = 4 * G;  // rows per lane
  static_assert(WAVES == 4 || WAVES == 8 || WAVES == 16, "4, 8 or 16 wavefronts");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int nh = p.nh;
  uint16_t* qkv = p.qkv + (long long)seq * p.qkv_stride;

  __shared__ float s_q[128], s_k[128], s_v[128], s_delta[128];
  __shared__ float s_part[32][128];
  __shared__ float s_gb[2];
  __shared__ float s_zs[128];  // SiLU(z) of the norm-gate, formed off the chain

  const int c4 = tid & 31;  // owns columns 4*c4 .. 4*c4+3
  const int rq = tid >> 5;  // owns row groups G*rq .. G*rq+G-1, i.e. rows M*rq .. M*rq+M-1
  // Load order: the conv operands, then the small g/beta and norm-gate
  // operands, then the state.  A wave's loads return in issue order, so the
  // conv waves start on their operands while the state stream is still in
  // flight, and no later phase waits on a memory round trip of its own.  Each
  // small operand is loaded only by the wave that uses it (wave-uniform
  // branches; nothing loaded is merged with another value at a join, which
  // would make the compiler wait for the load there): all of a CU's loads go
  // through one memory pipe, and a head's batch-1 step is bound by how fast
  // that pipe takes them.
  // values a wave does not load are left unspecified (opaque_u32), not 0: a
  // constant on the other side of the branch lets the compiler fold the
  // conversions into the loading block, where they would wait for the loads
  uint2 olds[2], wvs[2];
  uint32_t xs[2];  // fp16 bits, one per register (a packed pair would be merged at the join)
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    olds[half] = make_uint2(opaque_u32(), opaque_u32());
    wvs[half] = make_uint2(opaque_u32(), opaque_u32());
    xs[half] = opaque_u32();
  }
  const int conv_blk = wave < 3 ? wave : 2;  // wave 0: Q block, 1: K block, 2: V block
  const int ch0 = conv_blk * nh * 128 + h * 128;
  uint16_t* cs_seq = CONV ? p.conv_state + (long long)seq * p.conv_stride : nullptr;
  if (CONV && wave < 3) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int ch = ch0 + lane + 64 * half;
      olds[half] = *reinterpret_cast<const uint2*>(cs_seq + ch * 4);
      wvs[half] = *reinterpret_cast<const uint2*>(p.conv_w + ch * 4);
      xs[half] = qkv[ch];
    }
  }
  constexpr int kSiluWave = WAVES > 4 ? 4 : 3;  // forms SiLU(z) during the conv phase
  uint16_t a16 = (uint16_t)opaque_u32(), b16 = (uint16_t)opaque_u32();
  float a_log = __uint_as_float(opaque_u32()), dt_bias = __uint_as_float(opaque_u32());
  float g_tail = 0.0f, beta_tail = 0.0f;
  uint16_t z16[2] = {(uint16_t)opaque_u32(), (uint16_t)opaque_u32()};
  float nw[2] = {__uint_as_float(opaque_u32()), __uint_as_float(opaque_u32())};
  if (REC) {
    if (GB_TAIL) {
      const float* tail = p.state + (long long)seq * p.state_stride + (long long)nh * 128 * 128;
      g_tail = tail[h];
      beta_tail = tail[nh + h];
    } else if (wave == 3) {
      if constexpr (AB_IN) {
        a16 = a_in;
        b16 = b_in;
      } else {
        a16 = p.a[(long long)seq * p.ab_stride + h];
        b16 = p.b[(long long)seq * p.ab_stride + h];
      }
      a_log = p.alb[(p.layer * nh + h) * 2];
      dt_bias = p.alb[(p.layer * nh + h) * 2 + 1];
    }
    if (NORM_GATE && wave == kSiluWave) {
      const uint16_t* zr = p.z + (long long)seq * p.z_stride + h * 128;
      z16[0] = zr[lane];
      z16[1] = zr[lane + 64];
    }
    if (NORM_GATE && wave == 0) {
      nw[0] = p.norm_w[lane];
      nw[1] = p.norm_w[lane + 64];
    }
  }
  float4 S[M];
  float* st_head = nullptr;
  if (REC) {
    st_head = p.state + (long long)seq * p.state_stride + (long long)h * 128 * 128;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float* src = st_head + (rq * M + m) * 128 + c4 * 4;
      if (NT_STATE) {
        typedef float f4v __attribute__((ext_vector_type(4)));
        const f4v t = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(src));
        S[m] = make_float4(t.x, t.y, t.z, t.w);
      } else {
        S[m] = *reinterpret_cast<const float4*>(src);
      }
    }
  }

  if (REC && !GB_TAIL && wave == 3) {
    // g/beta while waves 0-2 run the conv (deltanet_recurrent_gbeta_norm_gate.comp:102-116)
    if (lane == 0) {
      const float av = spk::h2f(a16);
      const float bv = spk::h2f(b16);
      const float sp = spk::logf_det(1.0f + spk::expf_det(av + dt_bias));
      s_gb[0] = -spk::expf_det(a_log) * sp;
      s_gb[1] = 1.0f / (1.0f + spk::expf_det(-bv));
    }
  }
  if (REC && NORM_GATE && wave == kSiluWave) {
    // the gate's SiLU(z) depends on nothing the step computes: an idle wave
    // (wave 4; wave 3 beside g/beta when there are only four) forms it while
    // waves 0-2 run the conv, so the output phase only reads it
    s_zs[lane] = spk::silu_det(spk::h2f(z16[0]));
    s_zs[lane + 64] = spk::silu_det(spk::h2f(z16[1]));
  }
  if (CONV) {
    if (wave < 3) {
      uint16_t y[2];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int ch = ch0 + lane + 64 * half;
        uint2* csp = reinterpret_cast<uint2*>(cs_seq + ch * 4);
        const uint2 old = olds[half];
        const uint2 wv = wvs[half];
        const uint16_t x = (uint16_t)xs[half];
        // shifted window (conv_l2_qk.comp:48-58): [old1, old2, old3, x]
        const uint16_t s0 = (uint16_t)(old.x >> 16);
        const uint16_t s1 = (uint16_t)(old.y & 0xffffu);
        const uint16_t s2 = (uint16_t)(old.y >> 16);
        const uint16_t s3 = x;
        *csp = make_uint2((uint32_t)s0 | ((uint32_t)s1 << 16), (uint32_t)s2 | ((uint32_t)s3 << 16));
        float sum = 0.0f;
        sum = sum + spk::h2f(s0) * spk::h2f((uint16_t)(wv.x & 0xffffu));
        sum = sum + spk::h2f(s1) * spk::h2f((uint16_t)(wv.x >> 16));
        sum = sum + spk::h2f(s2) * spk::h2f((uint16_t)(wv.y & 0xffffu));
        sum = sum + spk::h2f(s3) * spk::h2f((uint16_t)(wv.y >> 16));
        y[half] = spk::f2h(spk::silu_det(sum));
      }
      if (wave < 2) {
        const float ya = spk::h2f(y[0]);
        const float yb = spk::h2f(y[1]);
        float v = ya * ya + yb * yb;          // tree step stride 64
        v = spk::tree64_to_lane0(v);          // strides 32..1
        const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));  // lane 0 broadcast, no LDS
        const float inv = spk::rsqrt_det(tot + 1e-6f);
        y[0] = spk::f2h(ya * inv);
        y[1] = spk::f2h(yb * inv);
      }
      qkv[ch0 + lane] = y[0];
      qkv[ch0 + lane + 64] = y[1];
      if (REC) {
        if (wave == 0) {
          s_q[lane] = spk::h2f(y[0]) * p.q_scale;
          s_q[lane + 64] = spk::h2f(y[1]) * p.q_scale;
        } else if (wave == 1) {
          s_k[lane] = spk::h2f(y[0]);
          s_k[lane + 64] = spk::h2f(y[1]);
        } else {
          s_v[lane] = spk::h2f(y[0]);
          s_v[lane + 64] = spk::h2f(y[1]);
        }
      }
    }
  } else if (REC) {
    if (tid < 128) {
      s_q[tid] = spk::h2f(qkv[h * 128 + tid]) * p.q_scale;
      s_k[tid] = spk::h2f(qkv[nh * 128 + h * 128 + tid]);
      s_v[tid] = spk::h2f(qkv[2 * nh * 128 + h * 128 + tid]);
    }
  }
  if (!REC) return;

  __syncthreads();
  float g, beta;
  if (GB_TAIL) {
    g = g_tail;
    beta = beta_tail;
  } else {
    g = s_gb[0];
    beta = s_gb[1];
  }

  // decay + kv partials, one per 4-row group
  const float eg = spk::expf_det(g);
#pragma unroll
  for (int gq = 0; gq < G; ++gq) {
    float kp0 = 0.f, kp1 = 0.f, kp2 = 0.f, kp3 = 0.f;
#pragma unroll
    for (int m = 4 * gq; m < 4 * gq + 4; ++m) {
      const float ki = s_k[rq * M + m];
      S[m].x = S[m].x * eg;
      S[m].y = S[m].y * eg;
      S[m].z = S[m].z * eg;
      S[m].w = S[m].w * eg;
      kp0 = __builtin_fmaf(S[m].x, ki, kp0);
      kp1 = __builtin_fmaf(S[m].y, ki, kp1);
      kp2 = __builtin_fmaf(S[m].z, ki, kp2);
      kp3 = __builtin_fmaf(S[m].w, ki, kp3);
    }
    *reinterpret_cast<float4*>(&s_part[G * rq + gq][c4 * 4]) = make_float4(kp0, kp1, kp2, kp3);
  }
  __syncthreads();
  if (tid < 128) {
    const float kv = tree32(s_part, tid);
    s_delta[tid] = (s_v[tid] - kv) * beta;
  }
  __syncthreads();

  // rank-1 update, output partials per 4-row group
  const float4 d4 = *reinterpret_cast<const float4*>(&s_delta[c4 * 4]);
#pragma unroll
  for (int gq = 0; gq < G; ++gq) {
    float op0 = 0.f, op1 = 0.f, op2 = 0.f, op3 = 0.f;
#pragma unroll
    for (int m = 4 * gq; m < 4 * gq + 4; ++m) {
      const float ki = s_k[rq * M + m];
      const float qi = s_q[rq * M + m];
      S[m].x = __builtin_fmaf(ki, d4.x, S[m].x);
      S[m].y = __builtin_fmaf(ki, d4.y, S[m].y);
      S[m].z = __builtin_fmaf(ki, d4.z, S[m].z);
      S[m].w = __builtin_fmaf(ki, d4.w, S[m].w);
      op0 = __builtin_fmaf(S[m].x, qi, op0);
      op1 = __builtin_fmaf(S[m].y, qi, op1);
      op2 = __builtin_fmaf(S[m].z, qi, op2);
      op3 = __builtin_fmaf(S[m].w, qi, op3);
    }
    *reinterpret_cast<float4*>(&s_part[G * rq + gq][c4 * 4]) = make_float4(op0, op1, op2, op3);
  }
  __syncthreads();

  // state write-back after the last barrier: issued before it, the 64 KiB of
  // stores of a head held that barrier (and so the norm-gate) until the CU
  // had taken them all; here they drain while wavefront 0 (the oldest, so
  // its own stores issue first) runs the norm-gate
#pragma unroll
  for (int m = 0; m < M; ++m) *reinterpret_cast<float4*>(st_head + (rq * M + m) * 128 + c4 * 4) = S[m];
  if (wave == 0) {
    const float oa = tree32(s_part, lane);
    const float ob = tree32(s_part, lane + 64);
    uint16_t* out = qkv + 2 * nh * 128 + h * 128;
    if (NORM_GATE) {
      float v = oa * oa + ob * ob;
      v = spk::tree64_to_lane0(v);
      const float tot = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));  // lane 0 broadcast, no LDS
      const float r = spk::rsqrt_det(tot / 128.0f + p.eps);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int j = lane + 64 * half;
        const float o = half ? ob : oa;
        const float normed = o * r;
        const float weighted = spk::h2f(spk::f2h(nw[half] * normed));
        out[j] = spk::f2h(weighted * s_zs[j]);
      }
    } else {
      out[lane] = spk::f2h(oa);
      out[lane + 64] = spk::f2h(ob);
    }
  }
}

// Kernel parameters from the C ABI arguments (q_scale and eps default to
// 1/sqrt(128) and 1e-6 when zero).
inline DecodeParams make_params(const SpkDecodeArgs* a) {
  DecodeParams p;
  p.nh = a->num_heads;
  p.layer = a->layer_idx;
  p.q_scale = a->q_scale != 0.0f ? a->q_scale : 1.0f / sqrtf(128.0f);
  p.eps = a->rms_eps != 0.0f ? a->rms_eps : 1e-6f;
  p.qkv = a->qkv;
  p.qkv_stride = a->qkv_stride;
  p.conv_state = a->conv_state;
  p.conv_stride = a->conv_state_stride;
  p.conv_w = a->conv_weight;
  p.a = a->a;
  p.b = a->b;
  p.ab_stride = a->ab_stride;
  p.alb = a->a_log_bias;
  p.state = a->state;
  p.state_stride = a->state_stride;
  p.z = a->z;
  p.z_stride = a->z_stride;
  p.norm_w = a->norm_weight;
  return p;
}

}  // namespace spk_dn
