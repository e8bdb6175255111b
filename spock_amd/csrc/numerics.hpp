// numerics.hpp -- device-side scalar numerics shared by the decode, GEMV and
// chunk-prefill kernels.
//
// The decode step, the GEMVs and argmax must give the same bits as the CPU
// restatement of the reference shaders, so every transcendental below is a
// fixed sequence of IEEE operations (no hardware approximations):
//   exp: Cody-Waite reduction x = k ln2 + r with ln2 split in a 15-bit head and
//        a tail, then the degree-7 Taylor polynomial of e^r by Horner (fma),
//        then an exact ldexp.
//   log: x = m 2^e with m in [sqrt(1/2), sqrt(2)), s = (m-1)/(m+1),
//        log m = 2 atanh(s) = 2s(1 + s^2/3 + ... + s^10/11).
//   rsqrt: 1/sqrt(x) as two correctly rounded operations.
// All HIP sources are compiled with -ffp-contract=off, so a*b+c rounds twice
// unless __builtin_fmaf is written.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace spk {

__device__ __forceinline__ float h2f(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}

// IEEE round-to-nearest-even conversion (v_cvt_f16_f32 under the default mode)
// of an fp32 value.  The empty asm pins `f` as a materialised fp32 register:
// without it the backend folds a producing multiply or fma into the
// conversion (v_fma_mix*_f16), rounding the exact product once to fp16
// instead of first to fp32 -- a different result about once in 2^13.
__device__ __forceinline__ uint16_t f2h(float f) {
  asm volatile("" : "+v"(f));
  _Float16 v = (_Float16)f;
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}

// Truncating conversion with flush to zero, the reference's float_to_half
// (vk_session.cpp:69-89; deltanet_chunk_last_to_fp16.comp:45-74).
__device__ __forceinline__ uint16_t f2h_trunc(float f) {
  const uint32_t bits = __float_as_uint(f);
  const uint32_t sign = (bits >> 31) & 1u;
  const uint32_t exponent = (bits >> 23) & 0xffu;
  const uint32_t mantissa = bits & 0x7fffffu;
  const uint32_t hs = sign << 15;
  if (exponent == 0u) return (uint16_t)hs;
  if (exponent == 0xffu) return (uint16_t)(hs | 0x7c00u | (mantissa ? 0x200u : 0u));
  const int new_exp = (int)exponent - 127 + 15;
  if (new_exp <= 0) return (uint16_t)hs;
  if (new_exp >= 31) return (uint16_t)(hs | 0x7c00u);
  return (uint16_t)(hs | ((uint32_t)new_exp << 10) | (mantissa >> 13));
}

__device__ __forceinline__ float expf_det(float x) {
  if (x != x) return x;
  if (x > 88.7228394f) return __builtin_inff();
  if (x < -103.972084f) return 0.0f;
  const float t = x * 1.44269504f;
  const float kf = __builtin_rintf(t);
  float r = __builtin_fmaf(-kf, 0.693145751953125f, x);
  r = __builtin_fmaf(-kf, 1.42860677e-06f, r);
  float p = 1.98412698e-4f;
  p = __builtin_fmaf(p, r, 1.38888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)kf);
}

__device__ __forceinline__ float logf_det(float x) {
  if (x != x) return x;
  if (x < 0.0f) return __builtin_nanf("");
  if (x == 0.0f) return -__builtin_inff();
  if (x == __builtin_inff()) return x;
  int e;
  float m = __builtin_frexpf(x, &e);
  if (m < 0.707106781f) { m = m * 2.0f; e -= 1; }
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float p = 9.09090909e-2f;
  p = __builtin_fmaf(p, s2, 1.11111111e-1f);
  p = __builtin_fmaf(p, s2, 1.42857143e-1f);
  p = __builtin_fmaf(p, s2, 2.0e-1f);
  p = __builtin_fmaf(p, s2, 3.33333333e-1f);
  const float ls = 2.0f * s;
  const float lm = __builtin_fmaf(ls * s2, p, ls);
  const float ef = (float)e;
  return __builtin_fmaf(ef, 0.693145751953125f, __builtin_fmaf(ef, 1.42860677e-06f, lm));
}

__device__ __forceinline__ float rsqrt_det(float x) { return 1.0f / __builtin_sqrtf(x); }

__device__ __forceinline__ float silu_det(float x) { return x / (1.0f + expf_det(-x)); }

// v <- v + (v of lane l + S), for lanes whose partner lies in the same row of
// 16 lanes (DPP row_shl:S); other lanes receive values no later level reads.
template <int S>
__device__ __forceinline__ float add_row_shl(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + S, 0xF, 0xF, true));
}

// Lanes 0..31 receive lane l+32's value (v_permlane32_swap of v with itself:
// a VALU lane exchange, no LDS round trip); lanes 32..63 keep their own.
__device__ __forceinline__ float lanes_down32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[1]);
}

// Lanes 0..15 (and 32..47) receive lane l+16's value (v_permlane16_swap);
// lanes 16..31 and 48..63 keep their own.
__device__ __forceinline__ float lanes_down16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[1]);
}

// Exact xor exchanges without LDS: lane l receives lane (l ^ m)'s value.
// 32 and 16 from the permlane swaps (r[1] is the lower half's / even rows'
// partner value, r[0] the upper half's / odd rows'), 8 as a DPP rotation by 8
// within the 16-lane row, 2 and 1 as DPP quad permutations.
__device__ __forceinline__ uint32_t lane_xor32_u(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (threadIdx.x & 32) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t lane_xor16_u(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  return (threadIdx.x & 16) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t lane_xor8_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xF, 0xF, false);  // row_ror:8
}
__device__ __forceinline__ uint32_t lane_xor2_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
}
__device__ __forceinline__ uint32_t lane_xor1_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
}
__device__ __forceinline__ float lane_xor32(float v) { return __uint_as_float(lane_xor32_u(__float_as_uint(v))); }
__device__ __forceinline__ float lane_xor16(float v) { return __uint_as_float(lane_xor16_u(__float_as_uint(v))); }
__device__ __forceinline__ float lane_xor8(float v) { return __uint_as_float(lane_xor8_u(__float_as_uint(v))); }
__device__ __forceinline__ float lane_xor2(float v) { return __uint_as_float(lane_xor2_u(__float_as_uint(v))); }
__device__ __forceinline__ float lane_xor1(float v) { return __uint_as_float(lane_xor1_u(__float_as_uint(v))); }

// Lane l receives the value of lane (l - S) mod 16 of its row (DPP row_ror:S).
template <int S>
__device__ __forceinline__ uint32_t row_ror_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x120 + S, 0xF, 0xF, false);
}

// Maximum over the 16 lanes of each row, in every lane (max is exact, so the
// rotation pattern gives the same value as any other complete reduction).
__device__ __forceinline__ float row_max16(float m) {
  m = fmaxf(m, __uint_as_float(row_ror_u<8>(__float_as_uint(m))));
  m = fmaxf(m, __uint_as_float(row_ror_u<4>(__float_as_uint(m))));
  m = fmaxf(m, __uint_as_float(row_ror_u<2>(__float_as_uint(m))));
  m = fmaxf(m, __uint_as_float(row_ror_u<1>(__float_as_uint(m))));
  return m;
}
// ... over each half wave (32 lanes) and over the whole wave, in every lane.
__device__ __forceinline__ float half_wave_max(float m) { return row_max16(fmaxf(m, lane_xor16(m))); }
__device__ __forceinline__ float wave_max(float m) { return half_wave_max(fmaxf(m, lane_xor32(m))); }

// 64-lane tree s[l] += s[l+stride], stride 32..1; the sum ends in lane 0
// (other lanes hold partial sums no caller reads).  Strides 32 and 16 by lane
// swaps, 8..1 as DPP row shifts: no LDS permute on the chain.  Every lane of
// the wave must be active.
__device__ __forceinline__ float tree64_to_lane0(float v) {
  v = v + lanes_down32(v);
  v = v + lanes_down16(v);
  v = add_row_shl<8>(v);
  v = add_row_shl<4>(v);
  v = add_row_shl<2>(v);
  v = add_row_shl<1>(v);
  return v;
}

// N independent 64-lane trees s[l] += s[l+stride], stride 32..1 (the order of
// tree64_to_lane0), interleaved level by level.  Sums end in lane 0; every
// lane of the wave must be active.
template <int N>
__device__ __forceinline__ void tree64_rows(float (&v)[N]) {
  float t[N];
#pragma unroll
  for (int i = 0; i < N; ++i) t[i] = lanes_down32(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = v[i] + t[i];
#pragma unroll
  for (int i = 0; i < N; ++i) t[i] = lanes_down16(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = v[i] + t[i];
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = add_row_shl<8>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = add_row_shl<4>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = add_row_shl<2>(v[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = add_row_shl<1>(v[i]);
}

}  // namespace spk
