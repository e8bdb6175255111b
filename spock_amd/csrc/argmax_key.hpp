// argmax_key.hpp -- argmax.comp:27-63 as a 64-bit key whose maximum is the
// shader's winner, so any reduction order (waves, workgroups, device-scope
// atomic max) gives the shader's index.
//
// With E = ceil(N/256) and element i in "lane" i/E, the shader keeps the first
// strict maximum inside each lane and a strictly-greater tree across lanes, so
// among equal maxima the winner is the lane with the smallest 8-bit-reversed
// lane id, then the smallest offset.  The key is (ordered value, rank) with
// that order; 0 never wins (NaN and -inf fail v > -FLT_MAX in the shader).
#pragma once

#include <float.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "numerics.hpp"

namespace spk {

__device__ __forceinline__ uint32_t ordered_f32(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7fffffffu) == 0u) u = 0u;  // +0 and -0 tie in argmax.comp
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Key of element idx with value v; 0 = never wins (NaN, -inf: fails v > -FLT_MAX).
__device__ __forceinline__ unsigned long long argmax_key(float v, uint32_t idx, uint32_t E) {
  if (!(v > -FLT_MAX)) return 0ull;
  const uint32_t lane = idx / E;
  const uint32_t off = idx - lane * E;
  const uint32_t rev = __builtin_bitreverse32(lane) >> 24;
  const uint32_t rank = ((255u - rev) << 24) | (0xffffffu - off);
  return ((unsigned long long)ordered_f32(v) << 32) | rank;
}

__device__ __forceinline__ uint32_t key_to_index(unsigned long long key, uint32_t E) {
  if (key == 0ull) return 0u;
  const uint32_t rank = (uint32_t)key;
  const uint32_t rev = 255u - (rank >> 24);
  const uint32_t lane = __builtin_bitreverse32(rev) >> 24;
  const uint32_t off = 0xffffffu - (rank & 0xffffffu);
  return lane * E + off;
}

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}

// Maximum over the wave, in every lane: lane swaps across the halves and
// rows, then DPP rotations inside each 16-lane row (max is exact, so any
// complete pattern gives the same key).  Every lane must be active.
__device__ __forceinline__ unsigned long long join64(uint32_t hi, uint32_t lo) {
  return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
  v = umax64(v, join64(lane_xor32_u((uint32_t)(v >> 32)), lane_xor32_u((uint32_t)v)));
  v = umax64(v, join64(lane_xor16_u((uint32_t)(v >> 32)), lane_xor16_u((uint32_t)v)));
  v = umax64(v, join64(row_ror_u<8>((uint32_t)(v >> 32)), row_ror_u<8>((uint32_t)v)));
  v = umax64(v, join64(row_ror_u<4>((uint32_t)(v >> 32)), row_ror_u<4>((uint32_t)v)));
  v = umax64(v, join64(row_ror_u<2>((uint32_t)(v >> 32)), row_ror_u<2>((uint32_t)v)));
  v = umax64(v, join64(row_ror_u<1>((uint32_t)(v >> 32)), row_ror_u<1>((uint32_t)v)));
  return v;
}

template <int NT>
__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long v) {
  __shared__ unsigned long long s_red[NT / 64];
  v = wave_max_u64(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) s_red[wave] = v;
  __syncthreads();
  unsigned long long r = 0ull;
#pragma unroll
  for (int w = 0; w < NT / 64; ++w) r = umax64(r, s_red[w]);
  return r;
}

}  // namespace spk
