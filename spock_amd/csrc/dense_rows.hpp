// dense_rows.hpp -- fp16 matrix rows loaded densely, regrouped into the
// lane order of lm_head_tiled.comp:46-62 (lane l owns the 8*N8 contiguous
// elements [8*N8*l, 8*N8*(l+1)) of a row of 512*N8).
//
// Loading each lane's N8 16-byte pieces directly (piece N8*l + k in load k)
// puts consecutive lanes 16*N8 bytes apart, so every load instruction of a
// wavefront touches all 4*N8 cache lines of the 1 KiB*N8 row at 1/N8
// density, and each line is requested N8 times.  Here load k of a row reads
// pieces 64k .. 64k+63 instead (1 KiB contiguous, 8 whole lines per
// instruction), and the wavefront exchanges the pieces through LDS: every
// lane writes the pieces it loaded in row order, then reads back its own N8.
// The products are then summed exactly as before (results bit-identical).
// Measured on MI355X over the 248320 x 1024 lm_head matrix, 4 rows per
// wavefront, non-temporal loads: 83.9 -> 72.9 us per GEMV.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace spk {

typedef uint32_t dense_u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ uint4 dense_ld(const uint4* p) {
  if constexpr (NT) {
    const dense_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const dense_u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *p;
  }
}

// Issue the loads of rows row0 .. row0+R-1 (rows past out_dim re-read the
// last row; callers discard their sums): wv[r][k] = piece 64k + lane.
template <int N8, int R, bool NT>
__device__ __forceinline__ void dense_rows_issue(const uint16_t* __restrict__ W, int row0, int out_dim,
                                                 int lane, uint4 (&wv)[R][N8]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r < out_dim ? row0 + r : out_dim - 1;
    const uint4* src = reinterpret_cast<const uint4*>(W + (size_t)row * (512 * N8)) + lane;
#pragma unroll
    for (int k = 0; k < N8; ++k) wv[r][k] = dense_ld<NT>(src + 64 * k);
  }
}

// Regroup through the wavefront's own LDS area of one row (64 * N8 pieces,
// N8 KiB), row by row: on return wv[r][k] = piece N8*lane + k of row r.
// Only this wavefront touches `lds`; LDS operations of a wavefront execute
// in order, and the fences keep the compiler from moving them across the
// wave barrier.
template <int N8, int R>
__device__ __forceinline__ void dense_rows_regroup(uint4 (&wv)[R][N8], uint4* lds, int lane) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
#pragma unroll
    for (int k = 0; k < N8; ++k) lds[k * 64 + lane] = wv[r][k];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int k = 0; k < N8; ++k) wv[r][k] = lds[N8 * lane + k];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

}  // namespace spk
