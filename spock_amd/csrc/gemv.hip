// gemv.hip -- batch-1 fp16 decode GEMV, tied lm_head fused with argmax, and a
// standalone argmax.  All are HBM streams (weights read once); no MFMA.
//
// One wavefront per output row at a time, R rows in flight per wavefront.
// Lane l sums the contiguous span [l*in/64, (l+1)*in/64) of the row
// (fp16*fp16 products, exact in fp32, in span order), then the 64-lane tree
// s[l] += s[l+stride] for stride 32..1 -- lm_head_tiled.comp:59-73's order --
// and rounds once to fp16 (RNE).  Decode-sized matrices load each lane's span
// directly with 16-byte loads (in=1024: 2 x dwordx4 per lane); the lm_head
// and other matrices of hundreds of MB load rows densely (1 KiB of a row per
// instruction) and regroup the pieces through LDS (dense_rows.hpp).
// spk_matvec_f16_order adds the reference's two other orders, matvec.comp's
// serial sum and matvec_tiled.comp's lane-strided one.
//
// Argmax keeps argmax.comp:27-63's exact result, including its tie rule, as
// the 64-bit keys of argmax_key.hpp.
#include "argmax_key.hpp"
#include "capi_common.hpp"
#include "dense_rows.hpp"
#include "numerics.hpp"

#include <float.h>

#include <mutex>

namespace {

using spk::argmax_key;
using spk::block_max_u64;
using spk::key_to_index;
using spk::umax64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Decode-sized matrices (a few MB) are read with plain (cached) 16-byte
// loads: non-temporal loads measured up to 2x slower there on MI355X.  The
// 0.5 GB lm_head stream is the opposite case and keeps non-temporal loads.
__device__ __forceinline__ uint4 ld_w(const uint4* p) { return *p; }
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void unpack8(const uint4& u, float* f) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = spk::h2f((uint16_t)(w[i] & 0xffffu));
    f[2 * i + 1] = spk::h2f((uint16_t)(w[i] >> 16));
  }
}

// Dot products of R rows (row0..row0+R-1, clipped to out_dim) with x; lane 0
// of the wave returns the fp32 sums.
template <int N8, int R, bool STREAM = false>
__device__ __forceinline__ void rows_dot(const uint16_t* __restrict__ W, int in_dim, int row0,
                                         int out_dim, const float* xf, int lane, float* sums) {
  // rows past out_dim re-read the last row (no load under a branch); callers
  // discard their sums
  uint4 wv[R][N8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(row0 + r, out_dim - 1);
    const uint4* src = reinterpret_cast<const uint4*>(W + (size_t)row * in_dim + lane * (8 * N8));
#pragma unroll
    for (int k = 0; k < N8; ++k) wv[r][k] = STREAM ? ld_stream(src + k) : ld_w(src + k);
  }
  // all R*N8 loads in flight before any use (else the scheduler trades
  // bytes in flight for registers)
  __builtin_amdgcn_sched_barrier(0);
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < N8; ++k) {
      float wf[8];
      unpack8(wv[r][k], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[r] = __builtin_fmaf(wf[e], xf[8 * k + e], acc[r]);
    }
  }
  spk::tree64_rows<R>(acc);
#pragma unroll
  for (int r = 0; r < R; ++r) sums[r] = acc[r];
}

template <int N8>
__device__ __forceinline__ void load_x(const uint16_t* __restrict__ x, int lane, float* xf) {
  const uint4* src = reinterpret_cast<const uint4*>(x + lane * (8 * N8));
#pragma unroll
  for (int k = 0; k < N8; ++k) unpack8(src[k], xf + 8 * k);
}

template <int N8, int R>
__global__ __launch_bounds__(256) void gemv_kernel(const uint16_t* __restrict__ W,
                                                   const uint16_t* __restrict__ x,
                                                   uint16_t* __restrict__ y, int out_dim) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int in_dim = 512 * N8;
  float xf[8 * N8];
  load_x<N8>(x, lane, xf);
  const int row0 = (blockIdx.x * 4 + wave) * R;
  float sums[R];
  rows_dot<N8, R>(W, in_dim, row0, out_dim, xf, lane, sums);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (row0 + r < out_dim) y[row0 + r] = spk::f2h(sums[r]);
  }
}

// Matrices of hundreds of MB (the lm_head class): 4 rows per wavefront read
// with dense non-temporal loads and regrouped into the span order
// (dense_rows.hpp); the same sums as gemv_kernel.
constexpr size_t kStreamBytes = size_t(128) << 20;
template <int N8>
__global__ __launch_bounds__(256) void gemv_stream_kernel(const uint16_t* __restrict__ W,
                                                          const uint16_t* __restrict__ x,
                                                          uint16_t* __restrict__ y, int out_dim) {
  constexpr int R = 4;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float xf[8 * N8];
  load_x<N8>(x, lane, xf);
  const int row0 = (blockIdx.x * 4 + wave) * R;
  __shared__ uint4 rows_lds[4][64 * N8];
  uint4 wv[R][N8];
  spk::dense_rows_issue<N8, R, true>(W, row0, out_dim, lane, wv);
  __builtin_amdgcn_sched_barrier(0);  // every row in flight before the regroup
  spk::dense_rows_regroup<N8, R>(wv, rows_lds[wave], lane);
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < N8; ++k) {
      float wf[8];
      unpack8(wv[r][k], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[r] = __builtin_fmaf(wf[e], xf[8 * k + e], acc[r]);
    }
  }
  spk::tree64_rows<R>(acc);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (row0 + r < out_dim) y[row0 + r] = spk::f2h(acc[r]);
  }
}

// Any in_dim % 64 == 0: scalar loads, same order.
__global__ __launch_bounds__(256) void gemv_generic_kernel(const uint16_t* __restrict__ W,
                                                           const uint16_t* __restrict__ x,
                                                           uint16_t* __restrict__ y, int out_dim,
                                                           int in_dim) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= out_dim) return;
  const int span = in_dim / 64;
  const uint16_t* wr = W + (size_t)row * in_dim + lane * span;
  const uint16_t* xr = x + lane * span;
  float acc = 0.0f;
  for (int j = 0; j < span; ++j) acc = __builtin_fmaf(spk::h2f(wr[j]), spk::h2f(xr[j]), acc);
  acc = spk::tree64_to_lane0(acc);
  if (lane == 0) y[row] = spk::f2h(acc);
}

template <int N8, int R>
__global__ __launch_bounds__(256) void lm_head_kernel(const uint16_t* __restrict__ W,
                                                      const uint16_t* __restrict__ x,
                                                      uint16_t* __restrict__ logits, int vocab,
                                                      uint32_t E,
                                                      unsigned long long* __restrict__ partial) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float xf[8 * N8];
  load_x<N8>(x, lane, xf);
  const int row0 = (blockIdx.x * 4 + wave) * R;
  // rows loaded densely and regrouped into the span order (dense_rows.hpp)
  __shared__ uint4 rows_lds[4][64 * N8];
  uint4 wv[R][N8];
  spk::dense_rows_issue<N8, R, true>(W, row0, vocab, lane, wv);
  __builtin_amdgcn_sched_barrier(0);  // every row in flight before the regroup
  spk::dense_rows_regroup<N8, R>(wv, rows_lds[wave], lane);
  float sums[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    sums[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < N8; ++k) {
      float wf[8];
      unpack8(wv[r][k], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) sums[r] = __builtin_fmaf(wf[e], xf[8 * k + e], sums[r]);
    }
  }
  spk::tree64_rows<R>(sums);
  unsigned long long key = 0ull;
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      if (row < vocab) {
        const uint16_t l16 = spk::f2h(sums[r]);
        if (logits) logits[row] = l16;
        key = umax64(key, argmax_key(spk::h2f(l16), (uint32_t)row, E));
      }
    }
  }
  key = block_max_u64<256>(key);
  if (threadIdx.x == 0) partial[blockIdx.x] = key;
}

__global__ __launch_bounds__(1024) void argmax_partials_kernel(const unsigned long long* __restrict__ partial,
                                                               int n, uint32_t E,
                                                               uint32_t* __restrict__ out) {
  unsigned long long key = 0ull;
  for (int i = threadIdx.x; i < n; i += 1024) key = umax64(key, partial[i]);
  key = block_max_u64<1024>(key);
  if (threadIdx.x == 0) *out = key_to_index(key, E);
}

__global__ __launch_bounds__(1024) void argmax_kernel(const uint16_t* __restrict__ vals, int n,
                                                      uint32_t E, uint32_t* __restrict__ out) {
  unsigned long long key = 0ull;
  for (int i = threadIdx.x; i < n; i += 1024)
    key = umax64(key, argmax_key(spk::h2f(vals[i]), (uint32_t)i, E));
  key = block_max_u64<1024>(key);
  if (threadIdx.x == 0) *out = key_to_index(key, E);
}

// Several GEMVs in one launch: workgroup ranges are assigned to descriptors by
// prefix sums; each workgroup runs 4 wavefronts x batch_rows(n8) rows of one
// descriptor with the same per-row order as gemv_kernel (bit-identical
// results).  A wavefront issues all of its weight loads (batch_rows rows x
// n8 16-byte loads per lane) before it reads x; one or two rows per
// wavefront (many workgroups) measured fastest for decode-sized projections.
constexpr int kMaxBatch = 4;
__host__ __device__ constexpr int batch_rows(int n8) { return n8 <= 2 ? 2 : 1; }
struct GemvBatch {
  const uint16_t* W[kMaxBatch];
  const uint16_t* x[kMaxBatch];
  uint16_t* y[kMaxBatch];
  int out_dim[kMaxBatch];
  int n8[kMaxBatch];
  int first_block[kMaxBatch + 1];
  int count;
};

template <int N8>
__device__ __forceinline__ void batched_rows(const uint16_t* __restrict__ W, const uint16_t* __restrict__ x,
                                             uint16_t* __restrict__ y, int out_dim, int blk, int wave,
                                             int lane) {
  constexpr int R = batch_rows(N8);
  constexpr int in_dim = 512 * N8;
  const int row0 = (blk * 4 + wave) * R;
  // x first (a wave's loads complete in issue order, so the dot can start on
  // the first weight row to arrive), then the weight rows
  uint4 xr[N8];
  const uint4* xsrc = reinterpret_cast<const uint4*>(x + lane * (8 * N8));
#pragma unroll
  for (int k = 0; k < N8; ++k) xr[k] = xsrc[k];
  uint4 wv[R][N8];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r < out_dim ? row0 + r : out_dim - 1;
    const uint4* src = reinterpret_cast<const uint4*>(W + (size_t)row * in_dim + lane * (8 * N8));
#pragma unroll
    for (int k = 0; k < N8; ++k) wv[r][k] = ld_w(src + k);
  }
  __builtin_amdgcn_sched_barrier(0);  // all loads in flight before any use
  float xf[8 * N8];
#pragma unroll
  for (int k = 0; k < N8; ++k) unpack8(xr[k], xf + 8 * k);
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < N8; ++k) {
      float wf[8];
      unpack8(wv[r][k], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[r] = __builtin_fmaf(wf[e], xf[8 * k + e], acc[r]);
    }
  }
  spk::tree64_rows<R>(acc);
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (lane == 0 && row0 + r < out_dim) y[row0 + r] = spk::f2h(acc[r]);
}

__global__ __launch_bounds__(256) void gemv_batched_kernel(GemvBatch b) {
  // Every descriptor is read and the workgroup's one selected by value, so
  // all kernel-argument loads go out in one round trip (indexing the arrays
  // by the selected d would wait for first_block before loading W, x, y).
  const uint16_t* W = b.W[0];
  const uint16_t* x = b.x[0];
  uint16_t* y = b.y[0];
  int out_dim = b.out_dim[0], n8 = b.n8[0], fb = 0;
#pragma unroll
  for (int i = 1; i < kMaxBatch; ++i) {
    const bool take = i < b.count && (int)blockIdx.x >= b.first_block[i];
    W = take ? b.W[i] : W;
    x = take ? b.x[i] : x;
    y = take ? b.y[i] : y;
    out_dim = take ? b.out_dim[i] : out_dim;
    n8 = take ? b.n8[i] : n8;
    fb = take ? b.first_block[i] : fb;
  }
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int blk = (int)blockIdx.x - fb;
  switch (n8) {
#define SPK_BATCH_CASE(n8_) \
  case n8_: batched_rows<n8_>(W, x, y, out_dim, blk, wave, lane); break;
    SPK_BATCH_CASE(1)
    SPK_BATCH_CASE(2)
    SPK_BATCH_CASE(3)
    SPK_BATCH_CASE(4)
    SPK_BATCH_CASE(5)
    SPK_BATCH_CASE(6)
    SPK_BATCH_CASE(7)
    default: batched_rows<8>(W, x, y, out_dim, blk, wave, lane); break;
#undef SPK_BATCH_CASE
  }
}

// matvec_tiled.comp:41-84's order: lane l sums j = l, l+64, l+128, ... < in_dim
// sequentially (fp32, from 0), then the 64-lane tree s[l] += s[l+stride] for
// stride 32..1; any in_dim.  One wavefront per R rows; each load instruction
// reads 64 consecutive fp16 of a row (128 coalesced bytes), U steps of every
// row in flight before the first is used.  Past in_dim a lane's index is
// clamped and its product not added.
template <int R, bool NT>
__global__ __launch_bounds__(256) void gemv_strided_kernel(const uint16_t* __restrict__ W,
                                                           const uint16_t* __restrict__ x,
                                                           uint16_t* __restrict__ y, int out_dim,
                                                           int in_dim) {
  constexpr int U = 8;
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  if (row0 >= out_dim) return;  // wave-uniform: the whole wavefront leaves
  const int steps = (in_dim + 63) / 64;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  for (int i0 = 0; i0 < steps; i0 += U) {
    uint16_t wv[R][U], xv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = min(lane + 64 * (i0 + u), in_dim - 1);
      xv[u] = x[j];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint16_t* p = W + (size_t)min(row0 + r, out_dim - 1) * in_dim + j;
        wv[r][u] = NT ? __builtin_nontemporal_load(p) : *p;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool valid = lane + 64 * (i0 + u) < in_dim;
      const float xf = spk::h2f(xv[u]);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float t = __builtin_fmaf(spk::h2f(wv[r][u]), xf, acc[r]);
        acc[r] = valid ? t : acc[r];
      }
    }
  }
  spk::tree64_rows<R>(acc);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (row0 + r < out_dim) y[row0 + r] = spk::f2h(acc[r]);
  }
}

// matvec.comp:28-41's order: one lane per row, j = 0 .. in_dim-1 sequentially
// (fp32, from 0).  Needs in_dim % 64 == 0 and 16-byte aligned W and x: each
// wavefront owns 64 rows and walks them in 64-column tiles, read
// row-coalesced (8 lanes x 16 B per 128-byte row segment, next tile's loads
// issued before this tile's products) into LDS, where each lane then reads its
// own row (rows padded by one dword, so the 64 lanes' reads hit 64 banks).
template <bool NT>
__global__ __launch_bounds__(256) void gemv_serial_kernel(const uint16_t* __restrict__ W,
                                                          const uint16_t* __restrict__ x,
                                                          uint16_t* __restrict__ y, int out_dim,
                                                          int in_dim) {
  __shared__ uint32_t tile[4][64][33];
  __shared__ float xs[4][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int row_base = (blockIdx.x * 4 + wave) * 64;
  const int sub = lane & 7;   // 16-byte piece of a 128-byte row segment
  const int rr = lane >> 3;   // rows rr, rr+8, ..., rr+56 of the tile
  const uint16_t* src[8];
#pragma unroll
  for (int q = 0; q < 8; ++q)
    src[q] = W + (size_t)min(row_base + rr + 8 * q, out_dim - 1) * in_dim + 8 * sub;
  const int tiles = in_dim / 64;
  uint4 v[8];
  uint16_t xv;
#pragma unroll
  for (int q = 0; q < 8; ++q) v[q] = spk::dense_ld<NT>(reinterpret_cast<const uint4*>(src[q]));
  xv = x[lane];
  float acc = 0.0f;
  for (int c = 0; c < tiles; ++c) {
    __syncthreads();  // every lane is done reading the previous tile
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      uint32_t* t = &tile[wave][rr + 8 * q][4 * sub];
      t[0] = v[q].x;
      t[1] = v[q].y;
      t[2] = v[q].z;
      t[3] = v[q].w;
    }
    xs[wave][lane] = spk::h2f(xv);
    __syncthreads();
    if (c + 1 < tiles) {  // next tile in flight while this one is summed
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = spk::dense_ld<NT>(reinterpret_cast<const uint4*>(src[q] + 64 * (c + 1)));
      xv = x[64 * (c + 1) + lane];
    }
#pragma unroll
    for (int j2 = 0; j2 < 32; ++j2) {
      const uint32_t d = tile[wave][lane][j2];
      acc = __builtin_fmaf(spk::h2f((uint16_t)(d & 0xffffu)), xs[wave][2 * j2], acc);
      acc = __builtin_fmaf(spk::h2f((uint16_t)(d >> 16)), xs[wave][2 * j2 + 1], acc);
    }
  }
  if (row_base + lane < out_dim) y[row_base + lane] = spk::f2h(acc);
}

// The same order for any in_dim and alignment: one lane per row, fp16 loads.
__global__ __launch_bounds__(256) void gemv_serial_generic_kernel(const uint16_t* __restrict__ W,
                                                                  const uint16_t* __restrict__ x,
                                                                  uint16_t* __restrict__ y,
                                                                  int out_dim, int in_dim) {
  const int row = blockIdx.x * 256 + threadIdx.x;
  if (row >= out_dim) return;
  const uint16_t* wr = W + (size_t)row * in_dim;
  float acc = 0.0f;
  for (int j = 0; j < in_dim; ++j) acc = __builtin_fmaf(spk::h2f(wr[j]), spk::h2f(x[j]), acc);
  y[row] = spk::f2h(acc);
}

constexpr int kLmRows = 4;  // rows per wavefront in the lm_head stream

int launch_gemv(const uint16_t* W, const uint16_t* x, uint16_t* y, int out_dim, int in_dim,
                hipStream_t s) {
  const bool vec = (in_dim % 512 == 0) && in_dim <= 8 * 512 && spk::aligned(W, 16) &&
                   spk::aligned(x, 16);
  if (!vec) {
    hipLaunchKernelGGL(gemv_generic_kernel, dim3((out_dim + 3) / 4), dim3(256), 0, s, W, x, y,
                       out_dim, in_dim);
    return spk::check_launch("spk_matvec_f16 (generic)");
  }
  if ((size_t)out_dim * (size_t)in_dim * 2 >= kStreamBytes) {
    const dim3 g((out_dim + 15) / 16);
    switch (in_dim / 512) {
#define SPK_GEMV_STREAM_CASE(n8) \
  case n8: hipLaunchKernelGGL((gemv_stream_kernel<n8>), g, dim3(256), 0, s, W, x, y, out_dim); break;
      SPK_GEMV_STREAM_CASE(1)
      SPK_GEMV_STREAM_CASE(2)
      SPK_GEMV_STREAM_CASE(3)
      SPK_GEMV_STREAM_CASE(4)
      SPK_GEMV_STREAM_CASE(5)
      SPK_GEMV_STREAM_CASE(6)
      SPK_GEMV_STREAM_CASE(7)
      default: hipLaunchKernelGGL((gemv_stream_kernel<8>), g, dim3(256), 0, s, W, x, y, out_dim); break;
#undef SPK_GEMV_STREAM_CASE
    }
    return spk::check_launch("spk_matvec_f16 (stream)");
  }
  // Rows per wave: enough workgroups to cover the chip for small outputs,
  // more bytes in flight per lane for large ones.
  const int R = out_dim >= 16384 ? 4 : 1;
  const int rows_per_block = 4 * R;
  dim3 grid((out_dim + rows_per_block - 1) / rows_per_block);
#define SPK_GEMV_CASE(n8)                                                                      \
  case n8:                                                                                     \
    if (R == 4)                                                                                \
      hipLaunchKernelGGL((gemv_kernel<n8, 4>), grid, dim3(256), 0, s, W, x, y, out_dim);       \
    else                                                                                       \
      hipLaunchKernelGGL((gemv_kernel<n8, 1>), grid, dim3(256), 0, s, W, x, y, out_dim);       \
    break;
  switch (in_dim / 512) {
    SPK_GEMV_CASE(1)
    SPK_GEMV_CASE(2)
    SPK_GEMV_CASE(3)
    SPK_GEMV_CASE(4)
    SPK_GEMV_CASE(5)
    SPK_GEMV_CASE(6)
    SPK_GEMV_CASE(7)
    SPK_GEMV_CASE(8)
    default:
      return spk::fail(SPK_ERR_SHAPE, "spk_matvec_f16: in_dim %d", in_dim);
  }
#undef SPK_GEMV_CASE
  return spk::check_launch("spk_matvec_f16");
}

int check_gemv(const uint16_t* W, const uint16_t* x, const uint16_t* y, int out_dim, int in_dim,
               const char* who) {
  if (!W || !x || !y) return spk::fail(SPK_ERR_NULL, "%s: NULL pointer", who);
  if (out_dim < 0 || in_dim <= 0 || in_dim % 64 != 0)
    return spk::fail(SPK_ERR_SHAPE, "%s: out_dim %d in_dim %d (in_dim must be a positive multiple of 64)",
                     who, out_dim, in_dim);
  return SPK_OK;
}

}  // namespace

extern "C" int spk_matvec_f16(const uint16_t* W, const uint16_t* x, uint16_t* y, int32_t out_dim,
                              int32_t in_dim, spk_stream_t stream) {
  const int rc = check_gemv(W, x, y, out_dim, in_dim, "spk_matvec_f16");
  if (rc) return rc;
  if (out_dim == 0) return SPK_OK;
  return launch_gemv(W, x, y, out_dim, in_dim, spk::to_hip(stream));
}

extern "C" int spk_matvec_f16_order(const uint16_t* W, const uint16_t* x, uint16_t* y,
                                    int32_t out_dim, int32_t in_dim, int32_t order,
                                    spk_stream_t stream) {
  const char* who = "spk_matvec_f16_order";
  if (order == SPK_MATVEC_ORDER_SPANS) return spk_matvec_f16(W, x, y, out_dim, in_dim, stream);
  if (order != SPK_MATVEC_ORDER_STRIDED && order != SPK_MATVEC_ORDER_SERIAL)
    return spk::fail(SPK_ERR_ARG, "%s: unknown order %d", who, order);
  if (!W || !x || !y) return spk::fail(SPK_ERR_NULL, "%s: NULL pointer", who);
  if (out_dim < 0 || in_dim <= 0)
    return spk::fail(SPK_ERR_SHAPE, "%s: out_dim %d in_dim %d", who, out_dim, in_dim);
  if (out_dim == 0) return SPK_OK;
  hipStream_t s = spk::to_hip(stream);
  if (order == SPK_MATVEC_ORDER_STRIDED) {
    if ((size_t)out_dim * (size_t)in_dim * 2 >= kStreamBytes)
      hipLaunchKernelGGL((gemv_strided_kernel<4, true>), dim3((out_dim + 15) / 16), dim3(256), 0, s, W, x, y,
                         out_dim, in_dim);
    else if (out_dim >= 16384)
      hipLaunchKernelGGL((gemv_strided_kernel<4, false>), dim3((out_dim + 15) / 16), dim3(256), 0, s, W, x, y,
                         out_dim, in_dim);
    else
      hipLaunchKernelGGL((gemv_strided_kernel<1, false>), dim3((out_dim + 3) / 4), dim3(256), 0, s, W, x, y,
                         out_dim, in_dim);
    return spk::check_launch(who);
  }
  if (in_dim % 64 == 0 && spk::aligned(W, 16) && spk::aligned(x, 16) &&
      (size_t)out_dim * (size_t)in_dim * 2 >= kStreamBytes)
    hipLaunchKernelGGL(gemv_serial_kernel<true>, dim3((out_dim + 255) / 256), dim3(256), 0, s, W, x, y,
                       out_dim, in_dim);
  else if (in_dim % 64 == 0 && spk::aligned(W, 16) && spk::aligned(x, 16))
    hipLaunchKernelGGL(gemv_serial_kernel<false>, dim3((out_dim + 255) / 256), dim3(256), 0, s, W, x, y,
                       out_dim, in_dim);
  else
    hipLaunchKernelGGL(gemv_serial_generic_kernel, dim3((out_dim + 255) / 256), dim3(256), 0, s, W, x, y,
                       out_dim, in_dim);
  return spk::check_launch(who);
}

extern "C" int spk_matvec_f16_batched(const SpkMatvecDesc* d, int32_t count, spk_stream_t stream) {
  if (count < 0 || (count > 0 && !d)) return spk::fail(SPK_ERR_ARG, "spk_matvec_f16_batched: bad descriptor list");
  for (int i = 0; i < count; ++i) {
    const int rc = check_gemv(d[i].W, d[i].x, d[i].y, d[i].out_dim, d[i].in_dim, "spk_matvec_f16_batched");
    if (rc) return rc;
  }
  hipStream_t s = spk::to_hip(stream);
  GemvBatch b;
  b.count = 0;
  int blocks = 0;
  auto flush = [&]() -> int {
    if (b.count == 0) return SPK_OK;
    b.first_block[b.count] = blocks;
    hipLaunchKernelGGL(gemv_batched_kernel, dim3(blocks), dim3(256), 0, s, b);
    b.count = 0;
    blocks = 0;
    return spk::check_launch("spk_matvec_f16_batched");
  };
  for (int i = 0; i < count; ++i) {
    if (d[i].out_dim == 0) continue;
    const bool vec = d[i].in_dim % 512 == 0 && d[i].in_dim <= 8 * 512 && spk::aligned(d[i].W, 16) &&
                     spk::aligned(d[i].x, 16);
    if (!vec) {  // rare shapes: their own launch, same per-row order
      const int rc = launch_gemv(d[i].W, d[i].x, d[i].y, d[i].out_dim, d[i].in_dim, s);
      if (rc) return rc;
      continue;
    }
    b.W[b.count] = d[i].W;
    b.x[b.count] = d[i].x;
    b.y[b.count] = d[i].y;
    b.out_dim[b.count] = d[i].out_dim;
    b.n8[b.count] = d[i].in_dim / 512;
    b.first_block[b.count] = blocks;
    const int rows_per_block = 4 * batch_rows(d[i].in_dim / 512);
    blocks += (d[i].out_dim + rows_per_block - 1) / rows_per_block;
    if (++b.count == kMaxBatch) {
      const int rc = flush();
      if (rc) return rc;
    }
  }
  return flush();
}

extern "C" int spk_argmax_f16(const uint16_t* vals, int32_t n, uint32_t* out_index,
                              spk_stream_t stream) {
  if (!vals || !out_index) return spk::fail(SPK_ERR_NULL, "spk_argmax_f16: NULL pointer");
  if (n <= 0) return spk::fail(SPK_ERR_SHAPE, "spk_argmax_f16: n %d", n);
  const uint32_t E = (uint32_t)((n + 255) / 256);
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, spk::to_hip(stream), vals, n, E, out_index);
  return spk::check_launch("spk_argmax_f16");
}

extern "C" size_t spk_lm_head_workspace_size(int32_t vocab) {
  if (vocab <= 0) return 0;
  const size_t blocks = ((size_t)vocab + 4 * kLmRows - 1) / (4 * kLmRows);
  return ((blocks * sizeof(unsigned long long) + 255) / 256) * 256;
}

namespace {

// Validation and the two launches shared by spk_lm_head_argmax and
// spk_lm_head_argmax_noalloc; `partial` holds one 64-bit key per workgroup.
int lm_head_argmax_launch(const char* name, const uint16_t* W, const uint16_t* x, int32_t vocab,
                          int32_t hidden, uint16_t* logits, uint32_t* out_index,
                          unsigned long long* partial, hipStream_t s) {
  const uint32_t E = (uint32_t)((vocab + 255) / 256);
  const int blocks = (vocab + 4 * kLmRows - 1) / (4 * kLmRows);
#define SPK_LM_CASE(n8)                                                                        \
  case n8:                                                                                     \
    hipLaunchKernelGGL((lm_head_kernel<n8, kLmRows>), dim3(blocks), dim3(256), 0, s, W, x,     \
                       logits, vocab, E, partial);                                             \
    break;
  switch (hidden / 512) {
    SPK_LM_CASE(1)
    SPK_LM_CASE(2)
    SPK_LM_CASE(3)
    SPK_LM_CASE(4)
    SPK_LM_CASE(5)
    SPK_LM_CASE(6)
    SPK_LM_CASE(7)
    SPK_LM_CASE(8)
    default:
      return spk::fail(SPK_ERR_SHAPE, "%s: hidden %d", name, hidden);
  }
#undef SPK_LM_CASE
  int rc = spk::check_launch(name);
  if (rc) return rc;
  hipLaunchKernelGGL(argmax_partials_kernel, dim3(1), dim3(1024), 0, s, partial, blocks, E, out_index);
  return spk::check_launch(name);
}

int lm_head_check_args(const char* name, const uint16_t* W, const uint16_t* x, int32_t vocab,
                       int32_t hidden, const uint32_t* out_index) {
  if (!W || !x || !out_index) return spk::fail(SPK_ERR_NULL, "%s: NULL pointer", name);
  if (vocab <= 0 || hidden <= 0 || hidden % 512 != 0 || hidden > 8 * 512)
    return spk::fail(SPK_ERR_SHAPE, "%s: vocab %d hidden %d (hidden must be a multiple of 512, <= 4096)",
                     name, vocab, hidden);
  if (!spk::aligned(W, 16) || !spk::aligned(x, 16))
    return spk::fail(SPK_ERR_ALIGN, "%s: W/x must be 16-byte aligned", name);
  return SPK_OK;
}

}  // namespace

extern "C" int spk_lm_head_argmax(const uint16_t* W, const uint16_t* x, int32_t vocab,
                                  int32_t hidden, uint16_t* logits, uint32_t* out_index,
                                  void* workspace, size_t workspace_bytes, spk_stream_t stream) {
  const char* name = "spk_lm_head_argmax";
  if (int rc = lm_head_check_args(name, W, x, vocab, hidden, out_index)) return rc;
  if (!workspace) return spk::fail(SPK_ERR_NULL, "%s: workspace is NULL", name);
  if (!spk::aligned(workspace, 8)) return spk::fail(SPK_ERR_ALIGN, "%s: workspace must be 8-byte aligned", name);
  if (workspace_bytes < spk_lm_head_workspace_size(vocab))
    return spk::fail(SPK_ERR_ARG, "%s: workspace %zu < %zu bytes", name, workspace_bytes,
                     spk_lm_head_workspace_size(vocab));
  return lm_head_argmax_launch(name, W, x, vocab, hidden, logits, out_index,
                               static_cast<unsigned long long*>(workspace), spk::to_hip(stream));
}

// ---------------------------------------------------------------------------
// spk_lm_head_argmax_noalloc: the same two kernels with their partial keys in
// a file-scope device array instead of a caller workspace, for callers that
// cannot allocate.  Every device holds its own copy of `scratch` for the life
// of the process; its address on the current device is looked up once
// (hipGetSymbolAddress) and kept per device.  Each call overwrites the keys
// it uses before reading them, so nothing has to start at zero; two calls
// that overlap on one device race on the array.
// ---------------------------------------------------------------------------
namespace {
constexpr int kNoAllocBlocks = (SPK_LM_HEAD_NOALLOC_MAX_VOCAB + 4 * kLmRows - 1) / (4 * kLmRows);
}  // namespace

static __device__ __align__(256) unsigned long long scratch[kNoAllocBlocks];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned long long* g_scratch_ptr[kMaxDevices] = {};

int scratch_on_current_device(const char* name, unsigned long long** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return spk::fail(SPK_ERR_HIP, "%s: hipGetDevice: %s", name, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return spk::fail(SPK_ERR_ARG, "%s: device %d out of range", name, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return spk::fail(SPK_ERR_HIP, "%s: hipGetSymbolAddress(scratch): %s", name, hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<unsigned long long*>(p);
  }
  *out = g_scratch_ptr[dev];
  return SPK_OK;
}
}  // namespace

extern "C" int spk_lm_head_argmax_noalloc(const uint16_t* W, const uint16_t* x, int32_t vocab,
                                          int32_t hidden, uint16_t* logits, uint32_t* out_index,
                                          spk_stream_t stream) {
  const char* name = "spk_lm_head_argmax_noalloc";
  if (int rc = lm_head_check_args(name, W, x, vocab, hidden, out_index)) return rc;
  if (vocab > SPK_LM_HEAD_NOALLOC_MAX_VOCAB)
    return spk::fail(SPK_ERR_SHAPE, "%s: vocab %d exceeds the static scratch limit of %d rows", name, vocab,
                     SPK_LM_HEAD_NOALLOC_MAX_VOCAB);
  unsigned long long* partial = nullptr;
  if (int rc = scratch_on_current_device(name, &partial)) return rc;
  return lm_head_argmax_launch(name, W, x, vocab, hidden, logits, out_index, partial, spk::to_hip(stream));
}
