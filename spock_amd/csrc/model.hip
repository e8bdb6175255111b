// model.hip -- the remaining per-token kernels of the Qwen3.5-0.8B decode loop
// (src/runtime/vk_session.cpp:2560-3400): projections with their input norm /
// SiLU gate fused in front and the residual add fused behind, the full-
// attention token mixer, and the element-wise operations the prefill needs.
//
// Every result is bit-identical to the CPU restatement (oracle/model.h lists
// the operation order); the orders are:
//   RMSNorm(1+w), n = 1024: 256 partials of 4 contiguous squares (fma chain),
//     tree s[t] += s[t+stride] for stride 128..1, nf = 1/sqrt(sum/1024 + eps),
//     y = fp16((x*nf)*(1+w))                                  (rms_norm.comp)
//   per-head RMSNorm, n = 256: partials x_t^2, same tree   (rms_norm_per_head.comp)
//   GEMV: 64 lanes x contiguous spans, fma chains from 0, then the 32..1 tree
//   attention: blocks of 64 positions; per block max, exp, 64-lane tree of the
//     weights and fma chains over positions; blocks combined in order.
#include "argmax_key.hpp"
#include "capi_common.hpp"
#include "numerics.hpp"
#include "dense_rows.hpp"
#include "dn_step.hpp"

#include <float.h>

namespace {

constexpr int kHidden = 1024;
constexpr int kLmKeyRows = 4;  // vocabulary rows per wavefront of the lm_head key kernels
constexpr int kHeadDim = 256;
constexpr int kQHeads = 8;
constexpr int kKvHeads = 2;
constexpr int kKvRow = 1024;  // K 2x256 | V 2x256 halves per cached position
constexpr int kAttnBlock = 64;
constexpr int kPartFloats = 2 + kHeadDim;  // attention block partials: m, S, O[256]

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Weight loads are plain (cached) 16-byte loads: for decode-sized matrices (a
// few MB per launch) non-temporal loads measured slower on MI355X, up to 2x for
// a single GEMV and 689.4 vs 684.7 us per config-4 token, although they stream
// faster over hundreds of MB.
__device__ __forceinline__ uint4 ld_w(const uint4* p) { return *p; }

__device__ __forceinline__ void unpack8(const uint4& u, float* f) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = spk::h2f((uint16_t)(w[i] & 0xffffu));
    f[2 * i + 1] = spk::h2f((uint16_t)(w[i] >> 16));
  }
}

__device__ __forceinline__ float round16(float v) { return spk::h2f(spk::f2h(v)); }

// Sum of the partials of threads 0..255 in the rms_norm.comp tree order
// (s[t] += s[t+128], += s[t+64], then strides 32..1); every thread of the
// block (256 or more threads) gets the result.  `red` is 256 floats of LDS.
__device__ __forceinline__ float block_tree256(float p, float* red) {
  const int t = threadIdx.x;
  if (t < 256) red[t] = p;
  __syncthreads();
  // every wavefront takes the first two levels (strides 128 and 64) for its
  // lane l from four LDS reads -- (p[l] + p[l+128]) + (p[l+64] + p[l+192]),
  // the tree's own pairs -- and the last six in registers: one barrier
  // instead of one per level.  red must not be written again in the kernel.
  const int l = t & 63;
  const float v = (red[l] + red[l + 128]) + (red[l + 64] + red[l + 192]);
  const float s = spk::tree64_to_lane0(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
}

// ---------------------------------------------------------------------------
// Fused GEMV: y_o = fp16(W_o . x) (+ residual), x = one of
//   PLAIN      x
//   RMSNORM    fp16(RMSNorm(h) * (1 + w)),  h = x (or row token[0] of x)
//   SILU_GATE  fp16(silu(gate) * up)
// computed once per workgroup into LDS (fp16-rounded values as floats).
// An output with a second matrix (W2) is the SiLU-gated pair of
// silu_gate.comp: y = fp16(silu(fp16(W . x)) * fp16(W2 . x)), both rows of a
// pair computed by the same wave.
// ---------------------------------------------------------------------------
constexpr int kMaxOut = 8;     // outputs per spk_gemv_fused call
constexpr int kLaunchOut = 4;  // outputs per launch (more are split over launches)
constexpr int kMaxIn = 4096;

struct FusedGemv {
  int kind;
  int in_dim;
  const uint16_t* x;
  const uint16_t* x2;
  const int32_t* token;
  int token_rows;
  uint16_t* h_out;
  int count;
  const uint16_t* W[kLaunchOut];
  const uint16_t* W2[kLaunchOut];
  uint16_t* y[kLaunchOut];
  const uint16_t* res[kLaunchOut];
  int out_dim[kLaunchOut];
  int first_block[kLaunchOut + 1];
  // the TOUCH form only (spk_attention_inproj): K/V cache rows 0 .. *touch_pos
  // (at most touch_rows) read and dropped, so that the attention launch that
  // follows finds them in the caches (spk_attention_inproj)
  const uint16_t* touch;
  const int32_t* touch_pos;
  int touch_rows;
};

template <int N8, int R>
__device__ __forceinline__ void load_rows(const uint16_t* __restrict__ W, int row0, int out_dim, int lane,
                                          uint4 (&wv)[R][N8]) {
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r < out_dim ? row0 + r : out_dim - 1;
    const uint4* src = reinterpret_cast<const uint4*>(W + (size_t)row * (512 * N8) + lane * (8 * N8));
#pragma unroll
    for (int k = 0; k < N8; ++k) wv[r][k] = ld_w(src + k);
  }
}

// Sequential fma chain over the lane's 8*N8 contiguous elements (from 0).
template <int N8>
__device__ __forceinline__ float lane_dot(const uint4 (&wr)[N8], const float* xf) {
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < N8; ++k) {
    float wf[8];
    unpack8(wr[k], wf);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_fmaf(wf[e], xf[8 * k + e], acc);
  }
  return acc;
}

// KIND is the input kind (compile time, so the input and weight loads sit in
// one straight-line block: the input operands are issued first and the
// prologue waits for them alone while the weight rows are in flight).
template <int N8, int R, bool PAIR, int KIND, bool TOUCH = false>
__global__ __launch_bounds__(256) void fused_gemv_kernel(FusedGemv a) {
  __shared__ float xs[kMaxIn];
  __shared__ float red[257];
  // Every output's descriptor is read and the workgroup's one selected by
  // value, so all kernel-argument loads go out in one round trip (indexing
  // the arrays by the selected output would wait for first_block before
  // loading the weight pointers).
  const uint16_t* Wd = a.W[0];
  const uint16_t* W2d = a.W2[0];
  uint16_t* yd = a.y[0];
  const uint16_t* resd = a.res[0];
  int out_dim = a.out_dim[0], fb = 0;
#pragma unroll
  for (int i = 1; i < kLaunchOut; ++i) {
    const bool take = i < a.count && (int)blockIdx.x >= a.first_block[i];
    Wd = take ? a.W[i] : Wd;
    W2d = take ? a.W2[i] : W2d;
    yd = take ? a.y[i] : yd;
    resd = take ? a.res[i] : resd;
    out_dim = take ? a.out_dim[i] : out_dim;
    fb = take ? a.first_block[i] : fb;
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  constexpr int in_dim = 512 * N8;
  const int row0 = (((int)blockIdx.x - fb) * 4 + wave) * R;
  constexpr int NV = in_dim / 8;  // 16-byte pieces of x
  constexpr int PER = (NV + 255) / 256;
  static_assert(256 * PER * 8 <= kMaxIn, "x staging overruns xs");
  // K/V rows for the next launch: 16 bytes per thread over the grid, issued
  // first (the position's load, then the rows) and waited for only at the end
  uint4 tv = make_uint4(0, 0, 0, 0);
  if (TOUCH) {
    const int rows = min(a.touch_pos[0] + 1, a.touch_rows);
    const size_t toff = ((size_t)blockIdx.x * 256 + tid) * 16;
    if (toff < (size_t)max(rows, 0) * (kKvRow * 2))
      tv = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(a.touch) + toff);
  }
  uint2 hv = make_uint2(0, 0), nwv = make_uint2(0, 0);
  uint4 xv[PER], uv[PER];
  if constexpr (KIND == SPK_GEMV_IN_RMSNORM) {  // in_dim == 1024: 4 elements per thread
    const uint16_t* h = a.x;
    if (a.token) {  // ids outside [0, token_rows) select row 0 instead of reading out of bounds
      const int id = a.token[0];
      h += (size_t)((id >= 0 && id < a.token_rows) ? id : 0) * kHidden;
    }
    hv = *reinterpret_cast<const uint2*>(h + 4 * tid);
    nwv = *reinterpret_cast<const uint2*>(a.x2 + 4 * tid);
  } else {
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const int idx = min(tid + 256 * c, NV - 1);
      xv[c] = *reinterpret_cast<const uint4*>(a.x + 8 * idx);
      if constexpr (KIND == SPK_GEMV_IN_SILU_GATE) uv[c] = *reinterpret_cast<const uint4*>(a.x2 + 8 * idx);
    }
  }
  // residual rows (or, without a residual, any in-bounds halves) ahead of
  // the weights, so the epilogue waits on no load of its own
  const uint16_t* __restrict__ res = resd;
  const uint16_t* rsrc = res ? res : Wd;
  uint16_t rv[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rv[r] = rsrc[min(row0 + r, out_dim - 1)];
  uint4 wv[R][N8];
  uint4 wv2[PAIR ? R : 1][N8];
  load_rows<N8, R>(Wd, row0, out_dim, lane, wv);
  if (PAIR) load_rows<N8, PAIR ? R : 1>(W2d, row0, out_dim, lane, wv2);
  __builtin_amdgcn_sched_barrier(0);  // every load in flight before the prologue
  if constexpr (KIND == SPK_GEMV_IN_RMSNORM) {
    const float v[4] = {spk::h2f(hv.x & 0xffffu), spk::h2f(hv.x >> 16), spk::h2f(hv.y & 0xffffu),
                        spk::h2f(hv.y >> 16)};
    const float w[4] = {spk::h2f(nwv.x & 0xffffu), spk::h2f(nwv.x >> 16), spk::h2f(nwv.y & 0xffffu),
                        spk::h2f(nwv.y >> 16)};
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) p = __builtin_fmaf(v[i], v[i], p);
    const float sum = block_tree256(p, red);
    const float nf = 1.0f / __builtin_sqrtf(sum / 1024.0f + 1e-6f);
#pragma unroll
    for (int i = 0; i < 4; ++i) xs[4 * tid + i] = round16((v[i] * nf) * (1.0f + w[i]));
  } else {
    // unconditional (pieces past NV repeat the last one into xs slots no lane
    // reads; 256 * PER * 8 <= kMaxIn), so no load is sunk under a branch
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const int idx = tid + 256 * c;
      float f[8];
      unpack8(xv[c], f);
      if constexpr (KIND == SPK_GEMV_IN_SILU_GATE) {
        float u[8];
        unpack8(uv[c], u);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = round16(spk::silu_det(f[e]) * u[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; e += 4) *reinterpret_cast<float4*>(&xs[8 * idx + e]) = make_float4(f[e], f[e + 1], f[e + 2], f[e + 3]);
    }
  }
  __syncthreads();
  float xf[8 * N8];
#pragma unroll
  for (int k = 0; k < 8 * N8; k += 4) {
    const float4 t = *reinterpret_cast<const float4*>(&xs[lane * (8 * N8) + k]);
    xf[k] = t.x;
    xf[k + 1] = t.y;
    xf[k + 2] = t.z;
    xf[k + 3] = t.w;
  }
  constexpr int NT = PAIR ? 2 * R : R;
  float acc[NT];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[r] = lane_dot<N8>(wv[r], xf);
    if (PAIR) acc[R + r] = lane_dot<N8>(wv2[PAIR ? r : 0], xf);
  }
  spk::tree64_rows<NT>(acc);
  uint16_t* __restrict__ y = yd;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
    if (lane == 0 && row < out_dim) {
      uint16_t o = spk::f2h(acc[r]);
      if (PAIR) o = spk::f2h(spk::silu_det(spk::h2f(o)) * spk::h2f(spk::f2h(acc[PAIR ? R + r : 0])));
      if (res) o = spk::f2h(spk::h2f(rv[r]) + spk::h2f(o));
      y[row] = o;
    }
  }
  // the first layer's input row (token embedding) becomes the residual stream
  if constexpr (KIND == SPK_GEMV_IN_RMSNORM)
    if (a.h_out && blockIdx.x == 0) *reinterpret_cast<uint2*>(a.h_out + 4 * tid) = hv;
  if constexpr (TOUCH) asm volatile("" ::"v"(tv.x));  // keeps the touch loads
}

// ---------------------------------------------------------------------------
// Attention decode (attention_decode.comp + rms_norm_per_head + rope_apply +
// kv_cache_store + sigmoid_gate for one token), position read from device.
// Kernel 1: one workgroup per (64-position block, KV head), wave w = query
// head 4*kvh + w.  Block of the current position also norms/ropes the new
// K row and stores K/V into the cache.  Writes per (query head, block):
// m_b, S_b, O_b[256].  Kernel 2: per query head, combine blocks in order,
// normalise, sigmoid gate.
// ---------------------------------------------------------------------------

// Per-head RMSNorm(1+w) of the 256 values a wave holds (lane l: d = 4l..4l+3),
// in the s[t] += s[t+stride] (stride 128..1) order; returns fp16-rounded values.
// wf: the lane's 4 norm weights.
__device__ __forceinline__ void head_norm_wave(float (&v)[4], const float (&wf)[4]) {
  float s[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) s[i] = v[i] * v[i];
  spk::tree64_rows<4>(s);  // strides 128, 64, ..., 4 (lane distance 32..1), sums in lane 0
  float sum = (s[0] + s[2]) + (s[1] + s[3]);  // strides 2 then 1 inside lane 0
  sum = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sum), 0));  // lane 0 broadcast, no LDS
  const float nf = 1.0f / __builtin_sqrtf(sum / 256.0f + 1e-6f);
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = round16((v[i] * nf) * (1.0f + wf[i]));
}

__device__ __forceinline__ void head_norm_wave(float (&v)[4], const uint16_t* w, int lane) {
  const uint2 wv = *reinterpret_cast<const uint2*>(w + 4 * lane);
  const float wf[4] = {spk::h2f(wv.x & 0xffffu), spk::h2f(wv.x >> 16), spk::h2f(wv.y & 0xffffu),
                       spk::h2f(wv.y >> 16)};
  head_norm_wave(v, wf);
}

// The (cos, sin) pairs of the lane's 4 dims d = 4l..4l+3 (pair index d & 31).
__device__ __forceinline__ void load_rope(const float* cs, int lane, float (&c)[8]) {
  const int p0 = (4 * lane) & 31;
  const float4 lo = *reinterpret_cast<const float4*>(cs + 2 * p0);
  const float4 hi = *reinterpret_cast<const float4*>(cs + 2 * p0 + 4);
  c[0] = lo.x; c[1] = lo.y; c[2] = lo.z; c[3] = lo.w;
  c[4] = hi.x; c[5] = hi.y; c[6] = hi.z; c[7] = hi.w;
}

// rope_apply.comp pairs (i, i+32), i < 32: lanes 0..7 hold d < 32, lanes 8..15 d in [32, 64).
__device__ __forceinline__ void rope_wave(float (&v)[4], const float (&c8)[8], int lane) {
  float o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = spk::lane_xor8(v[i]);
  if (lane < 16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // d < 32: v*c - o*s; else v*c + o*s (negating o first gives the same bits)
      const float os = (4 * lane + i < 32) ? -o[i] : o[i];
      v[i] = round16(v[i] * c8[2 * i] + os * c8[2 * i + 1]);
    }
  }
}

__device__ __forceinline__ void rope_wave(float (&v)[4], const float* cs, int lane) {
  float c8[8];
  load_rope(cs, lane, c8);
  rope_wave(v, c8, lane);
}

__device__ __forceinline__ void load4h(const uint16_t* p, float (&v)[4]) {
  const uint2 u = *reinterpret_cast<const uint2*>(p);
  v[0] = spk::h2f(u.x & 0xffffu);
  v[1] = spk::h2f(u.x >> 16);
  v[2] = spk::h2f(u.y & 0xffffu);
  v[3] = spk::h2f(u.y >> 16);
}

__device__ __forceinline__ uint2 pack4h(const float (&v)[4]) {
  uint2 u;
  u.x = (uint32_t)spk::f2h(v[0]) | ((uint32_t)spk::f2h(v[1]) << 16);
  u.y = (uint32_t)spk::f2h(v[2]) | ((uint32_t)spk::f2h(v[3]) << 16);
  return u;
}

struct AttnArgs {
  const uint16_t* qg;  // [T][4096] (T = 1 for decode)
  const uint16_t* k;   // [T][512]
  const uint16_t* v;   // [T][512]
  const uint16_t* q_norm_w;
  const uint16_t* k_norm_w;
  const float* rope;
  uint16_t* kv;        // layer cache [max_seq][1024]
  int max_seq;
  const int32_t* pos_dev;  // decode: device position
  int pos0;                // prefill: first position
  uint16_t* out;       // [T][2048]
  float* part;         // [T][8][max_blocks][kPartFloats]
  int max_blocks;      // blocks of 64 positions the grid covers
  int store_kv;        // decode: the current position's block stores its K/V row
  int tokens;          // T
  int32_t* arrive;     // decode with the combine: one count per KV head, 64 ints apart
};

// K rows in LDS are padded to 264 halves (528 B): lane p reading 16 B of row p
// and lane p+1 reading row p+1 land 4 banks apart, so a ds_read_b128 over 64
// rows is conflict-free.
constexpr int kKLd = kHeadDim + 8;

// One query-head wave over one block of positions [64b, 64b+64) of npos valid
// ones, operands staged in LDS (K as Ks[p][d], V as Vs[p][d], q as fp16: its
// values are fp16-rounded, so this is exact): writes m_b, S_b, O_b.  Lane =
// position for the scores: each lane reads its K row 8 dims at a time
// (ds_read_b128) and runs the d = 0..255 fma chain, the reads one 32-dim stage
// ahead of the chain; the weighted
// V sum visits positions j = 0..nvalid-1 in order, taking w_j by readlane,
// in whole groups of 8 positions with no per-position branch (the next
// group's V rows are read while the current one accumulates), then the
// block's last partial group.
__device__ __forceinline__ void v_group(const uint2 (&vv)[8], int wbits, int j0, int n, float (&acc)[4]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i < n) {
      const float wj = __int_as_float(__builtin_amdgcn_readlane(wbits, j0 + i));
      const float vf[4] = {spk::h2f(vv[i].x & 0xffffu), spk::h2f(vv[i].x >> 16), spk::h2f(vv[i].y & 0xffffu),
                           spk::h2f(vv[i].y >> 16)};
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = __builtin_fmaf(wj, vf[e], acc[e]);
    }
  }
}

__device__ __forceinline__ void attn_block_wave(const uint16_t* qs, const uint16_t (*Ks)[kKLd],
                                                const uint16_t (*Vs)[kHeadDim], int b, int npos, int lane,
                                                float* part) {
  const int p = kAttnBlock * b + lane;
  float sc = -INFINITY;
  if (p < npos) {
    // 8 stages of 32 dims; stage s+1's K and q pieces are read while stage s
    // runs its 32 chained fmas
    float dot = 0.0f;
    uint4 kc[4], qc[4], kn[4], qn[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kc[i] = *reinterpret_cast<const uint4*>(&Ks[lane][8 * i]);
      qc[i] = *reinterpret_cast<const uint4*>(&qs[8 * i]);
    }
#pragma unroll
    for (int st = 0; st < kHeadDim / 32; ++st) {
      if (st + 1 < kHeadDim / 32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          kn[i] = *reinterpret_cast<const uint4*>(&Ks[lane][32 * (st + 1) + 8 * i]);
          qn[i] = *reinterpret_cast<const uint4*>(&qs[32 * (st + 1) + 8 * i]);
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float kf[8], qf[8];
        unpack8(kc[i], kf);
        unpack8(qc[i], qf);
#pragma unroll
        for (int e = 0; e < 8; ++e) dot = __builtin_fmaf(qf[e], kf[e], dot);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kc[i] = kn[i];
        qc[i] = qn[i];
      }
    }
    sc = dot * 0.0625f;
  }
  float m = sc;
  m = spk::wave_max(m);
  const float w = (p < npos) ? spk::expf_det(sc - m) : 0.0f;
  const float S = spk::tree64_to_lane0(w);
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int nvalid = min(kAttnBlock, npos - kAttnBlock * b);
  const int nfull = nvalid & ~7;
  const int wbits = __float_as_int(w);
  uint2 cur[8], nxt[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cur[i] = *reinterpret_cast<const uint2*>(&Vs[i][4 * lane]);
  for (int j0 = 0; j0 < nfull; j0 += 8) {
    const int jn = min(j0 + 8, kAttnBlock - 8);  // rows of the next group (in bounds)
#pragma unroll
    for (int i = 0; i < 8; ++i) nxt[i] = *reinterpret_cast<const uint2*>(&Vs[jn + i][4 * lane]);
    v_group(cur, wbits, j0, 8, acc);
#pragma unroll
    for (int i = 0; i < 8; ++i) cur[i] = nxt[i];
  }
  if (nfull < nvalid) v_group(cur, wbits, nfull, nvalid - nfull, acc);  // cur holds rows nfull..nfull+7
  if (lane == 0) {
    part[0] = m;
    part[1] = S;
  }
  *reinterpret_cast<float4*>(part + 2 + 4 * lane) = make_float4(acc[0], acc[1], acc[2], acc[3]);
}

// grid (max_blocks, kv_heads, T); block 256.
// COMBINE (decode, T = 1): the grid is 1-D, workgroup id = 8 b + 4 kvh (the
// others exit at once), so the blocks of one KV head run on one XCD and share
// its L2; after writing its partials each block counts its arrival on the KV
// head's counter, and the last of the head's live blocks combines them for
// the head's 4 query heads (attn_combine_kernel's arithmetic, bit for bit)
// into out, and resets the counter.
template <bool COMBINE>
__global__ __launch_bounds__(256) void attn_blocks_kernel(AttnArgs a) {
  __shared__ __align__(16) uint16_t qs[4][kHeadDim];  // fp16-rounded q, stored exactly as fp16
  __shared__ __align__(16) uint16_t Ks[kAttnBlock][kKLd];
  __shared__ __align__(16) uint16_t Vs[kAttnBlock][kHeadDim];
  __shared__ int last;
  if (COMBINE && (blockIdx.x & 3)) return;
  const int b = COMBINE ? (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const int kvh = COMBINE ? (int)((blockIdx.x >> 2) & 1) : (int)blockIdx.y;
  const int t = COMBINE ? 0 : (int)blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int pos = a.pos_dev ? a.pos_dev[0] : a.pos0 + t;
  if (pos < 0 || pos >= a.max_seq) return;
  const int npos = pos + 1;
  if (kAttnBlock * b >= npos) return;
  const float* cs = a.rope + (size_t)pos * 64;
  const int cur = (a.store_kv && (pos / kAttnBlock) == b) ? pos - kAttnBlock * b : -1;
  const int qh = kvh * 4 + wave;
  // Loads first, small operands ahead of the block's K/V rows (a wave's loads
  // complete in issue order): this wave's q head with its norm weights and
  // RoPE pairs, the new K/V row when this block holds the current position,
  // then K/V of position 64b + tid/4 (quarter tid%4: 64 dims of K and of V;
  // rows past the current position read row 0 and stage zeros).
  float qv[4], qw[4], c8[8], gv[4];
  load4h(a.qg + (size_t)t * 4096 + qh * 512 + 4 * lane, qv);
  load4h(a.q_norm_w + 4 * lane, qw);
  load_rope(cs, lane, c8);
  // the output gate of this wave's query head, for the combine (read here
  // with the first operands, so the last workgroup's combine waits on no
  // load of its own after the partials)
  if constexpr (COMBINE) load4h(a.qg + qh * 512 + 256 + 4 * lane, gv);
  // the new K/V row, by the one wavefront that stores it (wavefront 0 of the
  // block holding the position); elsewhere the values start opaque, so no
  // load meets a constant at the branch join (the compiler would wait for it
  // there)
  const bool newrow = cur >= 0 && wave == 0;
  uint2 nk16 = make_uint2(spk_dn::opaque_u32(), spk_dn::opaque_u32());
  uint2 kw16 = make_uint2(spk_dn::opaque_u32(), spk_dn::opaque_u32());
  uint2 vb = make_uint2(spk_dn::opaque_u32(), spk_dn::opaque_u32());
  if (newrow) {
    nk16 = *reinterpret_cast<const uint2*>(a.k + (size_t)t * 512 + kvh * kHeadDim + 4 * lane);
    kw16 = *reinterpret_cast<const uint2*>(a.k_norm_w + 4 * lane);
    vb = *reinterpret_cast<const uint2*>(a.v + (size_t)t * 512 + kvh * kHeadDim + 4 * lane);
  }
  const int p = tid >> 2, q4 = tid & 3;
  const int gp = kAttnBlock * b + p;
  const bool live = gp < npos && p != cur;
  const uint16_t* row = a.kv + (size_t)(live ? gp : 0) * kKvRow + kvh * kHeadDim + q4 * 64;
  uint4 kv4[8], vv4[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    kv4[i] = *reinterpret_cast<const uint4*>(row + 8 * i);
    vv4[i] = *reinterpret_cast<const uint4*>(row + 512 + 8 * i);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the q work below
  head_norm_wave(qv, qw);
  rope_wave(qv, c8, lane);
  *reinterpret_cast<uint2*>(&qs[wave][4 * lane]) = pack4h(qv);
  if (newrow) {  // new K row: norm + rope; V row as projected
    float nk[4] = {spk::h2f(nk16.x & 0xffffu), spk::h2f(nk16.x >> 16), spk::h2f(nk16.y & 0xffffu),
                   spk::h2f(nk16.y >> 16)};
    const float kw[4] = {spk::h2f(kw16.x & 0xffffu), spk::h2f(kw16.x >> 16), spk::h2f(kw16.y & 0xffffu),
                         spk::h2f(kw16.y >> 16)};
    head_norm_wave(nk, kw);
    rope_wave(nk, c8, lane);
    const uint2 kb = pack4h(nk);
    *reinterpret_cast<uint2*>(&Ks[cur][4 * lane]) = kb;
    *reinterpret_cast<uint2*>(&Vs[cur][4 * lane]) = vb;
    uint16_t* crow = a.kv + (size_t)pos * kKvRow;  // kv_cache_store.comp:27-48
    *reinterpret_cast<uint2*>(crow + kvh * kHeadDim + 4 * lane) = kb;
    *reinterpret_cast<uint2*>(crow + 512 + kvh * kHeadDim + 4 * lane) = vb;
  }
  if (p != cur) {
    const uint32_t keep = live ? 0xffffffffu : 0u;  // rows past the current position stage zeros
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint4 k = make_uint4(kv4[i].x & keep, kv4[i].y & keep, kv4[i].z & keep, kv4[i].w & keep);
      const uint4 v = make_uint4(vv4[i].x & keep, vv4[i].y & keep, vv4[i].z & keep, vv4[i].w & keep);
      *reinterpret_cast<uint4*>(&Ks[p][q4 * 64 + 8 * i]) = k;
      *reinterpret_cast<uint4*>(&Vs[p][q4 * 64 + 8 * i]) = v;
    }
  }
  __syncthreads();
  float* part = a.part + (((size_t)t * kQHeads + qh) * a.max_blocks + b) * kPartFloats;
  attn_block_wave(qs[wave], Ks, Vs, b, npos, lane, part);
  if constexpr (COMBINE) {
    const int nb = (pos + kAttnBlock) / kAttnBlock;
    __builtin_amdgcn_s_waitcnt(0);  // this block's partials and K/V row stored
    __syncthreads();
    if (tid == 0)
      last = __hip_atomic_fetch_add(a.arrive + 64 * kvh, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == nb - 1;
    __syncthreads();
    if (!last) return;
    if (tid == 0) __hip_atomic_store(a.arrive + 64 * kvh, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // query head qh (this wavefront), dims 4 lane .. 4 lane + 3; the first
    // kPre blocks' partials are loaded in one round trip, later ones 8 at a
    // time, every load of a group issued before any is used
    constexpr int kPre = 16;
    const float* ph = a.part + (size_t)qh * a.max_blocks * kPartFloats;
    float mv[kPre], sv[kPre];
    float4 ovp[kPre];
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      const float* pb = ph + (size_t)min(i, nb - 1) * kPartFloats;
      mv[i] = pb[0];
      sv[i] = pb[1];
      ovp[i] = *reinterpret_cast<const float4*>(pb + 2 + 4 * lane);
    }
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < kPre; ++i) M = fmaxf(M, mv[i]);  // clamped copies of block nb-1 change no maximum
    for (int b0 = kPre; b0 < nb; b0 += 8) {
      float mm[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) mm[i] = ph[(size_t)min(b0 + i, nb - 1) * kPartFloats];
#pragma unroll
      for (int i = 0; i < 8; ++i) M = fmaxf(M, mm[i]);
    }
    float tot = 0.0f, o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
      if (i < nb) {
        const float c = spk::expf_det(mv[i] - M);
        tot = tot + sv[i] * c;
        o[0] = o[0] + ovp[i].x * c;
        o[1] = o[1] + ovp[i].y * c;
        o[2] = o[2] + ovp[i].z * c;
        o[3] = o[3] + ovp[i].w * c;
      }
    }
    for (int b0 = kPre; b0 < nb; b0 += 8) {
      float mm[8], ss[8];
      float4 oo[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float* pb = ph + (size_t)min(b0 + i, nb - 1) * kPartFloats;
        mm[i] = pb[0];
        ss[i] = pb[1];
        oo[i] = *reinterpret_cast<const float4*>(pb + 2 + 4 * lane);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (b0 + i < nb) {
          const float c = spk::expf_det(mm[i] - M);
          tot = tot + ss[i] * c;
          o[0] = o[0] + oo[i].x * c;
          o[1] = o[1] + oo[i].y * c;
          o[2] = o[2] + oo[i].z * c;
          o[3] = o[3] + oo[i].w * c;
        }
      }
    }
    const float inv = 1.0f / (tot + 1e-30f);
    uint16_t r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = spk::f2h(round16(o[e] * inv) * (1.0f / (1.0f + spk::expf_det(-gv[e]))));
    *reinterpret_cast<uint2*>(a.out + qh * kHeadDim + 4 * lane) =
        make_uint2((uint32_t)r[0] | ((uint32_t)r[1] << 16), (uint32_t)r[2] | ((uint32_t)r[3] << 16));
  }
}

// Prefill block pass: one workgroup per (64-position block b, KV head, group
// of kAttnGroup consecutive tokens), wave w = query head 4*kvh + w.  The
// block's K/V rows are staged once for the group (rows up to the group's last
// position; the rows themselves were stored by attn_store_kv_kernel).  Each
// wave runs its head's score chains for the group's tokens together: lane =
// position, one 16-byte K read per 8 dims feeds kAttnGroup independent
// d = 0..255 fma chains, q read as fp16 (its values are fp16-rounded, so
// this is exact).  Per token the arithmetic is attn_block_wave's: positions
// past the token's own are masked to -inf (weight 0), the weighted V sum
// visits positions 0..nvalid_t-1 in order.  Positions every token of the
// group sees are summed for all tokens at once; the last kAttnGroup-1 are
// added token by token, so a token never touches a position it cannot see.
constexpr int kAttnGroup = 4;

__global__ __launch_bounds__(256) void attn_prefill_blocks_kernel(AttnArgs a) {
  __shared__ __align__(16) uint16_t qs[4][kAttnGroup][kHeadDim];
  __shared__ __align__(16) uint16_t Ks[kAttnBlock][kKLd];
  __shared__ __align__(16) uint16_t Vs[kAttnBlock][kHeadDim];
  const int b = blockIdx.x, kvh = blockIdx.y, t0 = blockIdx.z * kAttnGroup;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tl = min(t0 + kAttnGroup, a.tokens) - 1;  // last token of the group
  const int npos0 = a.pos0 + t0 + 1;                  // positions token t0 sees
  const int npos_max = a.pos0 + tl + 1;
  if (kAttnBlock * b >= npos_max) return;
  const int qh = kvh * 4 + wave;
  // Loads first: q rows and RoPE pairs of the group's tokens (tokens past the
  // call's last read the last one's), the q norm weights, then the block's
  // K/V rows (position 64b + tid/4, quarter tid%4; rows past the group's last
  // position read row 0 and stage zeros).
  float qv[kAttnGroup][4], c8[kAttnGroup][8], qw[4];
#pragma unroll
  for (int i = 0; i < kAttnGroup; ++i) {
    const int t = min(t0 + i, tl);
    load4h(a.qg + (size_t)t * 4096 + qh * 512 + 4 * lane, qv[i]);
    load_rope(a.rope + (size_t)(a.pos0 + t) * 64, lane, c8[i]);
  }
  load4h(a.q_norm_w + 4 * lane, qw);
  const int p = tid >> 2, q4 = tid & 3;
  const int gp = kAttnBlock * b + p;
  const bool live = gp < npos_max;
  const uint16_t* row = a.kv + (size_t)(live ? gp : 0) * kKvRow + kvh * kHeadDim + q4 * 64;
  uint4 kv4[8], vv4[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    kv4[i] = *reinterpret_cast<const uint4*>(row + 8 * i);
    vv4[i] = *reinterpret_cast<const uint4*>(row + 512 + 8 * i);
  }
  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the q work below
#pragma unroll
  for (int i = 0; i < kAttnGroup; ++i) {
    head_norm_wave(qv[i], qw);
    rope_wave(qv[i], c8[i], lane);
    *reinterpret_cast<uint2*>(&qs[wave][i][4 * lane]) = pack4h(qv[i]);
  }
  const uint32_t keep = live ? 0xffffffffu : 0u;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint4 k = make_uint4(kv4[i].x & keep, kv4[i].y & keep, kv4[i].z & keep, kv4[i].w & keep);
    const uint4 v = make_uint4(vv4[i].x & keep, vv4[i].y & keep, vv4[i].z & keep, vv4[i].w & keep);
    *reinterpret_cast<uint4*>(&Ks[p][q4 * 64 + 8 * i]) = k;
    *reinterpret_cast<uint4*>(&Vs[p][q4 * 64 + 8 * i]) = v;
  }
  __syncthreads();

  // scores: kAttnGroup chains per lane (position 64b + lane)
  float dot[kAttnGroup];
#pragma unroll
  for (int i = 0; i < kAttnGroup; ++i) dot[i] = 0.0f;
#pragma unroll 2
  for (int d8 = 0; d8 < kHeadDim / 8; ++d8) {
    float kf[8];
    unpack8(*reinterpret_cast<const uint4*>(&Ks[lane][8 * d8]), kf);
#pragma unroll
    for (int i = 0; i < kAttnGroup; ++i) {
      float qf[8];
      unpack8(*reinterpret_cast<const uint4*>(&qs[wave][i][8 * d8]), qf);
#pragma unroll
      for (int e = 0; e < 8; ++e) dot[i] = __builtin_fmaf(qf[e], kf[e], dot[i]);
    }
  }
  const int pp = kAttnBlock * b + lane;
  float m[kAttnGroup], w[kAttnGroup];
  int nvalid[kAttnGroup];
#pragma unroll
  for (int i = 0; i < kAttnGroup; ++i) {
    const bool tok = t0 + i < a.tokens;
    nvalid[i] = tok ? min(kAttnBlock, npos0 + i - kAttnBlock * b) : 0;  // may be <= 0
    m[i] = (tok && pp < npos0 + i) ? dot[i] * 0.0625f : -INFINITY;
  }
#pragma unroll
  for (int i = 0; i < kAttnGroup; ++i) m[i] = spk::wave_max(m[i]);
#pragma unroll
  for (int i = 0; i < kAttnGroup; ++i)
    w[i] = (lane < nvalid[i]) ? spk::expf_det(dot[i] * 0.0625f - m[i]) : 0.0f;
  float acc[kAttnGroup][4];
#pragma unroll
  for (int i = 0; i < kAttnGroup; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[i][e] = 0.0f;
  // positions 0..nv_all-1 are seen by every token of the group
  const int nv_all = max(0, nvalid[0]);
  const int nv_max = min(kAttnBlock, npos_max - kAttnBlock * b);
  for (int j0 = 0; j0 < nv_all; j0 += 8) {
    uint2 vv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) vv[i] = *reinterpret_cast<const uint2*>(&Vs[j0 + i][4 * lane]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (j0 + i < nv_all) {
        const float vf[4] = {spk::h2f(vv[i].x & 0xffffu), spk::h2f(vv[i].x >> 16), spk::h2f(vv[i].y & 0xffffu),
                             spk::h2f(vv[i].y >> 16)};
#pragma unroll
        for (int t = 0; t < kAttnGroup; ++t) {
          const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[t]), j0 + i));
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[t][e] = __builtin_fmaf(wj, vf[e], acc[t][e]);
        }
      }
    }
  }
  for (int j = nv_all; j < nv_max; ++j) {  // at most kAttnGroup - 1 positions
    const uint2 v2 = *reinterpret_cast<const uint2*>(&Vs[j][4 * lane]);
    const float vf[4] = {spk::h2f(v2.x & 0xffffu), spk::h2f(v2.x >> 16), spk::h2f(v2.y & 0xffffu),
                         spk::h2f(v2.y >> 16)};
#pragma unroll
    for (int t = 0; t < kAttnGroup; ++t) {
      if (j < nvalid[t]) {
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w[t]), j));
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[t][e] = __builtin_fmaf(wj, vf[e], acc[t][e]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kAttnGroup; ++i) {
    const float S = spk::tree64_to_lane0(w[i]);
    if (nvalid[i] > 0) {
      float* part = a.part + (((size_t)(t0 + i) * kQHeads + qh) * a.max_blocks + b) * kPartFloats;
      if (lane == 0) {
        part[0] = m[i];
        part[1] = S;
      }
      *reinterpret_cast<float4*>(part + 2 + 4 * lane) = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
    }
  }
}

// Prefill: K/V rows of positions pos0..pos0+T-1, before any block pass reads
// them.  grid (T, kv_heads); one wave.
__global__ __launch_bounds__(64) void attn_store_kv_kernel(AttnArgs a) {
  const int t = blockIdx.x, kvh = blockIdx.y, lane = threadIdx.x;
  const int pos = a.pos0 + t;
  if (pos < 0 || pos >= a.max_seq) return;
  float v[4];
  load4h(a.k + (size_t)t * 512 + kvh * kHeadDim + 4 * lane, v);
  head_norm_wave(v, a.k_norm_w, lane);
  rope_wave(v, a.rope + (size_t)pos * 64, lane);
  uint16_t* row = a.kv + (size_t)pos * kKvRow;
  *reinterpret_cast<uint2*>(row + kvh * kHeadDim + 4 * lane) = pack4h(v);
  *reinterpret_cast<uint2*>(row + 512 + kvh * kHeadDim + 4 * lane) =
      *reinterpret_cast<const uint2*>(a.v + (size_t)t * 512 + kvh * kHeadDim + 4 * lane);
}

// grid (8 query heads, T); block 256 (thread = output dim).  Blocks are
// combined in order.  The O partials of the first 16 blocks are loaded
// together with the m/S values, ahead of the max reduction; later blocks'
// partials are loaded 8 at a time so the loads are in flight together.
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a) {
  __shared__ float cfac[1024], sfac[1024];
  __shared__ float red[257];
  constexpr int kPre = 16;
  const int qh = blockIdx.x, t = blockIdx.y, d = threadIdx.x;
  const int pos = a.pos_dev ? a.pos_dev[0] : a.pos0 + t;
  if (pos < 0 || pos >= a.max_seq) return;
  const int nb = (pos + kAttnBlock) / kAttnBlock;  // <= max_blocks <= 1024
  const float* part = a.part + ((size_t)t * kQHeads + qh) * a.max_blocks * kPartFloats;
  const uint16_t g16 = a.qg[(size_t)t * 4096 + qh * 512 + 256 + d];
  float ov0[kPre];
#pragma unroll
  for (int i = 0; i < kPre; ++i) ov0[i] = part[(size_t)min(i, nb - 1) * kPartFloats + 2 + d];
  float M = -INFINITY;
  for (int b = d; b < nb; b += 256) {
    const float m = part[(size_t)b * kPartFloats];
    cfac[b] = m;
    sfac[b] = part[(size_t)b * kPartFloats + 1];
    M = fmaxf(M, m);
  }
  red[d] = M;
  __syncthreads();
  if (d < 64) {
    float m = fmaxf(fmaxf(red[d], red[d + 64]), fmaxf(red[d + 128], red[d + 192]));
    m = spk::wave_max(m);
    if (d == 0) red[256] = m;
  }
  __syncthreads();
  M = red[256];
  for (int b = d; b < nb; b += 256) cfac[b] = spk::expf_det(cfac[b] - M);
  __syncthreads();
  float tot = 0.0f, o = 0.0f;
#pragma unroll
  for (int i = 0; i < kPre; ++i) {
    if (i < nb) {
      const float c = cfac[i];
      tot = tot + sfac[i] * c;
      o = o + ov0[i] * c;
    }
  }
  for (int b0 = kPre; b0 < nb; b0 += 8) {
    float ov[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) ov[i] = part[(size_t)min(b0 + i, nb - 1) * kPartFloats + 2 + d];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (b0 + i < nb) {
        const float c = cfac[b0 + i];
        tot = tot + sfac[b0 + i] * c;
        o = o + ov[i] * c;
      }
    }
  }
  const float att = round16(o * (1.0f / (tot + 1e-30f)));
  const float g = spk::h2f(g16);
  const float sig = 1.0f / (1.0f + spk::expf_det(-g));
  a.out[(size_t)t * 2048 + qh * kHeadDim + d] = spk::f2h(att * sig);
}

// ---------------------------------------------------------------------------
// Element-wise kernels
// ---------------------------------------------------------------------------

// RMSNorm(1+w) of rows of 1024 (one 256-thread block per row).
__global__ __launch_bounds__(256) void rmsnorm1024_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w,
                                                          uint16_t* __restrict__ y) {
  __shared__ float red[257];
  const int tid = threadIdx.x;
  const size_t base = (size_t)blockIdx.x * kHidden + 4 * tid;
  float v[4], wf[4];
  load4h(x + base, v);
  load4h(w + 4 * tid, wf);
  float p = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) p = __builtin_fmaf(v[i], v[i], p);
  const float sum = block_tree256(p, red);
  const float nf = 1.0f / __builtin_sqrtf(sum / 1024.0f + 1e-6f);
  float o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (v[i] * nf) * (1.0f + wf[i]);
  *reinterpret_cast<uint2*>(y + base) = pack4h(o);
}

// Per-head RMSNorm(1+w) over rows of 256 (one wave per row, 4 rows per block).
__global__ __launch_bounds__(256) void rmsnorm256_kernel(const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ w,
                                                         uint16_t* __restrict__ y, int rows) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  float v[4];
  load4h(x + (size_t)row * kHeadDim + 4 * lane, v);
  head_norm_wave(v, w, lane);
  *reinterpret_cast<uint2*>(y + (size_t)row * kHeadDim + 4 * lane) = pack4h(v);
}

__global__ void silu_gate_kernel(const uint16_t* __restrict__ g, const uint16_t* __restrict__ u,
                                 uint16_t* __restrict__ y, long long n) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
    y[i] = spk::f2h(spk::silu_det(spk::h2f(g[i])) * spk::h2f(u[i]));
}

__global__ void residual_add_kernel(const uint16_t* __restrict__ a, const uint16_t* __restrict__ b,
                                    uint16_t* __restrict__ y, long long n) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long long)gridDim.x * blockDim.x)
    y[i] = spk::f2h(spk::h2f(a[i]) + spk::h2f(b[i]));
}

// embedding_lookup.comp: y[t] = E[tokens[t]] (rows of 1024); ids outside
// [0, vocab) give a zero row.
__global__ __launch_bounds__(128) void embedding_kernel(const uint16_t* __restrict__ E,
                                                        const int32_t* __restrict__ tokens, int vocab,
                                                        uint16_t* __restrict__ y) {
  const int t = blockIdx.x;
  const int id = tokens[t];
  uint4 v = make_uint4(0, 0, 0, 0);
  if (id >= 0 && id < vocab) v = reinterpret_cast<const uint4*>(E + (size_t)id * kHidden)[threadIdx.x];
  reinterpret_cast<uint4*>(y + (size_t)t * kHidden)[threadIdx.x] = v;
}

// ---------------------------------------------------------------------------
// Final norm + tied lm_head + argmax in one launch (rms_norm.comp,
// lm_head_tiled.comp, argmax.comp): the RMSNorm(1+w) of h is recomputed by
// every workgroup while its weight rows are in flight (the fused GEMV's
// prologue), each wavefront streams R vocabulary rows with non-temporal
// 16-byte loads, and the workgroup's argmax key is folded into one of 64
// device words with a device-scope atomic max (posted: no return, no wait).
// One word for all workgroups serialises the atomics (measured: 7,760 of them
// add ~34 us to a 85 us stream); workgroup b uses word b % 64.  The take
// kernel of the next launch reduces and clears the 64 words.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// One-launch form: the workgroups' keys go to one slot each (agent-scope
// store, posted: no compute workgroup waits on a memory round trip), and one
// extra workgroup -- the last id, so the last dispatched -- polls the slots
// until every one is filled (the early ones first, then the last few
// thousand, take_slots), reduces them, clears them and records the token.  A slot holds key + 1 (keys are below 2^64 - 1: the largest,
// +inf's, has 0xff800000 above), so 0 means "not written yet".  The poll is
// bounded: after kTakePolls rounds (seconds) it gives up and records index
// 0xffffffff, so the kernel always ends.
constexpr int kTakePolls = 1 << 21;

struct TakeArgs {
  unsigned long long* slots;
  int nblocks;
  uint32_t* out;
  int32_t* pos;
  int32_t* count;
  int32_t* history;
  int cap;
};

// Slots one thread of the taker reads per group, all issued before any is
// used: a poll is one memory round trip per 256 x kTakePer slots (read one
// after the other, each waited for, a poll of 7,760 slots took ~30 loads'
// latency).
constexpr int kTakePer = 8;
// The taker is dispatched last, when the first of the last few thousand
// workgroups has finished: it reads (and, once all are seen written, clears)
// the slots of every workgroup but the last 256 x kTakeTail while those still
// run, then polls only those, kTakeTail per thread, one round trip a poll.
// Every slot is cleared only after a poll has seen it written, except after
// a give-up (index 0xffffffff), when slots still being written can stay set.
constexpr int kTakeTail = 8;

// Polls slots [j_begin, j_end) until all are written (bounded); *best takes
// their maximum.  Returns whether one was still missing when it gave up.
template <int PER>
__device__ __forceinline__ int take_range(const TakeArgs& t, int j_begin, int j_end, unsigned long long* best) {
  const int tid = threadIdx.x;
  int missing = j_end > j_begin;
  for (int it = 0; it < kTakePolls && missing; ++it) {
    unsigned long long b = 0ull;
    int miss = 0;
    for (int j0 = j_begin; j0 < j_end; j0 += 256 * PER) {
      unsigned long long v[PER];
#pragma unroll
      for (int i = 0; i < PER; ++i)  // past the end: the last slot of the range again
        v[i] = __hip_atomic_load(t.slots + min(j0 + tid + 256 * i, j_end - 1), __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        b = spk::umax64(b, v[i]);
        miss |= (v[i] == 0ull);
      }
    }
    missing = __syncthreads_or(miss);
    if (missing) {
      __builtin_amdgcn_s_sleep(2);
    } else {
      *best = spk::umax64(*best, b);
    }
  }
  return missing;
}

__device__ __forceinline__ void take_slots(const TakeArgs& t, uint32_t E) {
  const int tid = threadIdx.x;
  const int tail0 = max(t.nblocks - 256 * kTakeTail, 0);
  unsigned long long best = 0ull;
  // the early slots: read, then cleared while the last workgroups still run
  int missing = take_range<kTakePer>(t, 0, tail0, &best);
  for (int j = tid; j < tail0; j += 256)
    __hip_atomic_store(t.slots + j, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the last workgroups' slots
  missing |= take_range<kTakeTail>(t, tail0, t.nblocks, &best);
  for (int j = tail0 + tid; j < t.nblocks; j += 256)
    __hip_atomic_store(t.slots + j, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  best = spk::block_max_u64<256>(best);
  if (tid == 0) {
    const uint32_t idx = missing ? 0xffffffffu : spk::key_to_index(best - 1ull, E);
    *t.out = idx;
    if (t.pos) {
      const int i = t.count[0];
      if (i >= 0 && i < t.cap) t.history[i] = (int32_t)idx;
      t.count[0] = i + 1;
      t.pos[0] = t.pos[0] + 1;
    }
  }
}

template <int N8, int R, bool NORM, bool ONE = false>
__global__ __launch_bounds__(256) void lm_head_key_kernel(const uint16_t* __restrict__ W,
                                                          const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ norm_w,
                                                          uint16_t* __restrict__ logits, int vocab,
                                                          uint32_t E, unsigned long long* key_out,
                                                          TakeArgs take) {
  if constexpr (ONE) {
    if ((int)blockIdx.x == take.nblocks) {
      take_slots(take, E);
      return;
    }
  }
  __shared__ float xs[512 * N8];
  __shared__ float red[257];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  constexpr int in_dim = 512 * N8;
  constexpr int NV = in_dim / 8;  // 16-byte pieces of x
  constexpr int PER = (NV + 255) / 256;
  static_assert(!NORM || N8 == 2, "the norm prologue is rms_norm.comp's over 1024");
  const int row0 = (blockIdx.x * 4 + wave) * R;
  uint2 hv = make_uint2(0, 0), nwv = make_uint2(0, 0);
  uint4 xv[PER];
  if constexpr (NORM) {
    hv = *reinterpret_cast<const uint2*>(x + 4 * tid);
    nwv = *reinterpret_cast<const uint2*>(norm_w + 4 * tid);
  } else {
#pragma unroll
    for (int c = 0; c < PER; ++c) xv[c] = *reinterpret_cast<const uint4*>(x + 8 * min(tid + 256 * c, NV - 1));
  }
  // rows loaded densely, regrouped into the span order after the prologue
  // (dense_rows.hpp)
  __shared__ uint4 rows_lds[4][64 * N8];
  uint4 wv[R][N8];
  spk::dense_rows_issue<N8, R, true>(W, row0, vocab, lane, wv);
  __builtin_amdgcn_sched_barrier(0);  // every weight row in flight before the prologue
  if constexpr (NORM) {
    const float v[4] = {spk::h2f(hv.x & 0xffffu), spk::h2f(hv.x >> 16), spk::h2f(hv.y & 0xffffu),
                        spk::h2f(hv.y >> 16)};
    const float w[4] = {spk::h2f(nwv.x & 0xffffu), spk::h2f(nwv.x >> 16), spk::h2f(nwv.y & 0xffffu),
                        spk::h2f(nwv.y >> 16)};
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) p = __builtin_fmaf(v[i], v[i], p);
    const float sum = block_tree256(p, red);
    const float nf = 1.0f / __builtin_sqrtf(sum / 1024.0f + 1e-6f);
#pragma unroll
    for (int i = 0; i < 4; ++i) xs[4 * tid + i] = round16((v[i] * nf) * (1.0f + w[i]));
  } else {
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const int idx = min(tid + 256 * c, NV - 1);
      float f[8];
      unpack8(xv[c], f);
#pragma unroll
      for (int e = 0; e < 8; e += 4) *reinterpret_cast<float4*>(&xs[8 * idx + e]) = make_float4(f[e], f[e + 1], f[e + 2], f[e + 3]);
    }
  }
  __syncthreads();
  float xf[8 * N8];
#pragma unroll
  for (int k = 0; k < 8 * N8; k += 4) {
    const float4 t = *reinterpret_cast<const float4*>(&xs[lane * (8 * N8) + k]);
    xf[k] = t.x;
    xf[k + 1] = t.y;
    xf[k + 2] = t.z;
    xf[k + 3] = t.w;
  }
  spk::dense_rows_regroup<N8, R>(wv, rows_lds[wave], lane);
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = lane_dot<N8>(wv[r], xf);
  spk::tree64_rows<R>(acc);
  unsigned long long key = 0ull;
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int row = row0 + r;
      if (row < vocab) {
        const uint16_t l16 = spk::f2h(acc[r]);
        if (logits) logits[row] = l16;
        key = spk::umax64(key, spk::argmax_key(spk::h2f(l16), (uint32_t)row, E));
      }
    }
  }
  key = spk::block_max_u64<256>(key);
  if constexpr (ONE) {
    if (tid == 0) __hip_atomic_store(take.slots + blockIdx.x, key + 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    if (tid == 0 && key != 0ull)
      __hip_atomic_fetch_max(key_out + (blockIdx.x & (SPK_ARGMAX_KEY_WORDS - 1)), key, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
}

// *out = index of the largest of the 64 key words (which are then zeroed);
// with pos != NULL also the greedy loop's bookkeeping of record_token_kernel.
// One wavefront: lane l takes word l.
__global__ __launch_bounds__(64) void argmax_take_kernel(unsigned long long* key, uint32_t E, uint32_t* out,
                                                         int32_t* pos, int32_t* count, int32_t* history, int cap) {
  unsigned long long k = __hip_atomic_exchange(key + threadIdx.x, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  k = spk::wave_max_u64(k);
  if (threadIdx.x == 0) {
    const uint32_t idx = spk::key_to_index(k, E);
    *out = idx;
    if (pos) {
      const int i = count[0];
      if (i >= 0 && i < cap) history[i] = (int32_t)idx;
      count[0] = i + 1;
      pos[0] = pos[0] + 1;
    }
  }
}

__global__ void add_i32_kernel(int32_t* p, int32_t delta) {
  if (threadIdx.x == 0) p[0] += delta;
}

__global__ void record_token_kernel(const int32_t* token, int32_t* pos, int32_t* count, int32_t* history, int cap) {
  if (threadIdx.x == 0) {
    const int i = count[0];
    if (i >= 0 && i < cap) history[i] = token[0];
    count[0] = i + 1;
    pos[0] = pos[0] + 1;
  }
}

int grid_for(long long n) {
  long long b = (n + 255) / 256;
  return (int)(b > 4096 ? 4096 : (b < 1 ? 1 : b));
}


// ---------------------------------------------------------------------------
// DeltaNet layer input of a batch-1 decode step in one launch: the input
// RMSNorm and the q/k/v/z/a/b projections (fused_gemv_kernel's RMSNORM
// arithmetic, bit for bit), then each head's decode step (spk_dn::dn_step on
// the workgroup's NW wavefronts) in the last of the head's workgroups to
// finish.  Workgroup id = 8 (2i + h/8) + h%8 forms rows 2NW i .. 2NW i+2NW-1
// of head h's 512 q|k|v|z rows, so a head's workgroups have ids congruent
// mod 8: workgroups are dealt to the 8 XCDs round-robin, so they share one
// L2, which holds their rows for the head's step.  Each workgroup waits for
// its row stores, then adds one to the head's arrival count (relaxed
// atomic); the one that sees the count complete runs the step and resets the
// count for the next launch.  The 16 counts sit on separate cache lines (on
// one line the 1,024 atomics serialised: 20.3 us per launch against 11.0).
// Every workgroup also loads the head's a and b weight rows with its own,
// so the last one forms a and b without another round trip, and brings a
// share of the head's state and conv rows into the L2, so the step's first
// operands do not come from HBM (config 4: 676.4 -> 666.0 us per token).
// Measured per token, config 4, against the two launches: 4 wavefronts
// 666.0 vs 678.8 us, 8 wavefronts 660.5-661.6 vs 679.0-680.4, 16
// wavefronts 668.7 vs 680.6.
// ---------------------------------------------------------------------------
constexpr int kDnArriveStride = 64;  // ints between two heads' counts (256 B: own cache lines)
constexpr int kDnWaves = 8;          // wavefronts per workgroup

struct InprojStep {
  const uint16_t* x;       // hidden [1024], or the embedding table when token != NULL
  const uint16_t* norm_w;  // input RMSNorm weight [1024]
  const int32_t* token;
  int token_rows;
  uint16_t* h_out;  // the embedding row (layer 0), or NULL
  const uint16_t* Wqkv;
  const uint16_t* Wz;
  const uint16_t* Wa;
  const uint16_t* Wb;
  uint16_t* qkv;
  uint16_t* z;
  uint16_t* a;
  uint16_t* b;
  int32_t* arrive;  // [16 * kDnArriveStride]
  spk_dn::DecodeParams dp;
};

template <int NW>
__global__ __launch_bounds__(NW * 64) void dn_inproj_step_kernel(InprojStep s) {
  constexpr int kPieces = 256 / NW;  // workgroups per head (2 rows per wavefront)
  __shared__ float xs[kHidden];
  __shared__ float red[257];
  __shared__ int last;
  const int id = blockIdx.x;
  const int h = (id & 7) + 8 * ((id >> 3) & 1);
  const int piece = id >> 4;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // rows r, r+1 of the head's q|k|v|z block (region 0..3 = q, k, v, z)
  const int r = 2 * NW * piece + 2 * wave;
  const int region = r >> 7;
  const uint16_t* W = region < 3 ? s.Wqkv : s.Wz;
  uint16_t* y = region < 3 ? s.qkv : s.z;
  const int row = (region < 3 ? region * 2048 : 0) + h * 128 + (r & 127);

  // input operands first, then the weight rows (fused_gemv_kernel's order)
  const uint16_t* hsrc = s.x;
  if (s.token) {
    const int tk = s.token[0];
    hsrc += (size_t)((tk >= 0 && tk < s.token_rows) ? tk : 0) * kHidden;
  }
  // Each operand is loaded only by the wavefronts that use it (the CU's
  // memory pipe takes one wavefront load instruction at a time, whatever its
  // width): the norm input by the 256 threads of the norm prologue, the a/b
  // rows by wavefront 3 (the last workgroup's forms a and b and, as the
  // step's g/beta wavefront, uses them).  Values a wavefront
  // skips start opaque (spk_dn::opaque_u32), so no load meets a constant at
  // a branch join, where the compiler would wait for it.
  const int t4 = 4 * (tid & 255);
  uint2 hv = make_uint2(spk_dn::opaque_u32(), spk_dn::opaque_u32());
  uint2 nwv = make_uint2(spk_dn::opaque_u32(), spk_dn::opaque_u32());
  if (tid < 256) {
    hv = *reinterpret_cast<const uint2*>(hsrc + t4);
    nwv = *reinterpret_cast<const uint2*>(s.norm_w + t4);
  }
  uint4 wv[2][2], wab[2][2];
  load_rows<2, 2>(W, row, row + 2, lane, wv);
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int k = 0; k < 2; ++k)
      wab[i][k] = make_uint4(spk_dn::opaque_u32(), spk_dn::opaque_u32(), spk_dn::opaque_u32(), spk_dn::opaque_u32());
  if (wave == 3) {
    load_rows<2, 1>(s.Wa, h, h + 1, lane, *reinterpret_cast<uint4(*)[1][2]>(&wab[0]));
    load_rows<2, 1>(s.Wb, h, h + 1, lane, *reinterpret_cast<uint4(*)[1][2]>(&wab[1]));
  }
  // the head's step operands into this XCD's L2 for the last workgroup, one
  // 128-byte line per lane of wavefront 0: lanes 0-15 the workgroup's 16
  // lines (2 KiB) of the head's 64 KiB state, lanes 16-17 two of the 48 lines
  // of its six 1 KiB conv rows (state q|k|v, weights q|k|v), spread over the
  // head's first 24 workgroups
  static_assert(kPieces * 16 * 128 == 16384 * 4, "16 state lines per workgroup");
  uint32_t touch = spk_dn::opaque_u32();
  {
    const int cl = 2 * piece + (lane - 16);  // conv line of lanes 16, 17
    if (wave == 0 && (lane < 16 || (lane < 18 && cl < 48))) {
      const char* tp;
      if (lane < 16) {
        tp = reinterpret_cast<const char*>(s.dp.state + (size_t)h * 16384) + (size_t)(16 * piece + lane) * 128;
      } else {
        const int row = cl >> 3;
        const uint16_t* cbase = row < 3 ? s.dp.conv_state : s.dp.conv_w;
        tp = reinterpret_cast<const char*>(cbase + ((row % 3) * 2048 + h * 128) * 4) + (cl & 7) * 128;
      }
      touch = *reinterpret_cast<const uint32_t*>(tp);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // every load in flight before the prologue
  {
    const float v[4] = {spk::h2f(hv.x & 0xffffu), spk::h2f(hv.x >> 16), spk::h2f(hv.y & 0xffffu),
                        spk::h2f(hv.y >> 16)};
    const float w[4] = {spk::h2f(nwv.x & 0xffffu), spk::h2f(nwv.x >> 16), spk::h2f(nwv.y & 0xffffu),
                        spk::h2f(nwv.y >> 16)};
    float pp = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) pp = __builtin_fmaf(v[i], v[i], pp);
    // rms_norm.comp's 256-partial tree over the first 256 threads' partials
    const float sum = block_tree256(pp, red);
    const float nf = 1.0f / __builtin_sqrtf(sum / 1024.0f + 1e-6f);
    if (tid < 256) {
#pragma unroll
      for (int i = 0; i < 4; ++i) xs[t4 + i] = round16((v[i] * nf) * (1.0f + w[i]));
    }
  }
  __syncthreads();
  float xf[16];
#pragma unroll
  for (int k = 0; k < 16; k += 4) {
    const float4 t = *reinterpret_cast<const float4*>(&xs[lane * 16 + k]);
    xf[k] = t.x;
    xf[k + 1] = t.y;
    xf[k + 2] = t.z;
    xf[k + 3] = t.w;
  }
  float acc[2] = {lane_dot<2>(wv[0], xf), lane_dot<2>(wv[1], xf)};
  spk::tree64_rows<2>(acc);
  if (lane == 0) {
    y[row] = spk::f2h(acc[0]);
    y[row + 1] = spk::f2h(acc[1]);
  }
  if (s.h_out && id == 0 && tid < 256) *reinterpret_cast<uint2*>(s.h_out + t4) = hv;

  // arrival: this workgroup's row stores (and the L2 touches) complete, then
  // one count per workgroup
  asm volatile("" ::"v"(touch));
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    last = __hip_atomic_fetch_add(s.arrive + h * kDnArriveStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           kPieces - 1;
  __syncthreads();
  if (!last) return;
  if (tid == 0) __hip_atomic_store(s.arrive + h * kDnArriveStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // a[h] and b[h] (the projections' order) by wavefront 3, the step's g/beta
  // wavefront, which alone reads them (in lane 0): no barrier before the step
  uint16_t a_h = 0, b_h = 0;
  if (wave == 3) {
    float t[2] = {lane_dot<2>(wab[0], xf), lane_dot<2>(wab[1], xf)};
    spk::tree64_rows<2>(t);
    a_h = spk::f2h(t[0]);
    b_h = spk::f2h(t[1]);
    if (lane == 0) {
      s.a[h] = a_h;
      s.b[h] = b_h;
    }
  }
  spk_dn::dn_step<true, true, false, true, NW, true>(s.dp, h, 0, a_h, b_h);
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

// One launch of up to kLaunchOut outputs of spk_gemv_fused (validated by the
// caller); only the first launch of a call writes h_out.
static int launch_fused_gemv(const SpkGemvInput* in, const SpkGemvOutput* outs, int count, bool first, int n8, int R,
                             spk_stream_t stream, const uint16_t* touch = nullptr, const int32_t* touch_pos = nullptr,
                             int touch_rows = 0) {
  FusedGemv a;
  a.touch = touch;
  a.touch_pos = touch_pos;
  a.touch_rows = touch_rows;
  a.kind = in->kind;
  a.in_dim = in->in_dim;
  a.x = in->x;
  a.x2 = in->x2;
  a.token = in->token;
  a.token_rows = in->token_rows;
  a.h_out = first ? in->h_out : nullptr;
  a.count = count;
  int blocks = 0;
  for (int i = 0; i < count; ++i) {
    a.W[i] = outs[i].W;
    a.W2[i] = outs[i].W_up;
    a.y[i] = outs[i].y;
    a.res[i] = outs[i].residual;
    a.out_dim[i] = outs[i].out_dim;
    a.first_block[i] = blocks;
    blocks += (outs[i].out_dim + 4 * R - 1) / (4 * R);
  }
  for (int i = count; i < kLaunchOut; ++i) {
    a.W[i] = nullptr; a.W2[i] = nullptr; a.y[i] = nullptr; a.res[i] = nullptr; a.out_dim[i] = 0;
    a.first_block[i] = blocks;
  }
  a.first_block[kLaunchOut] = blocks;
  hipStream_t s = spk::to_hip(stream);
  const bool pair = outs[0].W_up != nullptr;
#define SPK_FGK(n8, r, kind)                                                                            \
  if (pair)                                                                                             \
    hipLaunchKernelGGL((fused_gemv_kernel<n8, r, true, kind>), dim3(blocks), dim3(256), 0, s, a);       \
  else                                                                                                  \
    hipLaunchKernelGGL((fused_gemv_kernel<n8, r, false, kind>), dim3(blocks), dim3(256), 0, s, a);
#define SPK_FG(n8, r)                                                                                   \
  case n8:                                                                                              \
    if (in->kind == SPK_GEMV_IN_SILU_GATE) {                                                            \
      SPK_FGK(n8, r, SPK_GEMV_IN_SILU_GATE)                                                             \
    } else {                                                                                            \
      SPK_FGK(n8, r, SPK_GEMV_IN_PLAIN)                                                                 \
    }                                                                                                   \
    break;
  if (in->kind == SPK_GEMV_IN_RMSNORM) {  // in_dim == kHidden (checked above)
    if (touch)
      hipLaunchKernelGGL((fused_gemv_kernel<2, 2, false, SPK_GEMV_IN_RMSNORM, true>), dim3(blocks), dim3(256), 0, s, a);
    else {
      SPK_FGK(2, 2, SPK_GEMV_IN_RMSNORM)
    }
    return spk::check_launch("spk_gemv_fused");
  }
  switch (n8) {
    SPK_FG(1, 2)
    SPK_FG(2, 2)
    SPK_FG(3, 1)
    SPK_FG(4, 1)
    SPK_FG(5, 1)
    SPK_FG(6, 1)
    SPK_FG(7, 1)
    SPK_FG(8, 1)
    default: return spk::fail(SPK_ERR_SHAPE, "spk_gemv_fused: in_dim %d", in->in_dim);
  }
#undef SPK_FGK
#undef SPK_FG
  return spk::check_launch("spk_gemv_fused");
}

// spk_gemv_fused's argument contract (its messages name it).
static int gemv_fused_check(const SpkGemvInput* in, const SpkGemvOutput* outs, int32_t count) {
  if (!in || (count > 0 && !outs)) return spk::fail(SPK_ERR_NULL, "spk_gemv_fused: NULL argument");
  if (count < 1 || count > kMaxOut) return spk::fail(SPK_ERR_ARG, "spk_gemv_fused: count %d (1..%d)", count, kMaxOut);
  const int in_dim = in->in_dim;
  if (in->kind < SPK_GEMV_IN_PLAIN || in->kind > SPK_GEMV_IN_SILU_GATE)
    return spk::fail(SPK_ERR_ARG, "spk_gemv_fused: input kind %d", in->kind);
  if (in_dim <= 0 || in_dim % 512 != 0 || in_dim > kMaxIn)
    return spk::fail(SPK_ERR_SHAPE, "spk_gemv_fused: in_dim %d (multiple of 512, <= %d)", in_dim, kMaxIn);
  if (in->kind == SPK_GEMV_IN_RMSNORM && in_dim != kHidden)
    return spk::fail(SPK_ERR_SHAPE, "spk_gemv_fused: RMSNorm input needs in_dim %d", kHidden);
  if (!in->x || (in->kind != SPK_GEMV_IN_PLAIN && !in->x2))
    return spk::fail(SPK_ERR_NULL, "spk_gemv_fused: NULL input vector");
  if (in->kind != SPK_GEMV_IN_RMSNORM && (in->token || in->h_out))
    return spk::fail(SPK_ERR_ARG, "spk_gemv_fused: token/h_out need the RMSNorm input");
  if (in->token && in->token_rows <= 0)
    return spk::fail(SPK_ERR_SHAPE, "spk_gemv_fused: token_rows %d", in->token_rows);
  if (!spk::aligned(in->x, 16) || (in->x2 && !spk::aligned(in->x2, 16)) || (in->h_out && !spk::aligned(in->h_out, 16)))
    return spk::fail(SPK_ERR_ALIGN, "spk_gemv_fused: input vectors must be 16-byte aligned");
  for (int i = 0; i < count; ++i) {
    const SpkGemvOutput& o = outs[i];
    if (!o.W || !o.y) return spk::fail(SPK_ERR_NULL, "spk_gemv_fused: output %d has a NULL pointer", i);
    if (o.out_dim <= 0) return spk::fail(SPK_ERR_SHAPE, "spk_gemv_fused: output %d out_dim %d", i, o.out_dim);
    if (!spk::aligned(o.W, 16)) return spk::fail(SPK_ERR_ALIGN, "spk_gemv_fused: W %d must be 16-byte aligned", i);
    // y may be the residual (in-place update of the stream) but never an input of this launch.
    if (o.y == in->x || o.y == in->x2)
      return spk::fail(SPK_ERR_ARG, "spk_gemv_fused: output %d aliases the input vector", i);
    if ((o.W_up != nullptr) != (outs[0].W_up != nullptr))
      return spk::fail(SPK_ERR_ARG, "spk_gemv_fused: SiLU-gated pairs and plain outputs in one launch");
    if (o.W_up && !spk::aligned(o.W_up, 16))
      return spk::fail(SPK_ERR_ALIGN, "spk_gemv_fused: W_up %d must be 16-byte aligned", i);
  }
  return SPK_OK;
}

extern "C" int spk_gemv_fused(const SpkGemvInput* in, const SpkGemvOutput* outs, int32_t count,
                              spk_stream_t stream) {
  if (int rc = gemv_fused_check(in, outs, count)) return rc;
  const int in_dim = in->in_dim;
  const int n8 = in_dim / 512;
  const int R = n8 <= 2 ? 2 : 1;
  for (int c0 = 0; c0 < count; c0 += kLaunchOut) {
    const int rc = launch_fused_gemv(in, outs + c0, (count - c0 < kLaunchOut ? count - c0 : kLaunchOut), c0 == 0, n8, R, stream);
    if (rc) return rc;
  }
  return SPK_OK;
}

extern "C" int spk_attention_inproj(const SpkGemvInput* in, const SpkGemvOutput* outs, const SpkAttnArgs* attn,
                                    spk_stream_t stream) {
  const char* name = "spk_attention_inproj";
  if (!in || !outs || !attn) return spk::fail(SPK_ERR_NULL, "%s: NULL argument", name);
  if (in->kind != SPK_GEMV_IN_RMSNORM)
    return spk::fail(SPK_ERR_ARG, "%s: the input must be the RMSNorm kind", name);
  if (!attn->kv_cache || !attn->pos_dev) return spk::fail(SPK_ERR_NULL, "%s: kv_cache/pos_dev NULL", name);
  if (attn->max_seq <= 0) return spk::fail(SPK_ERR_SHAPE, "%s: max_seq %d", name, attn->max_seq);
  if (!spk::aligned(attn->kv_cache, 16)) return spk::fail(SPK_ERR_ALIGN, "%s: kv_cache must be 16-byte aligned", name);
  static const int dims[3] = {4096, 512, 512};
  for (int i = 0; i < 3; ++i) {
    if (!outs[i].W || !outs[i].y) return spk::fail(SPK_ERR_NULL, "%s: output %d NULL", name, i);
    if (outs[i].out_dim != dims[i] || outs[i].residual || outs[i].W_up)
      return spk::fail(SPK_ERR_SHAPE, "%s: output %d must be a plain %d-row projection", name, i, dims[i]);
  }
  if (attn->qg != outs[0].y || attn->k != outs[1].y || attn->v != outs[2].y)
    return spk::fail(SPK_ERR_ARG, "%s: the attention's qg/k/v must be the projections' outputs", name);
  // the rest of the projections' contract is spk_gemv_fused's
  if (int rc = gemv_fused_check(in, outs, 3)) return rc;
  return launch_fused_gemv(in, outs, 3, true, 2, 2, stream, attn->kv_cache, attn->pos_dev, attn->max_seq);
}

extern "C" int spk_deltanet_inproj_step(const SpkGemvInput* in, const SpkGemvOutput* outs, const SpkDecodeArgs* d,
                                        int32_t* arrive, spk_stream_t stream) {
  if (!in || !outs || !d || !arrive) return spk::fail(SPK_ERR_NULL, "spk_deltanet_inproj_step: NULL argument");
  if (in->kind != SPK_GEMV_IN_RMSNORM || in->in_dim != kHidden || !in->x || !in->x2)
    return spk::fail(SPK_ERR_ARG, "spk_deltanet_inproj_step: the input must be the RMSNorm kind over %d", kHidden);
  if (in->token && in->token_rows <= 0)
    return spk::fail(SPK_ERR_SHAPE, "spk_deltanet_inproj_step: token_rows %d", in->token_rows);
  if (!spk::aligned(in->x, 16) || !spk::aligned(in->x2, 16) || (in->h_out && !spk::aligned(in->h_out, 16)))
    return spk::fail(SPK_ERR_ALIGN, "spk_deltanet_inproj_step: input vectors must be 16-byte aligned");
  static const int dims[4] = {3 * 2048, 2048, 16, 16};
  for (int i = 0; i < 4; ++i) {
    if (!outs[i].W || !outs[i].y) return spk::fail(SPK_ERR_NULL, "spk_deltanet_inproj_step: output %d NULL", i);
    if (outs[i].out_dim != dims[i] || outs[i].residual || outs[i].W_up)
      return spk::fail(SPK_ERR_SHAPE, "spk_deltanet_inproj_step: output %d must be a plain %d-row projection", i,
                       dims[i]);
    if (!spk::aligned(outs[i].W, 16)) return spk::fail(SPK_ERR_ALIGN, "spk_deltanet_inproj_step: W %d alignment", i);
    if (outs[i].y == in->x || outs[i].y == in->x2)
      return spk::fail(SPK_ERR_ARG, "spk_deltanet_inproj_step: output %d aliases the input", i);
  }
  if (d->batch != 1 || d->num_heads != 16)
    return spk::fail(SPK_ERR_SHAPE, "spk_deltanet_inproj_step: batch %d heads %d (batch 1, 16 heads)", d->batch,
                     d->num_heads);
  if (d->qkv != outs[0].y || d->z != outs[1].y || d->a != outs[2].y || d->b != outs[3].y)
    return spk::fail(SPK_ERR_ARG, "spk_deltanet_inproj_step: the step's qkv/z/a/b must be the projections' outputs");
  if (!d->conv_state || !d->conv_weight || !d->state || !d->a_log_bias || !d->norm_weight)
    return spk::fail(SPK_ERR_NULL, "spk_deltanet_inproj_step: step buffer NULL");
  if (!spk::aligned(d->conv_state, 8) || !spk::aligned(d->conv_weight, 8) || !spk::aligned(d->state, 16))
    return spk::fail(SPK_ERR_ALIGN, "spk_deltanet_inproj_step: conv buffers 8-byte, state 16-byte aligned");
  if (d->layer_idx < 0) return spk::fail(SPK_ERR_ARG, "spk_deltanet_inproj_step: layer_idx < 0");
  InprojStep s;
  s.x = in->x;
  s.norm_w = in->x2;
  s.token = in->token;
  s.token_rows = in->token_rows;
  s.h_out = in->h_out;
  s.Wqkv = outs[0].W;
  s.Wz = outs[1].W;
  s.Wa = outs[2].W;
  s.Wb = outs[3].W;
  s.qkv = outs[0].y;
  s.z = outs[1].y;
  s.a = outs[2].y;
  s.b = outs[3].y;
  s.arrive = arrive;
  s.dp = spk_dn::make_params(d);
  hipLaunchKernelGGL(dn_inproj_step_kernel<kDnWaves>, dim3(16 * 256 / kDnWaves), dim3(64 * kDnWaves), 0,
                     spk::to_hip(stream), s);
  return spk::check_launch("spk_deltanet_inproj_step");
}

// the blocks' partials, then (decode with o_proj) two arrival counts on
// lines of their own
static size_t attn_partials_bytes(int32_t positions, int32_t tokens) {
  const size_t nb = ((size_t)positions + kAttnBlock - 1) / kAttnBlock;
  return (((size_t)tokens * kQHeads * nb * kPartFloats * sizeof(float)) + 255) / 256 * 256;
}

extern "C" size_t spk_attention_workspace_size(int32_t positions, int32_t tokens) {
  if (positions <= 0 || tokens <= 0) return 0;
  return attn_partials_bytes(positions, tokens) + 2 * 256;
}

static int attention_common(const SpkAttnArgs* p, int T, int positions, const char* who, AttnArgs& a,
                            bool need_out = true) {
  if (!p) return spk::fail(SPK_ERR_NULL, "%s: NULL args", who);
  if (!p->qg || !p->k || !p->v || !p->q_norm_w || !p->k_norm_w || !p->rope || !p->kv_cache ||
      (need_out && !p->out) || !p->workspace)
    return spk::fail(SPK_ERR_NULL, "%s: NULL pointer", who);
  if (p->max_seq <= 0 || p->max_seq > 65536 || T <= 0 || positions > 65536)
    return spk::fail(SPK_ERR_SHAPE, "%s: max_seq %d (at most 65536) tokens %d", who, p->max_seq, T);
  if (p->workspace_bytes < spk_attention_workspace_size(positions, T))
    return spk::fail(SPK_ERR_ARG, "%s: workspace %zu < %zu bytes", who, p->workspace_bytes,
                     spk_attention_workspace_size(positions, T));
  const void* ptrs[] = {p->qg, p->k, p->v, p->q_norm_w, p->k_norm_w, p->kv_cache, need_out ? p->out : p->qg,
                        p->workspace};
  for (const void* q : ptrs)
    if (!spk::aligned(q, 16)) return spk::fail(SPK_ERR_ALIGN, "%s: buffers must be 16-byte aligned", who);
  a.qg = p->qg;
  a.k = p->k;
  a.v = p->v;
  a.q_norm_w = p->q_norm_w;
  a.k_norm_w = p->k_norm_w;
  a.rope = p->rope;
  a.kv = p->kv_cache;
  a.max_seq = p->max_seq;
  a.out = p->out;
  a.part = static_cast<float*>(p->workspace);
  a.max_blocks = (positions + kAttnBlock - 1) / kAttnBlock;
  a.tokens = T;
  return SPK_OK;
}

extern "C" int spk_attention_decode(const SpkAttnArgs* p, spk_stream_t stream) {
  AttnArgs a;
  int rc = attention_common(p, 1, p ? p->max_seq : 0, "spk_attention_decode", a);
  if (rc) return rc;
  if (!p->pos_dev) return spk::fail(SPK_ERR_NULL, "spk_attention_decode: NULL pos_dev");
  a.pos_dev = p->pos_dev;
  a.pos0 = 0;
  a.store_kv = 1;
  hipStream_t s = spk::to_hip(stream);
  hipLaunchKernelGGL(attn_blocks_kernel<false>, dim3(a.max_blocks, kKvHeads, 1), dim3(256), 0, s, a);
  rc = spk::check_launch("spk_attention_decode (blocks)");
  if (rc) return rc;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(kQHeads, 1), dim3(256), 0, s, a);
  return spk::check_launch("spk_attention_decode (combine)");
}

extern "C" int spk_attention_decode_oproj(const SpkAttnArgs* p, const SpkGemvOutput* o_proj, spk_stream_t stream) {
  const char* name = "spk_attention_decode_oproj";
  if (!o_proj || !o_proj->W || !o_proj->y) return spk::fail(SPK_ERR_NULL, "%s: NULL o_proj", name);
  if (o_proj->W_up || o_proj->out_dim <= 0)
    return spk::fail(SPK_ERR_SHAPE, "%s: o_proj out_dim %d (single projection)", name, o_proj->out_dim);
  if (!spk::aligned(o_proj->W, 16)) return spk::fail(SPK_ERR_ALIGN, "%s: o_proj W must be 16-byte aligned", name);
  AttnArgs a;
  int rc = attention_common(p, 1, p ? p->max_seq : 0, name, a);
  if (rc) return rc;
  if (!p->pos_dev) return spk::fail(SPK_ERR_NULL, "%s: NULL pos_dev", name);
  if (o_proj->y == p->out || o_proj->residual == p->out)
    return spk::fail(SPK_ERR_ARG, "%s: o_proj output aliases the attention output", name);
  a.pos_dev = p->pos_dev;
  a.pos0 = 0;
  a.store_kv = 1;
  a.arrive = reinterpret_cast<int32_t*>(static_cast<char*>(p->workspace) + attn_partials_bytes(p->max_seq, 1));
  hipStream_t s = spk::to_hip(stream);
  hipLaunchKernelGGL(attn_blocks_kernel<true>, dim3(8 * a.max_blocks), dim3(256), 0, s, a);
  rc = spk::check_launch(name);
  if (rc) return rc;
  SpkGemvInput gi{};
  gi.kind = SPK_GEMV_IN_PLAIN;
  gi.in_dim = kQHeads * kHeadDim;
  gi.x = p->out;
  return launch_fused_gemv(&gi, o_proj, 1, true, 4, 1, stream);
}

extern "C" int spk_attention_prefill(const SpkAttnArgs* p, int32_t pos0, int32_t tokens, spk_stream_t stream) {
  if (!p) return spk::fail(SPK_ERR_NULL, "spk_attention_prefill: NULL args");
  if (pos0 < 0 || tokens <= 0 || pos0 + tokens > p->max_seq)
    return spk::fail(SPK_ERR_SHAPE, "spk_attention_prefill: positions [%d, %d) exceed max_seq %d", pos0,
                     pos0 + tokens, p->max_seq);
  AttnArgs a;
  int rc = attention_common(p, tokens, pos0 + tokens, "spk_attention_prefill", a);
  if (rc) return rc;
  a.pos_dev = nullptr;
  a.pos0 = pos0;
  a.store_kv = 0;
  hipStream_t s = spk::to_hip(stream);
  // Tokens read the K/V rows of earlier tokens of the same call: all rows are
  // stored by one launch before the block passes read them.
  hipLaunchKernelGGL(attn_store_kv_kernel, dim3(tokens, kKvHeads), dim3(64), 0, s, a);
  rc = spk::check_launch("spk_attention_prefill (store)");
  if (rc) return rc;
  hipLaunchKernelGGL(attn_prefill_blocks_kernel, dim3(a.max_blocks, kKvHeads, (tokens + kAttnGroup - 1) / kAttnGroup),
                     dim3(256), 0, s, a);
  rc = spk::check_launch("spk_attention_prefill (blocks)");
  if (rc) return rc;
  hipLaunchKernelGGL(attn_combine_kernel, dim3(kQHeads, tokens), dim3(256), 0, s, a);
  return spk::check_launch("spk_attention_prefill (combine)");
}

extern "C" int spk_rmsnorm_f16(const uint16_t* x, const uint16_t* w, uint16_t* y, int32_t rows, int32_t n,
                               spk_stream_t stream) {
  if (!x || !w || !y) return spk::fail(SPK_ERR_NULL, "spk_rmsnorm_f16: NULL pointer");
  if (rows <= 0 || (n != kHidden && n != kHeadDim))
    return spk::fail(SPK_ERR_SHAPE, "spk_rmsnorm_f16: rows %d n %d (n must be 1024 or 256)", rows, n);
  if (!spk::aligned(x, 8) || !spk::aligned(w, 8) || !spk::aligned(y, 8))
    return spk::fail(SPK_ERR_ALIGN, "spk_rmsnorm_f16: 8-byte alignment required");
  hipStream_t s = spk::to_hip(stream);
  if (n == kHidden)
    hipLaunchKernelGGL(rmsnorm1024_kernel, dim3(rows), dim3(256), 0, s, x, w, y);
  else
    hipLaunchKernelGGL(rmsnorm256_kernel, dim3((rows + 3) / 4), dim3(256), 0, s, x, w, y, rows);
  return spk::check_launch("spk_rmsnorm_f16");
}

extern "C" int spk_silu_gate_f16(const uint16_t* g, const uint16_t* u, uint16_t* y, int64_t n, spk_stream_t stream) {
  if (!g || !u || !y) return spk::fail(SPK_ERR_NULL, "spk_silu_gate_f16: NULL pointer");
  if (n <= 0) return spk::fail(SPK_ERR_SHAPE, "spk_silu_gate_f16: n %lld", (long long)n);
  hipLaunchKernelGGL(silu_gate_kernel, dim3(grid_for(n)), dim3(256), 0, spk::to_hip(stream), g, u, y, (long long)n);
  return spk::check_launch("spk_silu_gate_f16");
}

extern "C" int spk_residual_add_f16(const uint16_t* a, const uint16_t* b, uint16_t* y, int64_t n,
                                    spk_stream_t stream) {
  if (!a || !b || !y) return spk::fail(SPK_ERR_NULL, "spk_residual_add_f16: NULL pointer");
  if (n <= 0) return spk::fail(SPK_ERR_SHAPE, "spk_residual_add_f16: n %lld", (long long)n);
  hipLaunchKernelGGL(residual_add_kernel, dim3(grid_for(n)), dim3(256), 0, spk::to_hip(stream), a, b, y, (long long)n);
  return spk::check_launch("spk_residual_add_f16");
}

extern "C" int spk_embedding_f16(const uint16_t* E, const int32_t* tokens, int32_t n_tokens, int32_t vocab,
                                 uint16_t* y, spk_stream_t stream) {
  if (!E || !tokens || !y) return spk::fail(SPK_ERR_NULL, "spk_embedding_f16: NULL pointer");
  if (n_tokens <= 0 || vocab <= 0) return spk::fail(SPK_ERR_SHAPE, "spk_embedding_f16: %d tokens, vocab %d", n_tokens, vocab);
  if (!spk::aligned(E, 16) || !spk::aligned(y, 16)) return spk::fail(SPK_ERR_ALIGN, "spk_embedding_f16: 16-byte alignment");
  hipLaunchKernelGGL(embedding_kernel, dim3(n_tokens), dim3(128), 0, spk::to_hip(stream), E, tokens, vocab, y);
  return spk::check_launch("spk_embedding_f16");
}

extern "C" int spk_add_i32(int32_t* p, int32_t delta, spk_stream_t stream) {
  if (!p) return spk::fail(SPK_ERR_NULL, "spk_add_i32: NULL pointer");
  hipLaunchKernelGGL(add_i32_kernel, dim3(1), dim3(64), 0, spk::to_hip(stream), p, delta);
  return spk::check_launch("spk_add_i32");
}

extern "C" int spk_lm_head_argmax_key(const uint16_t* W, const uint16_t* x, const uint16_t* norm_w,
                                      int32_t vocab, int32_t hidden, uint16_t* logits, uint64_t* key,
                                      spk_stream_t stream) {
  const char* name = "spk_lm_head_argmax_key";
  if (!W || !x || !key) return spk::fail(SPK_ERR_NULL, "%s: NULL pointer", name);
  if (vocab <= 0 || hidden <= 0 || hidden % 512 != 0 || hidden > 4096 || (norm_w && hidden != kHidden))
    return spk::fail(SPK_ERR_SHAPE, "%s: vocab %d hidden %d (multiple of 512, <= 4096; 1024 with norm_w)", name,
                     vocab, hidden);
  if (!spk::aligned(W, 16) || !spk::aligned(x, 16) || !spk::aligned(key, 8) || (norm_w && !spk::aligned(norm_w, 8)))
    return spk::fail(SPK_ERR_ALIGN, "%s: W/x must be 16-byte aligned, key and norm_w 8-byte", name);
  constexpr int R = kLmKeyRows;
  const uint32_t E = (uint32_t)((vocab + 255) / 256);
  const int blocks = (vocab + 4 * R - 1) / (4 * R);
  hipStream_t s = spk::to_hip(stream);
  auto* k = reinterpret_cast<unsigned long long*>(key);
  if (norm_w) {
    hipLaunchKernelGGL((lm_head_key_kernel<2, R, true>), dim3(blocks), dim3(256), 0, s, W, x, norm_w, logits,
                       vocab, E, k, TakeArgs{});
    return spk::check_launch(name);
  }
#define SPK_LMK_CASE(n8)                                                                                      \
  case n8:                                                                                                    \
    hipLaunchKernelGGL((lm_head_key_kernel<n8, R, false>), dim3(blocks), dim3(256), 0, s, W, x, nullptr,   \
                       logits, vocab, E, k, TakeArgs{});                                                      \
    break;
  switch (hidden / 512) {
    SPK_LMK_CASE(1)
    SPK_LMK_CASE(2)
    SPK_LMK_CASE(3)
    SPK_LMK_CASE(4)
    SPK_LMK_CASE(5)
    SPK_LMK_CASE(6)
    SPK_LMK_CASE(7)
    SPK_LMK_CASE(8)
    default:
      return spk::fail(SPK_ERR_SHAPE, "%s: hidden %d", name, hidden);
  }
#undef SPK_LMK_CASE
  return spk::check_launch(name);
}

extern "C" int spk_argmax_key_take(uint64_t* key, int32_t vocab, uint32_t* out_index, int32_t* pos,
                                   int32_t* count, int32_t* history, int32_t capacity, spk_stream_t stream) {
  if (!key || !out_index) return spk::fail(SPK_ERR_NULL, "spk_argmax_key_take: NULL pointer");
  if (vocab <= 0) return spk::fail(SPK_ERR_SHAPE, "spk_argmax_key_take: vocab %d", vocab);
  if (pos && (!count || !history)) return spk::fail(SPK_ERR_NULL, "spk_argmax_key_take: count/history NULL with pos");
  const uint32_t E = (uint32_t)((vocab + 255) / 256);
  hipLaunchKernelGGL(argmax_take_kernel, dim3(1), dim3(64), 0, spk::to_hip(stream),
                     reinterpret_cast<unsigned long long*>(key), E, out_index, pos, count, history, capacity);
  return spk::check_launch("spk_argmax_key_take");
}

extern "C" size_t spk_lm_head_take_slots(int32_t vocab) {
  return vocab > 0 ? (size_t)((vocab + 4 * kLmKeyRows - 1) / (4 * kLmKeyRows)) : 0;
}

extern "C" int spk_lm_head_argmax_take(const uint16_t* W, const uint16_t* x, const uint16_t* norm_w, int32_t vocab,
                                       int32_t hidden, uint16_t* logits, uint64_t* slots, size_t slot_words,
                                       uint32_t* out_index, int32_t* pos, int32_t* count, int32_t* history,
                                       int32_t capacity, spk_stream_t stream) {
  const char* name = "spk_lm_head_argmax_take";
  if (!W || !x || !slots || !out_index) return spk::fail(SPK_ERR_NULL, "%s: NULL pointer", name);
  if (vocab > 0 && slot_words < spk_lm_head_take_slots(vocab))
    return spk::fail(SPK_ERR_ARG, "%s: %zu slot words < %zu for vocab %d", name, slot_words,
                     spk_lm_head_take_slots(vocab), vocab);
  if (pos && (!count || !history)) return spk::fail(SPK_ERR_NULL, "%s: count/history NULL with pos", name);
  if (vocab <= 0 || hidden <= 0 || hidden % 512 != 0 || hidden > 4096 || (norm_w && hidden != kHidden))
    return spk::fail(SPK_ERR_SHAPE, "%s: vocab %d hidden %d (multiple of 512, <= 4096; 1024 with norm_w)", name,
                     vocab, hidden);
  if (!spk::aligned(W, 16) || !spk::aligned(x, 16) || !spk::aligned(slots, 8) || (norm_w && !spk::aligned(norm_w, 8)))
    return spk::fail(SPK_ERR_ALIGN, "%s: W/x must be 16-byte aligned, slots and norm_w 8-byte", name);
  constexpr int R = kLmKeyRows;
  const uint32_t E = (uint32_t)((vocab + 255) / 256);
  const int blocks = (int)spk_lm_head_take_slots(vocab);
  const TakeArgs take{reinterpret_cast<unsigned long long*>(slots), blocks, out_index, pos, count, history, capacity};
  hipStream_t s = spk::to_hip(stream);
  // one more workgroup than the rows need: the last one takes the argmax
  if (norm_w) {
    hipLaunchKernelGGL((lm_head_key_kernel<2, R, true, true>), dim3(blocks + 1), dim3(256), 0, s, W, x, norm_w,
                       logits, vocab, E, nullptr, take);
    return spk::check_launch(name);
  }
#define SPK_LMT_CASE(n8)                                                                                      \
  case n8:                                                                                                    \
    hipLaunchKernelGGL((lm_head_key_kernel<n8, R, false, true>), dim3(blocks + 1), dim3(256), 0, s, W, x,    \
                       nullptr, logits, vocab, E, nullptr, take);                                             \
    break;
  switch (hidden / 512) {
    SPK_LMT_CASE(1)
    SPK_LMT_CASE(2)
    SPK_LMT_CASE(3)
    SPK_LMT_CASE(4)
    SPK_LMT_CASE(5)
    SPK_LMT_CASE(6)
    SPK_LMT_CASE(7)
    SPK_LMT_CASE(8)
    default:
      return spk::fail(SPK_ERR_SHAPE, "%s: hidden %d", name, hidden);
  }
#undef SPK_LMT_CASE
  return spk::check_launch(name);
}

extern "C" int spk_record_token(const int32_t* token, int32_t* pos, int32_t* count, int32_t* history,
                                int32_t capacity, spk_stream_t stream) {
  if (!token || !pos || !count || !history) return spk::fail(SPK_ERR_NULL, "spk_record_token: NULL pointer");
  hipLaunchKernelGGL(record_token_kernel, dim3(1), dim3(64), 0, spk::to_hip(stream), token, pos, count, history,
                     capacity);
  return spk::check_launch("spk_record_token");
}
