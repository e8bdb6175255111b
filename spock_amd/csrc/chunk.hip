// chunk.hip -- gated-DeltaNet chunk prefill (WY/UT chunk rule) on fp32 MFMA.
//
// Math (deltanet_chunk.cpp:134-268, deltanet_chunk_prefill_tiled.comp:116-262):
// per (sequence, head) and chunk of C=64 tokens with cumulative log-decay
// gcum and Gamma_ij = exp(gcum_i - gcum_j):
//   L  = strict_lower(beta_i (k_i . k_j) Gamma_ij),   T = (I + L)^{-1}
//   U  = T (V * beta),   W = T (K * beta * e^gcum)
//   A  = lower(q_i . k_j * scale * Gamma_ij)
//   v_new = U - W S,  o = (Q scale e^gcum) S + A v_new,
//   S <- e^{gcum_last} S + (K e^{gcum_last - gcum})^T v_new.
// Computed here with T moved next to the matrices that meet it:
//   R  = V * beta - (K S) * beta e^gcum          (so v_new = T R)
//   o  = (Q scale e^gcum) S + (A T) R
//   S <- e^{gcum_last} S + K'^T R,  K' = T^T diag(e^{gcum_last - gcum}) K
// -- the same sums in another association (measured in fp32 against the
// reference algorithm: same distance from the fp64 result).  A T and K' do
// not depend on S, so all chunks form them in parallel; U, W and v_new are
// never stored.
//
// Two launches:
//  1. chunk_intra_kernel -- one workgroup per (chunk, head), all chunks of all
//     sequences in parallel.  Every global load is issued up front; K rows
//     are staged in LDS in the input type (34 KB of LDS for fp16, so four
//     workgroups share a CU).  K K^T and Q K^T are 16x16x4 fp32 MFMA tiles,
//     five independent accumulators per wavefront; T is inverted blockwise (4
//     diagonal 16x16 blocks by per-lane forward substitution, written over L's,
//     off-diagonal blocks T_IJ = -T_II sum_M L_IM T_MJ as MFMA products); A T
//     and K' are MFMA products over the nonzero blocks of T with Ks applied to
//     the K operand as it is read.  They go to the workspace with the
//     per-token scales.
//  2. chunk_state_kernel -- one workgroup per (sequence, head, 16-column tile
//     of the value dim): columns of S evolve independently, so the sequential
//     chunk scan runs on 8*H*num_seqs workgroups.  The 128x16 state tile lives
//     in LDS; wavefront M owns token block M of K S, Q S, R and the output,
//     and state rows 32M..32M+31 of the update (S += K'^T R), all 16x16x4
//     MFMA, with the next chunk's operands prefetched into registers during
//     the current one.
// MFMA operand trick: the contraction index of a 16x16x4 step is a free
// permutation, so lane (m = l%16, g = l/16) reads a float4 at k = 16u + 4g and
// feeds its elements to 4 consecutive steps; the B operand uses the same map.
#include <algorithm>
#include <type_traits>

#include "capi_common.hpp"
#include "numerics.hpp"

namespace {

typedef float f4v __attribute__((ext_vector_type(4)));

// Workspace record stores are non-temporal: the record is read back by the
// scan (a later launch, mostly on other XCDs), so keeping it dirty in the
// writer's L2 only adds to the end-of-launch write-back (config 2: 0.956 ->
// 0.949 ms per call).
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void ws_store(float* p, float a, float b, float c, float d) {
  const f4v v = {a, b, c, d};
  __builtin_nontemporal_store(v, reinterpret_cast<f4v*>(p));
}
__device__ __forceinline__ void ws_store(void* p, uint32_t a, uint32_t b) {
  const u32x2v v = {a, b};
  __builtin_nontemporal_store(v, reinterpret_cast<u32x2v*>(p));
}

constexpr int kC = 64;
constexpr int kD = 128;
// Workspace record per (chunk, head), in floats.  The chunk rule is stored
// with T = (I + L)^{-1} folded into the two matrices that meet it: with
// R = beta*V - (beta e^g ik)*(K S) (per-token row scales),
//   v_new = U - W S = T R,   o = Qs*(Q S) + (A T) R,
//   S' = e^{gL} S + K^T diag(Ks) v_new = e^{gL} S + K'^T R,  K' = T^T diag(Ks) K,
// so the scan needs A T and K' (and raw K, Q, V from the input) instead of
// U, W and A: 49 KB of record instead of 74 KB, and the intra kernel never
// reads V.  The matrices are in the scan's MFMA fragment order: fragment f of
// wavefront M is 64 lanes x 4 consecutive elements, so every load of the scan
// reads one contiguous 1 KB block.  Loads whose 64 lanes touch 16 separate
// rows (the row-major alternative) cost the vector-memory pipe more per byte;
// the raw K and Q rows of stage A are read that way, 16 rows x 64 bytes per
// load (8 consecutive elements per lane), which measured as fast as a
// fragment-order copy of K in the record (at 16 rows x 32 bytes per load the
// copy had been 25% faster).  Lane l = 16*lg + li.
//   K'  [M 4][u 4][t 2][lane][4]  K'[16u+4lg+e][32M+2li+t]          fp32
//   AT  [M 4][J 4][lane][4]       (A T)[16M+li][16J+4lg+e], J <= M   fp32
//   Qs  [64] Q scale (q_scale iq e^gcum)
//   C1  [64] beta           C2 [64] beta e^gcum ik
//   Misc[0] e^{gL}
// A T's blocks above the diagonal (zero) are neither stored nor multiplied.
constexpr int kWsKp = 0;
constexpr int kWsA = 8192;
constexpr int kWsQs = 12288;
constexpr int kWsC1 = 12352;
constexpr int kWsC2 = 12416;
constexpr int kWsMisc = 12480;
constexpr int kWsStride = 12544;  // 50176 bytes, a multiple of 256
// Word 3 of a raw buffer resource on gfx9-family parts: 32-bit data format,
// which untyped loads/stores need for the num_records range check to apply.
constexpr int kBufDword3 = 0x00020000;

__device__ __forceinline__ f4v mfma4(float a, float b, f4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Sequences of a launch: with up to kSelMax of them the host fills the
// tables below from its copy of cu_seqlens, in the order the scan starts them
// (longest first), so no workgroup searches cu_seqlens (measured: config 2
// 1.01 -> 0.94 ms); with more (nsel == 0) the kernels find their sequence and
// chunk from the device cu_seqlens.  Workspace records use the pack's global
// chunk numbering.
constexpr int kSelMax = 32;
struct ChunkParams {
  int H;
  int N;
  int S;
  int l2;
  float q_scale;
  const void* q;
  const void* k;
  const void* v;
  const float* g;
  const float* beta;
  const float* init;
  float* core;
  long long core_hs;
  float* state;
  const int* cu;
  float* ws;
  int chunks;                   // workspace records per head (host count)
  int nsel;
  int sel_seq[kSelMax];         // sequence index (row of initial/out state)
  int sel_t0[kSelMax];          // its first token
  int sel_len[kSelMax];         // its tokens
  int sel_co[kSelMax];          // global index of its first chunk (workspace record)
  int sel_chunk0[kSelMax + 1];  // prefix sums of chunks over the table (intra grid)
};

__device__ __forceinline__ float4 load4(const float* p, size_t i) {
  return *reinterpret_cast<const float4*>(p + i);
}
__device__ __forceinline__ float4 load4(const uint16_t* p, size_t i) {
  const uint2 u = *reinterpret_cast<const uint2*>(p + i);
  return make_float4(spk::h2f((uint16_t)(u.x & 0xffffu)), spk::h2f((uint16_t)(u.x >> 16)),
                     spk::h2f((uint16_t)(u.y & 0xffffu)), spk::h2f((uint16_t)(u.y >> 16)));
}
__device__ __forceinline__ float load1(const float* p, size_t i) { return p[i]; }
__device__ __forceinline__ float load1(const uint16_t* p, size_t i) { return spk::h2f(p[i]); }

__device__ __forceinline__ float elem(const float4& v, int e) {
  return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}

// Span of sequence s from the device cu_seqlens (packs of more than kSelMax
// sequences).  The launch was sized from the host copy; a span that does not
// lie inside [0, N] counts as empty, and both kernels apply the same rule, so
// their workspace numbering agrees and no access leaves the tensors even if
// the device copy differs from the host one.
__device__ __forceinline__ int seq_span(const ChunkParams& p, int s, int& t0) {
  t0 = p.cu[s];
  const int t1 = p.cu[s + 1];
  return (t0 >= 0 && t1 >= t0 && t1 <= p.N) ? t1 - t0 : 0;
}

// Global chunk id -> (sequence, chunk within it, first token, valid tokens).
__device__ __forceinline__ void locate_chunk(const ChunkParams& p, int gchunk, int& seq,
                                             int& t0, int& len) {
  if (p.cu == nullptr) {
    seq = 0;
    t0 = gchunk * kC;
    len = min(kC, p.N - t0);
    return;
  }
  int acc = 0;
  for (int s = 0; s < p.S; ++s) {
    int ts;
    const int L = seq_span(p, s, ts);
    const int n = (L + kC - 1) / kC;
    if (gchunk < acc + n) {
      const int c = gchunk - acc;
      seq = s;
      t0 = ts + c * kC;
      len = min(kC, L - c * kC);
      return;
    }
    acc += n;
  }
  seq = -1;
  t0 = 0;
  len = 0;
}

// Raw (unconverted) element types: operands are loaded early and converted
// (and scaled) at use, so a load never stalls on arithmetic.
template <typename TIn> struct RawOf;
template <> struct RawOf<float> {
  static __device__ __forceinline__ float4 ld4(const float* p, size_t i) { return *reinterpret_cast<const float4*>(p + i); }
  static __device__ __forceinline__ float4 cvt4(const float4& r) { return r; }
  // 8 consecutive elements (two 16-byte loads), element i converted at use
  struct R8 {
    float4 a, b;
  };
  static __device__ __forceinline__ R8 ld8(const float* p) {
    return R8{*reinterpret_cast<const float4*>(p), *reinterpret_cast<const float4*>(p + 4)};
  }
  static __device__ __forceinline__ float get8(const R8& r, int i) { return elem(i < 4 ? r.a : r.b, i & 3); }
};
template <> struct RawOf<uint16_t> {
  // 4 halves kept as two 32-bit words in .x/.y of a float4
  static __device__ __forceinline__ float4 ld4(const uint16_t* p, size_t i) {
    const uint2 u = *reinterpret_cast<const uint2*>(p + i);
    return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), 0.f, 0.f);
  }
  static __device__ __forceinline__ float4 cvt4(const float4& r) {
    const uint32_t x = __float_as_uint(r.x), y = __float_as_uint(r.y);
    return make_float4(spk::h2f((uint16_t)(x & 0xffffu)), spk::h2f((uint16_t)(x >> 16)),
                       spk::h2f((uint16_t)(y & 0xffffu)), spk::h2f((uint16_t)(y >> 16)));
  }
  // 8 consecutive halves (one 16-byte load), half i converted at use
  typedef uint4 R8;
  static __device__ __forceinline__ R8 ld8(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
  static __device__ __forceinline__ float get8(const R8& r, int i) {
    const uint32_t w = (i >> 1) == 0 ? r.x : (i >> 1) == 1 ? r.y : (i >> 1) == 2 ? r.z : r.w;
    return spk::h2f((uint16_t)((i & 1) ? w >> 16 : w & 0xffffu));
  }
};

// V elements of the scan's stage B: row 16M+li, value columns n0+4lg..+3 (one
// 8-byte (fp16) or 16-byte (fp32) load per lane), read through a buffer
// resource of the chunk's len rows, so rows past the chunk read 0 (the
// hardware range check) with no clamp or select.
// The whole byte offset goes in the VGPR offset and the scalar offset stays 0:
// on gfx9-family raw buffers the range check compares only voffset +
// inst_offset with num_records, so a row offset passed as soffset would read
// past the chunk (the next sequence's rows, or past the tensor) unchecked.
template <typename TIn> struct VTile;
template <> struct VTile<float> {
  float x[4];
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, int voff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, 0);
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = __uint_as_float(v[e]);
  }
  __device__ __forceinline__ float get(int e) const { return x[e]; }
};
template <> struct VTile<uint16_t> {
  uint32_t x[2];
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t r, int voff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0);
    x[0] = v[0];
    x[1] = v[1];
  }
  __device__ __forceinline__ float get(int e) const {
    return spk::h2f((uint16_t)((e & 1) ? x[e / 2] >> 16 : x[e / 2] & 0xffffu));
  }
};

// K rows staged in LDS in the input type (fp16 rows stay fp16) with a
// row stride of 132 elements: the 16 rows of one 16-lane group of an 8-byte
// operand read (fp16), or the 8 rows of an 8-lane group of a 16-byte read
// (fp32), start on distinct bank groups.
template <typename TIn> struct RowStage;
template <> struct RowStage<uint16_t> {
  static constexpr int kLd = 132;  // halves (264 B)
  typedef uint16_t T;
  // raw: 4 halves as loaded by RawOf<uint16_t>::ld4
  static __device__ __forceinline__ void put4(T* s, int r, int c, const float4& raw) {
    *reinterpret_cast<uint2*>(s + r * kLd + c) = make_uint2(__float_as_uint(raw.x), __float_as_uint(raw.y));
  }
  static __device__ __forceinline__ float4 get4(const T* s, int r, int c) {
    const uint2 u = *reinterpret_cast<const uint2*>(s + r * kLd + c);
    return make_float4(spk::h2f((uint16_t)(u.x & 0xffffu)), spk::h2f((uint16_t)(u.x >> 16)),
                       spk::h2f((uint16_t)(u.y & 0xffffu)), spk::h2f((uint16_t)(u.y >> 16)));
  }
  static __device__ __forceinline__ float get1(const T* s, int r, int c) { return spk::h2f(s[r * kLd + c]); }
};
template <> struct RowStage<float> {
  static constexpr int kLd = 132;  // floats (528 B)
  typedef float T;
  static __device__ __forceinline__ void put4(T* s, int r, int c, const float4& raw) {
    *reinterpret_cast<float4*>(s + r * kLd + c) = raw;
  }
  static __device__ __forceinline__ float4 get4(const T* s, int r, int c) {
    return *reinterpret_cast<const float4*>(s + r * kLd + c);
  }
  static __device__ __forceinline__ float get1(const T* s, int r, int c) { return s[r * kLd + c]; }
};

// L is block lower triangular: its 10 blocks (I >= J) of 16x16 are stored
// packed, block (I,J) at (I(I+1)/2 + J) * 256, row-major with stride 16.  T =
// (I + L)^{-1} has the same shape.  Its diagonal blocks and its column-0
// blocks overwrite L's: L_II once solved, and L_I0 when T_I0 is formed, by the
// wavefront that is the last to read L_I0 (T_I0 is the last block of row I
// to be formed, by distance).  T_21, T_31 and T_32 go to a 3-block buffer of
// their own, since L_21, L_31 and L_32 are read again for T_20 and T_30.
// (With all six off-diagonal blocks in a buffer, the intra kernel held 34.3
// KB of LDS: 4 workgroups per CU instead of 5.)
__device__ __forceinline__ int blk(int I, int J) { return (I * (I + 1) / 2 + J) * 256; }
__device__ __forceinline__ int tslot(int I, int J) { return (I == 2 ? 0 : J) * 256; }  // (2,1), (3,1), (3,2)
// T's block (I, J), I >= J, once formed
__device__ __forceinline__ const float* tblk(const float* sL, const float* sT, int I, int J) {
  return (I == J || J == 0) ? sL + blk(I, J) : sT + tslot(I, J);
}

constexpr float kLog2e = 1.44269504f;

// Gram tiles of one wavefront: the K K^T row blocks I in KMASK (tiles J =
// 0..I each, rows 16I.., L's strict lower triangle) and, when QB >= 0, the
// K Q^T tiles of query block QB (J = 0..QB), which must be the wavefront's own
// Q rows (qa).  Without a split, wavefront W takes row block 3-W and query
// block W: five tiles each.  Each tile is one MFMA chain over the 128 key
// dims, the same whichever wavefront runs it and in whatever order, so the
// assignment never changes a value.  The chains are accumulated together so
// that the MFMA stream carries up to five independent ones, and the K rows of
// block J are read once for all of them.  A is produced transposed so that
// each lane holds four consecutive key positions of one query row: the
// A-operand fragment of the state scan.
struct GramTile {
  int I, J;
  bool q;  // K Q^T tile (query block I) rather than K K^T
};
template <unsigned KMASK, int QB>
__host__ __device__ constexpr int gram_ntiles() {
  int n = QB >= 0 ? QB + 1 : 0;
  for (int I = 0; I < 4; ++I)
    if ((KMASK >> I) & 1u) n += I + 1;
  return n;
}
template <unsigned KMASK, int QB>
__host__ __device__ constexpr GramTile gram_tile(int t) {
  for (int I = 3; I >= 0; --I)
    if ((KMASK >> I) & 1u) {
      if (t <= I) return GramTile{I, t, false};
      t -= I + 1;
    }
  return GramTile{QB, t, true};
}
template <unsigned KMASK, int QB>
__host__ __device__ constexpr int gram_nj() {  // K row blocks read: 0 .. nJ-1
  int m = QB;
  for (int I = 0; I < 4; ++I)
    if ((KMASK >> I) & 1u) m = I > m ? I : m;
  return m + 1;
}

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

template <typename TIn, unsigned KMASK, int QB>
__device__ __forceinline__ void gram_tiles(const typename RowStage<TIn>::T* sK, const float4 (&qa)[8],
                                           int li, int lg, f4v (&acc)[5]) {
  typedef RowStage<TIn> RS;
  typedef RawOf<TIn> R;
  constexpr int NT = gram_ntiles<KMASK, QB>();
  constexpr int nJ = gram_nj<KMASK, QB>();
  static_assert(NT <= 5, "at most five Gram tiles per wavefront");
#pragma unroll
  for (int t = 0; t < 5; ++t) acc[t] = f4v{0.f, 0.f, 0.f, 0.f};
  if constexpr (std::is_same<TIn, uint16_t>::value) {
    // fp16 inputs: the products of two halves are exact in fp32, so the
    // 16x16x32 f16 MFMA (fp32 accumulation) forms the same dot products as
    // the fp32 one up to the summation order, at 1/32 of its issue cycles.
    // Lane (li, lg) feeds keys 32v+4lg..+3 and 32v+16+4lg..+3 (its Q
    // registers qa[2v], qa[2v+1]) to both operands.
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      h8v kb[nJ];
#pragma unroll
      for (int J = 0; J < nJ; ++J) {
        const uint2 a = *reinterpret_cast<const uint2*>(sK + (16 * J + li) * RS::kLd + 32 * v + 4 * lg);
        const uint2 b = *reinterpret_cast<const uint2*>(sK + (16 * J + li) * RS::kLd + 32 * v + 16 + 4 * lg);
        kb[J] = __builtin_bit_cast(h8v, (u32x4v{a.x, a.y, b.x, b.y}));
      }
      const h8v qf = __builtin_bit_cast(h8v, (u32x4v{__float_as_uint(qa[2 * v].x), __float_as_uint(qa[2 * v].y),
                                                      __float_as_uint(qa[2 * v + 1].x),
                                                      __float_as_uint(qa[2 * v + 1].y)}));
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const GramTile g = gram_tile<KMASK, QB>(t);
        if (g.q)
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[g.J], qf, acc[t], 0, 0, 0);
        else
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kb[g.I], kb[g.J], acc[t], 0, 0, 0);
      }
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    float4 kb[nJ];
#pragma unroll
    for (int J = 0; J < nJ; ++J) kb[J] = RS::get4(sK, 16 * J + li, 16 * u + 4 * lg);
    const float4 qf = R::cvt4(qa[u]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const GramTile g = gram_tile<KMASK, QB>(t);
        if (g.q)
          acc[t] = mfma4(elem(kb[g.J], e), elem(qf, e), acc[t]);
        else
          acc[t] = mfma4(elem(kb[g.I], e), elem(kb[g.J], e), acc[t]);
      }
    }
  }
}

// Epilogue of the Gram tiles: L = strict_lower(beta_i k_i.k_j Gamma_ij) into
// LDS; A = lower(q_i.k_j scale Gamma_ij) stays in the K Q^T tiles' registers
// (replacing the raw dot products) until T is known and A T is formed (with
// the inverse L2 norms when requested; 1 otherwise).  iq_scale is the scale of
// query row 16 QB + li.
template <unsigned KMASK, int QB>
__device__ __forceinline__ void gram_store(f4v (&acc)[5], const float* sG, const float* sB, const float* sIK,
                                           float iq_scale, float* sL, int li, int lg) {
  constexpr int NT = gram_ntiles<KMASK, QB>();
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const GramTile g = gram_tile<KMASK, QB>(t);
    if (!g.q) {
      const int Ik = g.I, J = g.J;
      const int j = 16 * J + li;
      const float ikj = sIK[j];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * Ik + 4 * lg + r;
        const float dec = __builtin_amdgcn_exp2f((sG[i] - sG[j]) * kLog2e);
        sL[blk(Ik, J) + (4 * lg + r) * 16 + li] = (j < i) ? sB[i] * (acc[t][r] * (sIK[i] * ikj)) * dec : 0.0f;
      }
    } else {
      // lane (li, lg) holds A[i][j], i = 16QB + li, j = 16J + 4lg + r
      const int W = g.I, J = g.J;
      const int i = 16 * W + li;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 16 * J + 4 * lg + r;
        const float dec = __builtin_amdgcn_exp2f((sG[i] - sG[j]) * kLog2e);
        acc[t][r] = (j <= i) ? (acc[t][r] * (iq_scale * sIK[j])) * dec : 0.0f;
      }
    }
  }
}

// (A T)^T blocks of query block QB: lane (li, lg) of block (QB, K), K <= QB,
// ends up holding (A T)[16 QB + li][16K + 4lg + r] -- the A-operand fragment
// of the scan's stage C.  MFMA A operand T^T (T's block (J, K) read by
// column), B operand A^T (the lane's own A values of block J: acc[nK + J]).
// T is unit lower triangular, so the sum runs over J = K .. QB.
template <unsigned KMASK, int QB>
__device__ __forceinline__ void at_store(const f4v (&acc)[5], const float* sL, const float* sT, float* ws,
                                         int li, int lg, int lane) {
  if constexpr (QB >= 0) {
    constexpr int nK = gram_ntiles<KMASK, -1>();  // the K K^T tiles come first
#pragma unroll
    for (int K = 0; K <= QB; ++K) {
      f4v x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int J = K; J <= QB; ++J) {
        const float* tb = tblk(sL, sT, J, K);
#pragma unroll
        for (int e = 0; e < 4; ++e) x = mfma4(tb[(4 * lg + e) * 16 + li], acc[nK + J][e], x);
      }
      ws_store(ws + kWsA + ((QB * 4 + K) * 64 + lane) * 4, x[0], x[1], x[2], x[3]);
    }
  }
}

// Gram work of wavefront `wave` in part `part` of PARTS, dispatched to the
// instance (KMASK, QB) that holds it.  Without a split: row block 3-w and
// query block w (five tiles).  With one, only the wavefronts that own their
// A block (w % PARTS == part) form K Q^T tiles, and the ten K K^T tiles are
// spread so that no wavefront runs more than four:
//   4 / 8 parts, owner o: o takes query block o alone; the others, in
//     wavefront order, take row blocks {3}, {2}, {1,0}; (8 parts without an
//     owner: {3}, {2}, {1}, {0});
//   2 parts: part 0 -> w0 {2}+q0, w1 {3}, w2 {0}+q2, w3 {1};
//            part 1 -> w0 {3}, w1 {1}+q1, w2 {2,0}, w3 q3.
template <typename TIn>
struct GramTilesOp {
  const typename RowStage<TIn>::T* sK;
  const float4 (&qa)[8];
  int li, lg;
  f4v (&acc)[5];
  template <unsigned KM, int QB>
  __device__ __forceinline__ void run() const {
    gram_tiles<TIn, KM, QB>(sK, qa, li, lg, acc);
  }
};
struct GramStoreOp {
  f4v (&acc)[5];
  const float *sG, *sB, *sIK;
  float iq_scale;
  float* sL;
  int li, lg;
  template <unsigned KM, int QB>
  __device__ __forceinline__ void run() const {
    gram_store<KM, QB>(acc, sG, sB, sIK, iq_scale, sL, li, lg);
  }
};
struct AtStoreOp {
  const f4v (&acc)[5];
  const float *sL, *sT;
  float* ws;
  int li, lg, lane;
  template <unsigned KM, int QB>
  __device__ __forceinline__ void run() const {
    at_store<KM, QB>(acc, sL, sT, ws, li, lg, lane);
  }
};

template <int PARTS, typename F>
__device__ __forceinline__ void gram_dispatch(int part, int wave, const F& f) {
  if constexpr (PARTS == 1) {
    switch (wave) {
      case 0: f.template run<8u, 0>(); break;
      case 1: f.template run<4u, 1>(); break;
      case 2: f.template run<2u, 2>(); break;
      default: f.template run<1u, 3>(); break;
    }
  } else if constexpr (PARTS == 2) {
    switch (part * 4 + wave) {
      case 0: f.template run<4u, 0>(); break;
      case 1: f.template run<8u, -1>(); break;
      case 2: f.template run<1u, 2>(); break;
      case 3: f.template run<2u, -1>(); break;
      case 4: f.template run<8u, -1>(); break;
      case 5: f.template run<2u, 1>(); break;
      case 6: f.template run<5u, -1>(); break;
      default: f.template run<0u, 3>(); break;
    }
  } else {
    if (part < 4 && wave == part) {
      switch (wave) {
        case 0: f.template run<0u, 0>(); break;
        case 1: f.template run<0u, 1>(); break;
        case 2: f.template run<0u, 2>(); break;
        default: f.template run<0u, 3>(); break;
      }
    } else {
      const int rank = part < 4 ? wave - (wave > part ? 1 : 0) : wave;  // among the non-owners
      if (part < 4) {
        switch (rank) {
          case 0: f.template run<8u, -1>(); break;
          case 1: f.template run<4u, -1>(); break;
          default: f.template run<3u, -1>(); break;
        }
      } else {
        switch (rank) {
          case 0: f.template run<8u, -1>(); break;
          case 1: f.template run<4u, -1>(); break;
          case 2: f.template run<2u, -1>(); break;
          default: f.template run<1u, -1>(); break;
        }
      }
    }
  }
}

// fp16 inputs, one workgroup per (chunk, head): 4 workgroups per CU (34 KB of
// LDS each), so at most 128 VGPRs (with V staged in LDS as well, 50 KB and
// three per CU measured 0.921 vs 0.907 ms for config 2); the split forms run
// at most one workgroup per CU and keep a 168-VGPR budget.  fp32 inputs stage
// 51 KB and are compiled for one workgroup per CU.
//
// PARTS workgroups per (chunk, head) (blockIdx.z = part), for launches with
// too few (chunk, head) pairs to fill the chip: every part loads K and the
// value columns it needs, forms L's Gram tiles and T (the serial part), then
// computes and stores only its share of the record: K' column tiles
// 4*part..4*part+3 (PARTS 2, one per wavefront), 2*part and 2*part+1
// (PARTS 4: wavefronts 0-1 form row blocks {0,3} of the two tiles, 2-3
// blocks {1,2}) or tile `part` (PARTS 8: wavefront w forms row block w),
// and the A T blocks of the wavefronts w with w % PARTS == part.
// Each value is computed by the same operation sequence whatever PARTS is, so
// the record is bit-identical.
template <typename TIn, int PARTS>
__global__ __launch_bounds__(256, sizeof(TIn) == 2 ? 5 : 1) void chunk_intra_kernel(ChunkParams p) {
  typedef RawOf<TIn> R;
  typedef RowStage<TIn> RS;
  __shared__ __align__(16) typename RS::T sK[64 * RS::kLd];  // K rows, raw
  __shared__ __align__(16) float sL[10 * 256];  // L blocks; diagonal blocks become T's
  __shared__ __align__(16) float sT[3 * 256];   // T_21, T_31, T_32
  __shared__ __align__(16) float sG[64];   // gcum
  __shared__ __align__(16) float sB[64];   // beta
  __shared__ __align__(16) float sKS[64];  // Ks = e^{gL - gcum} ik
  __shared__ __align__(16) float sIK[64];  // inverse K norms (1 without L2 normalisation)

  int gchunk = blockIdx.x;
  const int h = blockIdx.y;
  int seq, t0, len;
  if (p.nsel > 0) {  // local chunk id -> table entry (chunk prefix sums held in SGPRs)
    int i = 0;
    while (i + 1 < p.nsel && (int)blockIdx.x >= p.sel_chunk0[i + 1]) ++i;
    const int c = blockIdx.x - p.sel_chunk0[i];
    seq = p.sel_seq[i];
    t0 = p.sel_t0[i] + c * kC;
    len = min(kC, p.sel_len[i] - c * kC);
    gchunk = p.sel_co[i] + c;
  } else {
    locate_chunk(p, gchunk, seq, t0, len);
  }
  if (seq < 0) return;
  const int part = PARTS > 1 ? (int)blockIdx.z : 0;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int li = lane & 15;
  const int lg = lane >> 4;
  const bool own_block = (wave % PARTS) == part;  // this wave's A block (and raw Q rows)
  const TIn* q = static_cast<const TIn*>(p.q);
  const TIn* k = static_cast<const TIn*>(p.k);
  float* ws = p.ws + ((size_t)gchunk * p.H + h) * kWsStride;

  // ---- every global load first: g/beta (wave 0), Q row block `wave` as MFMA
  // A-operand registers, 8 K row segments per thread (padding rows read row 0
  // and are zeroed when staged).  V is not needed here: the scan reads it.
  float gv = 0.0f, bv = 0.0f;
  if (wave == 0) {
    const int tt = lane < len ? lane : 0;
    gv = p.g[(size_t)h * p.N + t0 + tt];
    bv = p.beta[(size_t)h * p.N + t0 + tt];
    if (lane >= len) gv = bv = 0.0f;
  }
  // Only the wavefronts that form K Q^T tiles (their own A block) need their
  // Q rows; the others read row 0 (one cached row) so no load sits under a
  // branch.  A split launch's part needs the value columns of its own U
  // tiles only: 128 / PARTS of them.
  float4 qa[8];
  {
    const int row = 16 * wave + li;
    const int rr = (own_block && row < len) ? row : 0;
#pragma unroll
    for (int u = 0; u < 8; ++u) qa[u] = R::ld4(q, ((size_t)h * p.N + t0 + rr) * kD + 16 * u + 4 * lg);
  }
  float4 kr[8];
  const int c4 = (tid & 31) * 4;
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int r = (tid >> 5) + 8 * it;
    kr[it] = R::ld4(k, ((size_t)h * p.N + t0 + (r < len ? r : 0)) * kD + c4);
  }
  // K' column tiles ct = 2M + t of this wavefront (keys 32M + 2c + t)
  constexpr int kTilesPerWave = PARTS == 1 ? 2 : 1;
  auto kp_tile = [&](int jj) {
    return PARTS == 1 ? 2 * wave + jj : PARTS == 2 ? 4 * part + wave : PARTS == 4 ? 2 * part + (wave & 1) : part;
  };
  // gcum (running sum in token order, deltanet_chunk.cpp:137-142): lane t adds
  // g_0 .. g_t left to right (adding +0 past t), so every lane's sum is
  // rounded exactly as the reference's running sum
  // (g_j taken by v_readlane: with __shfl the 64 reads became a serial chain
  // of LDS permutes)
  if (wave == 0) {
    float run = 0.0f;
    const int gbits = __float_as_int(gv);
#pragma unroll
    for (int j = 0; j < 64; ++j) {
      const float gj = __int_as_float(__builtin_amdgcn_readlane(gbits, j));
      run = run + (j <= lane ? gj : 0.0f);
    }
    sG[lane] = run;
    sB[lane] = bv;
  }
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int r = (tid >> 5) + 8 * it;
    float4 kx = kr[it];
    if (r >= len) kx = make_float4(0.f, 0.f, 0.f, 0.f);
    RS::put4(sK, r, c4, kx);
  }
  __syncthreads();

  // ---- inverse L2 norms (eps inside the sqrt, deltanet_chunk.cpp:27-39):
  // K rows from LDS, 4 threads per row; Q rows from this lane's registers
  float iq = 1.0f;
  if (p.l2) {
    float ssq = 0.0f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const float4 x = R::cvt4(qa[u]);
      ssq = ssq + x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
    }
    ssq = ssq + spk::lane_xor16(ssq);
    ssq = ssq + spk::lane_xor32(ssq);
    iq = 1.0f / sqrtf(ssq + 1e-6f);
    const int r = tid >> 2, part = tid & 3;
    float sk = 0.0f;
#pragma unroll
    for (int c = 0; c < 32; c += 4) {
      const float4 x = RS::get4(sK, r, 32 * part + c);
      sk = sk + x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
    }
    sk = sk + spk::lane_xor1(sk);
    sk = sk + spk::lane_xor2(sk);
    if (part == 0) sIK[r] = 1.0f / sqrtf(sk + 1e-6f);
  } else if (tid < 64) {
    sIK[tid] = 1.0f;
  }

  // ---- Gram tiles (raw dot products; decays and scales in the epilogue)
  f4v acc[5];
  gram_dispatch<PARTS>(part, wave, GramTilesOp<TIn>{sK, qa, li, lg, acc});
  __syncthreads();

  // ---- epilogue: L into LDS, A into the workspace; per-token scales
  const float iq_scale = iq * p.q_scale;  // lane li of any group: row 16*wave + li
  gram_dispatch<PARTS>(part, wave, GramStoreOp{acc, sG, sB, sIK, iq_scale, sL, li, lg});
  const float gL = sG[63];
  if (lg == 0 && own_block) ws[kWsQs + 16 * wave + li] = iq_scale * expf(sG[16 * wave + li]);  // the scan re-reads Q raw
  if (tid < 64) {
    sKS[tid] = expf(gL - sG[tid]) * sIK[tid];
    if (part == 0) {
      ws[kWsC1 + tid] = sB[tid];
      ws[kWsC2 + tid] = sB[tid] * expf(sG[tid]) * sIK[tid];
    }
  }
  if (tid == 0 && part == 0) ws[kWsMisc] = expf(gL);
  __syncthreads();

  // ---- diagonal blocks of T by forward substitution, lane j < 16 of wave w
  // solving column j of block w; written over L's block once it is read
  if (li == lane) {
    float* Lb = sL + blk(wave, wave);
    const int j = lane;
    float tc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float s = 0.0f;
#pragma unroll
      for (int m = 0; m < i; ++m) s = __builtin_fmaf(Lb[i * 16 + m], tc[m], s);
      tc[i] = (i == j) ? 1.0f : (i < j ? 0.0f : -s);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) Lb[i * 16 + j] = tc[i];
  }
  __syncthreads();

  // ---- off-diagonal blocks by distance d = I - J: T_IJ = -T_II sum_M L_IM T_MJ.
  // With contraction index k = 4*lg + s, the product's C fragment is already
  // the B operand of the second product: no LDS round trip.
  for (int d = 1; d < 4; ++d) {
    if (wave < 4 - d) {
      const int J = wave;
      const int I = J + d;
      f4v x = {0.f, 0.f, 0.f, 0.f};
      for (int M = J; M < I; ++M) {
        const float4 a4 = *reinterpret_cast<const float4*>(&sL[blk(I, M) + li * 16 + 4 * lg]);
        const float* tmj = tblk(sL, sT, M, J);
#pragma unroll
        for (int s = 0; s < 4; ++s) x = mfma4(elem(a4, s), tmj[(4 * lg + s) * 16 + li], x);
      }
      const float4 a4 = *reinterpret_cast<const float4*>(&sL[blk(I, I) + li * 16 + 4 * lg]);
      f4v y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) y = mfma4(elem(a4, s), x[s], y);
      // over L_I0 (J == 0: this wavefront read it last, above) or into sT
      float* tij = (J == 0) ? sL + blk(I, 0) : sT + tslot(I, J);
#pragma unroll
      for (int r = 0; r < 4; ++r) tij[(4 * lg + r) * 16 + li] = -y[r];
    }
    __syncthreads();
  }

  // ---- A T for this wavefront's A block (the owner of query block `wave`)
  gram_dispatch<PARTS>(part, wave, AtStoreOp{acc, sL, sT, ws, li, lg, lane});

  // ---- K' = T^T diag(Ks) K, by 16-column key tiles ct = 2M + t (keys
  // 32M + 2c + t, c = 0..15: the pair of adjacent keys a lane of the scan's
  // stage D holds) and row blocks u = 0..3 (two tiles per wavefront without a
  // split).  MFMA A operand T^T (T's block (J, u) read by column, J >= u),
  // B operand Ks * K with the per-token factor applied as it is read; lane
  // (li, lg) ends up holding K'[16u+4lg+r][32M+2li+t].
#pragma unroll
  for (int jj = 0; jj < kTilesPerWave; ++jj) {
    const int ct = kp_tile(jj);
    const int M = ct >> 1, t = ct & 1;
    // row blocks u of this wave: all; {0,3} or {1,2} (4 parts: by wave / 2);
    // block `wave` (8 parts: 4, 3, 2, 1 block products)
    const bool odd_rows = (wave >> 1) != 0;
    const unsigned umask = PARTS == 8 ? (1u << wave) : PARTS == 4 ? (odd_rows ? 0x6u : 0x9u) : 0xFu;
    const int jmin = PARTS == 8 ? wave : PARTS == 4 ? (odd_rows ? 1 : 0) : 0;
    const int n = 32 * M + 2 * li + t;
    f4v ak[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) ak[u] = f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      if (J < jmin) continue;
      const int tk = 16 * J + 4 * lg;
      const float4 ks = *reinterpret_cast<const float4*>(&sKS[tk]);
      float kb[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) kb[e] = RS::get1(sK, tk + e, n) * elem(ks, e);
#pragma unroll
      for (int u = 0; u <= J; ++u) {
        if (!((umask >> u) & 1u)) continue;
        const float* tb = tblk(sL, sT, J, u);
#pragma unroll
        for (int e = 0; e < 4; ++e) ak[u] = mfma4(tb[(4 * lg + e) * 16 + li], kb[e], ak[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (!((umask >> u) & 1u)) continue;
      ws_store(ws + kWsKp + (((M * 4 + u) * 2 + t) * 64 + lane) * 4, ak[u][0], ak[u][1], ak[u][2], ak[u][3]);
    }
    __builtin_amdgcn_sched_barrier(0);  // one column tile's operands live at a time
  }
}

// Sequence with rank `slot` by decreasing length (ties: lower index first).
__device__ __forceinline__ int lpt_sequence(const ChunkParams& p, int slot) {
  if (p.cu == nullptr || p.S > 64) return slot;
  for (int s = 0; s < p.S; ++s) {
    int t;
    const int Ls = seq_span(p, s, t);
    int rank = 0;
    for (int s2 = 0; s2 < p.S; ++s2) {
      const int L2 = seq_span(p, s2, t);
      rank += (L2 > Ls) || (L2 == Ls && s2 < s);
    }
    if (rank == slot) return s;
  }
  return slot;
}

constexpr int kTiles = 8;   // 16-column tiles of the value dim per (sequence, head)
constexpr int kLdST = 132;  // LDS row stride of the transposed state tile (floats)
constexpr int kLdVT = 68;   // LDS row stride of the transposed R tile (floats)

// Operands of one chunk for stage A (prefetched a chunk ahead) and for stages
// B-D (loaded at the start of the chunk's own step, in flight during stage A).
template <typename TIn>
struct ScanEarly {
  typename RawOf<TIn>::R8 k[4];  // raw K rows: token 16M+li, key dims 32j+8lg..+7
  typename RawOf<TIn>::R8 q[4];  // raw Q rows, same map
};
template <typename TIn>
struct ScanLate {
  VTile<TIn> v;  // V: token 16M+li, columns n0+4lg..+3
  float c1;      // beta of token 16M+li
  float c2;      // beta e^gcum ik of the same token
  float qs;      // Qs of the same token
  float4 a[4];   // A T rows: token 16M+li, tokens 16u+4lg..+3
  float gle;     // e^{gL}
  float4 kq[4][2];  // K'[16u+4lg..+3][32M+2li+t] at [u][t]
};

// Sequential chunk scan over one 128x16 state tile: one workgroup of 4
// wavefronts per (sequence, head, 16-column tile), so a 16-head batch of 8
// sequences gives 1024 workgroups and three run on each CU (independent
// barriers: one workgroup's waits are the others' issue slots).  Wavefront M:
//   A  rows of token block M: K_M S and Q_M S
//   B  R = beta V - (beta e^g ik) (K S)  -> LDS
//   C  o = qs (Q S) + (A T) R -> core
//   D  S rows 32M..32M+31 <- e^{gL} S + K'^T R
// 100-112 MFMA per wavefront per chunk (stage C: 4 (M+1)).
// MINB workgroups per CU.  fp16 inputs, large launches: three (168 VGPRs;
// the instance spills 16 bytes per lane): more resident wavefronts measured faster than two
// workgroups holding both operand sets double-buffered.  fp32 inputs hold
// twice the Q and K operand registers: at 168 VGPRs they spilled 236 bytes
// per lane inside the chunk loop (6.5-9 us per chunk step against 3.1 for
// fp16), so they run two workgroups per CU without spilling, as do small
// fp16 launches.
// ZERO_INIT (no initial state): S is zero entering each sequence's first
// chunk, so that chunk's K S and Q S are exactly zero and stage A is skipped.
template <typename TIn, bool ZERO_INIT, int MINB>
__global__ __launch_bounds__(256, MINB) void chunk_state_kernel(ChunkParams p) {
  typedef RawOf<TIn> R;
  // S tile and R stored transposed ([column][contraction index]) so one
  // ds_read_b128 feeds four consecutive MFMA steps; strides 132 and 68 keep
  // the 8-lane groups of a b128 access on distinct banks.
  __shared__ __align__(16) float sST[16 * kLdST];
  __shared__ __align__(16) float sVT[16 * kLdVT];  // R = beta V - (beta e^g ik) K S

  // Workgroup -> (tile, head, sequence).  Groups (sequence, head) are dealt
  // longest sequence first so the longest chunk scans start earliest, and the
  // eight tiles of a group get workgroup ids congruent mod 8 -- the same XCD
  // (ids are dealt to the 8 XCDs round-robin) -- so they share one L2 for W,
  // A and the Q and K rows.
  const int b = blockIdx.x;
  const int groups = (p.nsel > 0 ? p.nsel : p.S) * p.H;
  int gi, tile;
  if ((groups & 7) == 0) {
    gi = (b >> 6) * 8 + (b & 7);
    tile = (b >> 3) & 7;
  } else {
    gi = b >> 3;
    tile = b & 7;
  }
  const int h = gi % p.H;
  const int slot = gi / p.H;
  const int seq = p.nsel > 0 ? p.sel_seq[slot] : lpt_sequence(p, slot);
  const int n0 = tile * 16;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Wavefront w of a workgroup runs on SIMD w, and the roles' MFMA counts
  // differ (stage C: 4 (M+1)); rotating the role by the workgroup id spreads
  // the heavy roles of the workgroups sharing a CU over its four SIMDs
  // (config 2: 0.760 -> 0.726 ms per call, bit-identical).
  const int M = __builtin_amdgcn_readfirstlane(((tid >> 6) + b) & 3);  // wave-uniform (SGPR)
  const int li = lane & 15;
  const int lg = lane >> 4;

  int t_begin = 0, L = p.N, co = 0;
  if (p.nsel > 0) {
    t_begin = p.sel_t0[slot];
    L = p.sel_len[slot];
    co = p.sel_co[slot];
  } else if (p.cu) {
    L = seq_span(p, seq, t_begin);
    for (int s = 0; s < seq; ++s) {
      int ts;
      co += (seq_span(p, s, ts) + kC - 1) / kC;
    }
    if (co + (L + kC - 1) / kC > p.chunks) L = 0;  // records past the workspace: empty
  }
  const int nchunks = (L + kC - 1) / kC;

  const float* init = p.init ? p.init + ((size_t)seq * p.H + h) * kD * kD : nullptr;
  for (int i = tid; i < 128 * 16; i += 256) {
    const int r = i >> 4;
    const int c = i & 15;
    sST[c * kLdST + r] = init ? init[r * kD + n0 + c] : 0.0f;
  }

  // Every load is unconditional (the intra kernel's padding Q rows are row 0
  // of the chunk, zeroed here through qs; the last chunk is prefetched again
  // rather than guarded), so the compiler's vmcnt bookkeeping stays exact.
  // Each record load instruction reads one contiguous fragment.
  auto record = [&](int c) { return p.ws + ((size_t)(co + c) * p.H + h) * kWsStride; };
  // raw K and Q rows 16M+li from the input (padding rows read the chunk's
  // row 0, as the intra kernel's Q operand does; their K S rows meet beta = 0
  // in stage B and their output rows are dropped)
  const size_t in_off = ((size_t)h * p.N + t_begin) * kD;
  const TIn* qin = static_cast<const TIn*>(p.q) + in_off + 8 * lg;
  const TIn* kin = static_cast<const TIn*>(p.k) + in_off + 8 * lg;
  auto load_early = [&](ScanEarly<TIn>& e, int c) {
    const int row = 16 * M + li;
    const size_t ro = (size_t)(c * kC + (row < L - c * kC ? row : 0)) * kD;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      e.k[j] = R::ld8(kin + ro + 32 * j);
      e.q[j] = R::ld8(qin + ro + 32 * j);
    }
  };
  // Stage B-D operands, in the order the stages use them (a wave's loads
  // complete in issue order): V through a buffer resource of the chunk's len
  // rows (padding rows read 0) and the per-token factors, then A T, then K'.
  const TIn* vin = static_cast<const TIn*>(p.v) + in_off;
  auto load_late = [&](ScanLate<TIn>& l, int c) {
    const float* ws = record(c);
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<TIn*>(vin + (size_t)c * kC * kD), 0, min(kC, L - c * kC) * kD * (int)sizeof(TIn), kBufDword3);
    l.v.load(vr, ((16 * M + li) * kD + n0 + 4 * lg) * (int)sizeof(TIn));
    l.c1 = ws[kWsC1 + 16 * M + li];
    l.c2 = ws[kWsC2 + 16 * M + li];
    l.qs = ws[kWsQs + 16 * M + li];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      l.a[u] = *reinterpret_cast<const float4*>(ws + kWsA + ((M * 4 + u) * 64 + lane) * 4);
    l.gle = ws[kWsMisc];
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int t = 0; t < 2; ++t)
        l.kq[u][t] = *reinterpret_cast<const float4*>(ws + kWsKp + (((M * 4 + u) * 2 + t) * 64 + lane) * 4);
  };

  // zero_s: S is zero (first chunk without an initial state)
  auto step = [&](const ScanEarly<TIn>& e, const ScanLate<TIn>& l, int c, auto zero_s) {
    const int tok0 = t_begin + c * kC;
    const int len = min(kC, L - c * kC);

    // ---- stage A: (K_M S)^T = S^T K_M^T and (Q_M S)^T share the A operand
    // (S^T, from LDS); lane (li, lg) ends up holding row 16M+li, columns
    // n0+4lg..+3 of K S and Q S.  The per-row factors are applied to the
    // products.
    f4v aw = {0.f, 0.f, 0.f, 0.f}, aq = {0.f, 0.f, 0.f, 0.f};
    if constexpr (!decltype(zero_s)::value) {
      // the S piece of step u+1 is read while step u's MFMAs run
      // step u contracts key dims 32(u/2) + 8lg + 4(u%2) + k over (lg, k)
      float4 sb_next = *reinterpret_cast<const float4*>(&sST[li * kLdST + 8 * lg]);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float4 sb = sb_next;
        if (u + 1 < 8)
          sb_next = *reinterpret_cast<const float4*>(&sST[li * kLdST + 32 * ((u + 1) >> 1) + 8 * lg + 4 * ((u + 1) & 1)]);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          aw = mfma4(elem(sb, k), R::get8(e.k[u >> 1], 4 * (u & 1) + k), aw);
          aq = mfma4(elem(sb, k), R::get8(e.q[u >> 1], 4 * (u & 1) + k), aq);
        }
      }
      // The loads issued just before this stage (same scheduling region, 25
      // of them) are spread over the MFMA stream rather than issued as one
      // burst, which would queue in the CU's vector-memory pipe behind the
      // other wavefronts' bursts: 2 and 3 loads around each 4 MFMAs.  Measured
      // on config 2 (ms per call, same box, bit-identical): 2+3 0.755, 1+2
      // 0.760, 1+3 0.763 (with 4-element K and Q fragments, 33 loads: 2+3
      // 0.875-0.878, 3+2 0.875-0.878, 2+4 0.878-0.881, 1+4 0.879-0.883, 1+3
      // 0.881-0.885, 2+2 0.895-0.898, 4+2 0.899, 4+4 0.967).
      // (masks: 0x100 LDS read, 0x020 VMEM read, 0x008 MFMA) -- the S piece
      // of step u+1 goes out before step u's 8 MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 3, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        if (i < 6) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }

    // ---- stage B: R = beta V - (beta e^g ik) (K S) for the rows of token
    // block M (v_new = T R itself is never formed: T sits in A T and K'),
    // stored transposed
#pragma unroll
    for (int e = 0; e < 4; ++e) sVT[(4 * lg + e) * kLdVT + 16 * M + li] = l.c1 * l.v.get(e) - l.c2 * aw[e];
    __syncthreads();

    // ---- stage C: o^T = (Q S)^T diag(qs) + R^T (A T)^T over the blocks
    // J <= M of A T's row block (two accumulator chains: J = 0, 1 and
    // J = 2, 3); lane (li, lg) ends up holding row 16M+li, columns
    // n0+4lg..+3 of o
    {
      float4 vb[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) vb[u] = *reinterpret_cast<const float4*>(&sVT[li * kLdVT + 16 * u + 4 * lg]);
      f4v ac = {aq[0] * l.qs, aq[1] * l.qs, aq[2] * l.qs, aq[3] * l.qs};
      f4v ad = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        if (u <= M) {
#pragma unroll
          for (int k = 0; k < 4; ++k) ac = mfma4(elem(vb[u], k), elem(l.a[u], k), ac);
        }
        if (u + 2 <= M) {
#pragma unroll
          for (int k = 0; k < 4; ++k) ad = mfma4(elem(vb[u + 2], k), elem(l.a[u + 2], k), ad);
        }
      }
      aq = ac + ad;
    }
    // rows tok0 .. tok0+len-1 of this head through a buffer resource of len
    // rows: the hardware drops the padding rows' stores (offset past
    // num_records), with no branch around the store
    {
      const __amdgpu_buffer_rsrc_t out = __builtin_amdgcn_make_buffer_rsrc(
          p.core + ((size_t)h * p.core_hs + tok0) * kD, 0, len * kD * (int)sizeof(float), kBufDword3);
      typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
      const u32x4v ov = {__float_as_uint(aq[0]), __float_as_uint(aq[1]), __float_as_uint(aq[2]), __float_as_uint(aq[3])};
      __builtin_amdgcn_raw_buffer_store_b128(ov, out, ((16 * M + li) * kD + n0 + 4 * lg) * (int)sizeof(float), 0, 0);
    }

    // ---- stage D: S^T <- e^{gL} S^T + R^T K', computed transposed so that
    // K' is the B operand in the record's fragment order: lane (li, lg) holds
    // S^T[column 4lg+r][key 32M+2li+t] in s0 (t = 0) and s1 (t = 1).
    f4v s0, s1;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float2 x = *reinterpret_cast<const float2*>(&sST[(4 * lg + r) * kLdST + 32 * M + 2 * li]);
      s0[r] = x.x * l.gle;
      s1[r] = x.y * l.gle;
    }
    float4 vs[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) vs[u] = *reinterpret_cast<const float4*>(&sVT[li * kLdVT + 16 * u + 4 * lg]);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float a = elem(vs[u], k);
        s0 = mfma4(a, elem(l.kq[u][0], k), s0);
        s1 = mfma4(a, elem(l.kq[u][1], k), s1);
      }
    }
    // every wave read sST (stage A) before the barrier above and only its own
    // keys here, so they are replaced in place
#pragma unroll
    for (int r = 0; r < 4; ++r)
      *reinterpret_cast<float2*>(&sST[(4 * lg + r) * kLdST + 32 * M + 2 * li]) = make_float2(s0[r], s1[r]);
    __syncthreads();
  };

  // Stage-A operands double-buffered (the loads of chunk c+1 are in flight
  // while chunk c computes); stage B-D operands of chunk c are loaded at the
  // start of its own step and arrive during stage A.  ZERO_INIT peels the
  // first chunk to drop its stage A at compile time (a run-time flag, or the
  // peeled loop for every launch, made the fp16 instance spill more).
  using NZ = std::integral_constant<bool, false>;
  ScanEarly<TIn> ea, eb;
  ScanLate<TIn> lt;
  if constexpr (ZERO_INIT) {
    __syncthreads();
    if (nchunks > 0) {
      load_late(lt, 0);
      load_early(eb, min(1, nchunks - 1));
      step(ea, lt, 0, std::integral_constant<bool, true>{});
    }
    for (int c = 1; c < nchunks; c += 2) {
      load_late(lt, c);
      load_early(ea, min(c + 1, nchunks - 1));
      step(eb, lt, c, NZ{});
      if (c + 1 >= nchunks) break;
      load_late(lt, c + 1);
      load_early(eb, min(c + 2, nchunks - 1));
      step(ea, lt, c + 1, NZ{});
    }
  } else {
    if (nchunks > 0) load_early(ea, 0);
    __syncthreads();
    for (int c = 0; c < nchunks; c += 2) {
      load_late(lt, c);
      load_early(eb, min(c + 1, nchunks - 1));
      step(ea, lt, c, NZ{});
      if (c + 1 >= nchunks) break;
      load_late(lt, c + 1);
      load_early(ea, min(c + 2, nchunks - 1));
      step(eb, lt, c + 1, NZ{});
    }
  }

  float* outs = p.state + ((size_t)seq * p.H + h) * kD * kD;
  for (int i = tid; i < 128 * 16; i += 256) {
    const int r = i >> 4;
    const int c = i & 15;
    outs[r * kD + n0 + c] = sST[c * kLdST + r];
  }
}

__global__ void prefill_collect_kernel(const uint16_t* __restrict__ qkv, const float* __restrict__ gb,
                                       float* qo, float* ko, float* vo, float* go, float* bo, int H,
                                       int T, int tok, int dk, int dv) {
  const int h = blockIdx.x;
  const int lid = threadIdx.x;
  if (lid < dk) {
    qo[((size_t)h * T + tok) * dk + lid] = spk::h2f(qkv[h * dk + lid]);
    ko[((size_t)h * T + tok) * dk + lid] = spk::h2f(qkv[H * dk + h * dk + lid]);
  }
  if (lid < dv) vo[((size_t)h * T + tok) * dv + lid] = spk::h2f(qkv[2 * H * dk + h * dv + lid]);
  if (lid == 0) {
    go[(size_t)h * T + tok] = gb[h];
    bo[(size_t)h * T + tok] = gb[H + h];
  }
}

__global__ void last_to_fp16_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst, int H,
                                    int dv, int T, int total) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= H * dv) return;
  const int h = idx / dv;
  const int d = idx - h * dv;
  dst[idx] = spk::f2h_trunc(src[((size_t)h * total + (T - 1)) * dv + d]);
}

size_t ws_bytes_for(int H, long long chunks) { return (size_t)chunks * H * kWsStride * sizeof(float); }

// ---- host side of the launches --------------------------------------------

struct SeqEntry {
  int seq, t0, len, chunks, co;
};

void fill_tables(ChunkParams& p, const SeqEntry* e, int n) {
  p.nsel = n;
  p.sel_chunk0[0] = 0;
  for (int i = 0; i < n; ++i) {
    p.sel_seq[i] = e[i].seq;
    p.sel_t0[i] = e[i].t0;
    p.sel_len[i] = e[i].len;
    p.sel_co[i] = e[i].co;
    p.sel_chunk0[i + 1] = p.sel_chunk0[i] + e[i].chunks;
  }
}

// Workgroups per (chunk, head): split while the split launch still has at
// most one workgroup per CU (256 CUs).  Past that the parts' repeated Gram
// and T work costs more than the split saves (fp16, 8 chunks x 16 heads: 4
// parts 23.9 us, 1 part 20.2 us).
int intra_parts(long long pairs) {
  if (pairs * 8 <= 256) return 8;
  if (pairs * 4 <= 256) return 4;
  if (pairs * 2 <= 256) return 2;
  return 1;
}

template <typename TIn>
void launch_intra_t(const ChunkParams& p, int chunks, int parts, hipStream_t s) {
  dim3 g((unsigned)chunks, (unsigned)p.H, (unsigned)parts);
  if (parts == 8)
    hipLaunchKernelGGL((chunk_intra_kernel<TIn, 8>), g, dim3(256), 0, s, p);
  else if (parts == 4)
    hipLaunchKernelGGL((chunk_intra_kernel<TIn, 4>), g, dim3(256), 0, s, p);
  else if (parts == 2)
    hipLaunchKernelGGL((chunk_intra_kernel<TIn, 2>), g, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((chunk_intra_kernel<TIn, 1>), g, dim3(256), 0, s, p);
}

int launch_intra(const ChunkParams& p, int chunks, bool f32, hipStream_t s) {
  const int parts = intra_parts((long long)chunks * p.H);
  if (f32)
    launch_intra_t<float>(p, chunks, parts, s);
  else
    launch_intra_t<uint16_t>(p, chunks, parts, s);
  return spk::check_launch("spk_chunk_prefill (intra)");
}

int launch_scan(const ChunkParams& p, int nseq, bool f32, hipStream_t s) {
  dim3 g((unsigned)(kTiles * p.H * nseq));
  // Three fp16 workgroups per CU (168 VGPRs, a 16-byte spill) only when the
  // launch has that many workgroups to keep resident; otherwise two per CU
  // without spilling, with the first-chunk skip when there is no initial
  // state (that instance's peeled loop spilled more at 168 VGPRs).  Measured,
  // fp16, 16 heads: one 104-token sequence 9.0 -> 8.0 us; config 2 (1024
  // workgroups) unchanged either way within noise, so it keeps the old path.
  const bool z = p.init == nullptr;
  const bool big = g.x > 2u * 256u;
  if (f32 && z)
    hipLaunchKernelGGL((chunk_state_kernel<float, true, 2>), g, dim3(256), 0, s, p);
  else if (f32)
    hipLaunchKernelGGL((chunk_state_kernel<float, false, 2>), g, dim3(256), 0, s, p);
  else if (big)
    hipLaunchKernelGGL((chunk_state_kernel<uint16_t, false, 3>), g, dim3(256), 0, s, p);
  else if (z)
    hipLaunchKernelGGL((chunk_state_kernel<uint16_t, true, 2>), g, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((chunk_state_kernel<uint16_t, false, 2>), g, dim3(256), 0, s, p);
  return spk::check_launch("spk_chunk_prefill (state)");
}

}  // namespace

extern "C" size_t spk_chunk_prefill_workspace_size(int32_t num_heads, int32_t total_tokens,
                                                   int32_t num_seqs, int32_t chunk_size) {
  if (num_heads <= 0 || total_tokens < 0 || num_seqs <= 0 || chunk_size != kC) return 0;
  const long long bound = (total_tokens + kC - 1) / kC + num_seqs;
  return ws_bytes_for(num_heads, bound);
}

extern "C" int spk_chunk_prefill(const SpkChunkArgs* a, spk_stream_t stream) {
  if (!a) return spk::fail(SPK_ERR_NULL, "spk_chunk_prefill: args is NULL");
  if (a->key_dim != kD || a->value_dim != kD || a->chunk_size != kC)
    return spk::fail(SPK_ERR_SHAPE, "spk_chunk_prefill: need key_dim == value_dim == 128 and chunk_size == 64 (got %d, %d, %d)",
                     a->key_dim, a->value_dim, a->chunk_size);
  if (a->num_heads <= 0 || a->total_tokens < 0)
    return spk::fail(SPK_ERR_SHAPE, "spk_chunk_prefill: num_heads %d total_tokens %d", a->num_heads, a->total_tokens);
  if (a->input_dtype != SPK_F32 && a->input_dtype != SPK_F16)
    return spk::fail(SPK_ERR_ARG, "spk_chunk_prefill: input_dtype %d", a->input_dtype);
  const int S = a->cu_seqlens ? a->num_seqs : 1;
  if (S <= 0) return spk::fail(SPK_ERR_SHAPE, "spk_chunk_prefill: num_seqs %d", a->num_seqs);
  if (!a->out_state || !a->workspace) return spk::fail(SPK_ERR_NULL, "spk_chunk_prefill: out_state/workspace NULL");
  if (a->total_tokens > 0 && (!a->q || !a->k || !a->v || !a->g || !a->beta || !a->out_core))
    return spk::fail(SPK_ERR_NULL, "spk_chunk_prefill: q/k/v/g/beta/out_core NULL");
  long long chunks = 0;
  if (a->cu_seqlens) {
    if (!a->cu_seqlens_host) return spk::fail(SPK_ERR_NULL, "spk_chunk_prefill: cu_seqlens_host is required with cu_seqlens");
    const int32_t* cu = a->cu_seqlens_host;
    if (cu[0] != 0 || cu[S] != a->total_tokens)
      return spk::fail(SPK_ERR_SHAPE, "spk_chunk_prefill: cu_seqlens must start at 0 and end at total_tokens");
    for (int s = 0; s < S; ++s) {
      if (cu[s + 1] < cu[s]) return spk::fail(SPK_ERR_SHAPE, "spk_chunk_prefill: cu_seqlens not monotonic at %d", s);
      chunks += (cu[s + 1] - cu[s] + kC - 1) / kC;
    }
  } else {
    chunks = (a->total_tokens + kC - 1) / kC;
  }
  const size_t need = ws_bytes_for(a->num_heads, chunks);
  if (a->workspace_bytes < need)
    return spk::fail(SPK_ERR_ARG, "spk_chunk_prefill: workspace %zu < %zu bytes", a->workspace_bytes, need);
  const size_t vec = a->input_dtype == SPK_F32 ? 16 : 8;
  if (!spk::aligned(a->q, vec) || !spk::aligned(a->k, vec) || !spk::aligned(a->v, vec) ||
      !spk::aligned(a->workspace, 16) || !spk::aligned(a->out_state, 4) || !spk::aligned(a->out_core, 4))
    return spk::fail(SPK_ERR_ALIGN, "spk_chunk_prefill: q/k/v must be %zu-byte aligned, workspace 16-byte", vec);
  const long long hs = a->core_head_stride ? a->core_head_stride : a->total_tokens;
  if (hs < a->total_tokens) return spk::fail(SPK_ERR_SHAPE, "spk_chunk_prefill: core_head_stride < total_tokens");

  ChunkParams p;
  p.H = a->num_heads;
  p.N = a->total_tokens;
  p.S = S;
  p.l2 = a->use_qk_l2norm ? 1 : 0;
  p.q_scale = a->q_scale != 0.0f ? a->q_scale : 1.0f / sqrtf((float)kD);
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.g = a->g;
  p.beta = a->beta;
  p.init = a->initial_state;
  p.core = a->out_core;
  p.core_hs = hs;
  p.state = a->out_state;
  p.cu = a->cu_seqlens;
  p.ws = static_cast<float*>(a->workspace);
  p.chunks = (int)chunks;
  p.nsel = 0;
  hipStream_t s = spk::to_hip(stream);
  const bool f32 = a->input_dtype == SPK_F32;
  if (!a->cu_seqlens || S > kSelMax) {  // one sequence, or more than the tables hold
    if (chunks > 0) {
      if (int rc = launch_intra(p, (int)chunks, f32, s)) return rc;
    }
    return launch_scan(p, S, f32, s);
  }

  // Sequences from the host copy of cu_seqlens, longest first (stable), in
  // the kernels' tables.  (Splitting off the longest sequences so that their
  // scan overlaps the others' intra work, on a second stream, measured slower
  // for config 2 -- 1.08 vs 0.94 ms: the intra workgroups fill the CUs' LDS,
  // so the early scan gets no slots until they drain.)
  SeqEntry seqs[kSelMax];
  {
    int co = 0;
    for (int i = 0; i < S; ++i) {
      const int t0 = a->cu_seqlens_host[i], len = a->cu_seqlens_host[i + 1] - t0;
      const int n = (len + kC - 1) / kC;
      seqs[i] = {i, t0, len, n, co};
      co += n;
    }
    std::stable_sort(seqs, seqs + S, [](const SeqEntry& x, const SeqEntry& y) { return x.len > y.len; });
  }
  fill_tables(p, seqs, S);
  if (chunks > 0) {
    if (int rc = launch_intra(p, p.sel_chunk0[p.nsel], f32, s)) return rc;
  }
  return launch_scan(p, p.nsel, f32, s);
}

extern "C" int spk_prefill_collect(const uint16_t* dn_qkv, const float* g_beta, float* q_out,
                                   float* k_out, float* v_out, float* g_out, float* beta_out,
                                   int32_t num_heads, int32_t seq_len, int32_t token_idx,
                                   int32_t key_dim, int32_t value_dim, spk_stream_t stream) {
  if (!dn_qkv || !g_beta || !q_out || !k_out || !v_out || !g_out || !beta_out)
    return spk::fail(SPK_ERR_NULL, "spk_prefill_collect: NULL pointer");
  if (num_heads <= 0 || seq_len <= 0 || token_idx < 0 || token_idx >= seq_len || key_dim <= 0 ||
      value_dim <= 0 || key_dim > 1024 || value_dim > 1024)
    return spk::fail(SPK_ERR_SHAPE, "spk_prefill_collect: bad shape");
  const int threads = ((key_dim > value_dim ? key_dim : value_dim) + 63) / 64 * 64;
  hipLaunchKernelGGL(prefill_collect_kernel, dim3(num_heads), dim3(threads), 0, spk::to_hip(stream), dn_qkv,
                     g_beta, q_out, k_out, v_out, g_out, beta_out, num_heads, seq_len, token_idx,
                     key_dim, value_dim);
  return spk::check_launch("spk_prefill_collect");
}

extern "C" int spk_chunk_last_to_fp16(const float* src, uint16_t* dst, int32_t num_heads,
                                      int32_t value_dim, int32_t seq_len, int32_t total_seq,
                                      spk_stream_t stream) {
  if (!src || !dst) return spk::fail(SPK_ERR_NULL, "spk_chunk_last_to_fp16: NULL pointer");
  if (num_heads <= 0 || value_dim <= 0 || seq_len <= 0 || total_seq < seq_len)
    return spk::fail(SPK_ERR_SHAPE, "spk_chunk_last_to_fp16: bad shape");
  const int n = num_heads * value_dim;
  hipLaunchKernelGGL(last_to_fp16_kernel, dim3((n + 63) / 64), dim3(64), 0, spk::to_hip(stream), src, dst,
                     num_heads, value_dim, seq_len, total_seq);
  return spk::check_launch("spk_chunk_last_to_fp16");
}
