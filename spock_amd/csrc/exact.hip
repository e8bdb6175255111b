// exact.hip -- prompt-wide kernels in the operation order of the CPU
// restatement, so a prompt processed on the GPU gives the same bits as the
// oracle (and therefore the same greedy tokens downstream):
//
//   spk_matvec_f16_rows: the decode matvec (64 contiguous spans fma-chained
//     from 0, then the s[l] += s[l+stride] tree, one fp16 rounding; the order
//     of lm_head_tiled.comp) applied to every row of a prompt.  Each output is
//     bit-identical to spk_matvec_f16 on that row.
//   spk_chunk_prefill_ordered: run_deltanet_chunk_rule's loop nests
//     (deltanet_chunk.cpp:53-284) with every reduction in the reference's
//     sequential order and no contraction, exp = the library's deterministic
//     exp (numerics.hpp).
//
// These are the parity forms of spk_gemm_f16 (matrix cores) and
// spk_chunk_prefill (MFMA WY/UT kernels); they spend VALU cycles to keep the
// reference's order and are used where bit-exact prompt results are required.
#include "capi_common.hpp"
#include "numerics.hpp"

namespace {

// ---------------------------------------------------------------------------
// spk_matvec_f16_rows
// ---------------------------------------------------------------------------
constexpr int kTile = 64;  // 64 W rows x 64 prompt rows per 256-thread block

struct RowsArgs {
  const uint16_t* W;
  const uint16_t* X;
  long long ldx;
  uint16_t* Y;
  long long ldy;
  const uint16_t* R;
  int rows, out_dim, in_dim, span;
};

struct Acc16 {
  float v[16];
};

__device__ __forceinline__ void unpack8h(const uint4& u, float* f) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = spk::h2f((uint16_t)(w[i] & 0xffffu));
    f[2 * i + 1] = spk::h2f((uint16_t)(w[i] >> 16));
  }
}

// Leaf i (in bit-reversed order: span l = bitrev6(i)) of the 64-span tree for
// the thread's 4 x 4 outputs.  The tree s[l] += s[l+32], ..., s[l] += s[l+1]
// pairs spans whose indices differ in bit 5 first; visiting spans in
// bit-reversed order makes every pair of neighbouring visits a pair of that
// tree, so a recursive split of the visit order reproduces it exactly.
__device__ __forceinline__ Acc16 leaf(const RowsArgs& a, int i, float (*Ws)[65], float (*Xs)[65], int r0, int t0) {
  const int l = (int)(__builtin_bitreverse32((uint32_t)i) >> 26);
  const int tid = threadIdx.x;
  const int S = a.span;
  __syncthreads();
  for (int idx = tid; idx < kTile * S; idx += 256) {
    const int row = idx / S, j = idx - (idx / S) * S;
    const int wr = r0 + row, xr = t0 + row;
    Ws[row][j] = wr < a.out_dim ? spk::h2f(a.W[(long long)wr * a.in_dim + l * S + j]) : 0.0f;
    Xs[row][j] = xr < a.rows ? spk::h2f(a.X[(long long)xr * a.ldx + l * S + j]) : 0.0f;
  }
  __syncthreads();
  const int tx = tid & 15, ty = tid >> 4;
  Acc16 acc;
#pragma unroll
  for (int k = 0; k < 16; ++k) acc.v[k] = 0.0f;
  for (int j = 0; j < S; ++j) {
    float w[4], x[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      w[q] = Ws[tx * 4 + q][j];
      x[q] = Xs[ty * 4 + q][j];
    }
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int q = 0; q < 4; ++q) acc.v[p * 4 + q] = __builtin_fmaf(w[p], x[q], acc.v[p * 4 + q]);
  }
  return acc;
}

template <int LEVEL>
__device__ __forceinline__ Acc16 node(const RowsArgs& a, int j, float (*Ws)[65], float (*Xs)[65], int r0, int t0) {
  if constexpr (LEVEL == 0) {
    return leaf(a, j, Ws, Xs, r0, t0);
  } else {
    Acc16 lo = node<LEVEL - 1>(a, 2 * j, Ws, Xs, r0, t0);
    const Acc16 hi = node<LEVEL - 1>(a, 2 * j + 1, Ws, Xs, r0, t0);
#pragma unroll
    for (int k = 0; k < 16; ++k) lo.v[k] = lo.v[k] + hi.v[k];
    return lo;
  }
}

__global__ __launch_bounds__(256) void matvec_rows_kernel(RowsArgs a) {
  __shared__ float Ws[kTile][65];
  __shared__ float Xs[kTile][65];
  const int r0 = blockIdx.x * kTile, t0 = blockIdx.y * kTile;
  const Acc16 s = node<6>(a, 0, Ws, Xs, r0, t0);
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
#pragma unroll
  for (int p = 0; p < 4; ++p)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = r0 + tx * 4 + p, t = t0 + ty * 4 + q;
      if (r < a.out_dim && t < a.rows) {
        uint16_t o = spk::f2h(s.v[p * 4 + q]);
        if (a.R) o = spk::f2h(spk::h2f(a.R[(long long)t * a.ldy + r]) + spk::h2f(o));
        a.Y[(long long)t * a.ldy + r] = o;
      }
    }
}

// Matrix-core form (in_dim % 512 == 0).  v_mfma_f32_16x16x1_4b_f32 adds one
// product per output per instruction, C + a*b with a single rounding; with
// fp16-valued operands the product is exact, so a chain of these is the
// sequential fma chain bit for bit.  Its 4 blocks run spans l, l+16, l+32 and
// l+48 together (lane = block * 16 + row/column): blocks 0+2 and 1+3 are the
// tree's stride-32 pairs and their sum its stride-16 pair, all register-wise
// adds (every block keeps row 4*(lane/16) + k, column lane%16 in register
// 4*block + k).  The 16 values of l are visited in 4-bit bit-reversed order
// and merged like a binary counter, which reproduces strides 8..1.  One wave
// computes TR x TT tiles of 16 W rows x 16 prompt rows; operands are read
// straight from global memory (L1/L2), 8 halves per lane per load, one chunk
// of 8 steps ahead.
typedef float v16f __attribute__((ext_vector_type(16)));

template <int S, int TR, int TT>
__global__ __launch_bounds__(256) void matvec_rows_mfma_kernel(RowsArgs a, int n_tt, int n_tiles) {
  const int lane = threadIdx.x & 63;
  const int tile = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tile >= n_tiles) return;  // whole wave; the kernel has no barrier
  const int r0 = (tile / n_tt) * 16 * TR, t0 = (tile % n_tt) * 16 * TT;
  const int blk = lane >> 4, li = lane & 15;
  constexpr int C = S / 8;  // 16-byte chunks per span
  const uint16_t* wrow[TR];
  const uint16_t* xrow[TT];
#pragma unroll
  for (int i = 0; i < TR; ++i) wrow[i] = a.W + (size_t)min(r0 + 16 * i + li, a.out_dim - 1) * a.in_dim;
#pragma unroll
  for (int j = 0; j < TT; ++j) xrow[j] = a.X + (size_t)min(t0 + 16 * j + li, a.rows - 1) * a.ldx;
  auto span_of = [&](int v) { return (int)(__builtin_bitreverse32((uint32_t)v) >> 28) + 16 * blk; };
  uint4 nw[TR], nx[TT];
  auto issue = [&](int v, int c) {
    const int off = span_of(v) * S + 8 * c;
#pragma unroll
    for (int i = 0; i < TR; ++i) nw[i] = *reinterpret_cast<const uint4*>(wrow[i] + off);
#pragma unroll
    for (int j = 0; j < TT; ++j) nx[j] = *reinterpret_cast<const uint4*>(xrow[j] + off);
  };
  float stack[4][TR * TT * 4];
  float cur[TR * TT * 4];
  issue(0, 0);
#pragma unroll 1
  for (int v = 0; v < 16; ++v) {
    v16f acc[TR][TT];
#pragma unroll
    for (int i = 0; i < TR; ++i)
#pragma unroll
      for (int j = 0; j < TT; ++j) acc[i][j] = v16f{};
    for (int c = 0; c < C; ++c) {
      float wf[TR][8], xf[TT][8];
#pragma unroll
      for (int i = 0; i < TR; ++i) unpack8h(nw[i], wf[i]);
#pragma unroll
      for (int j = 0; j < TT; ++j) unpack8h(nx[j], xf[j]);
      if (c + 1 < C)
        issue(v, c + 1);
      else if (v + 1 < 16)
        issue(v + 1, 0);
#pragma unroll
      for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int i = 0; i < TR; ++i)
#pragma unroll
          for (int j = 0; j < TT; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x1f32(wf[i][e], xf[j][e], acc[i][j], 0, 0, 0);
    }
    // (P_l + P_{l+32}) + (P_{l+16} + P_{l+48})
#pragma unroll
    for (int i = 0; i < TR; ++i)
#pragma unroll
      for (int j = 0; j < TT; ++j)
#pragma unroll
        for (int k = 0; k < 4; ++k)
          cur[(i * TT + j) * 4 + k] = (acc[i][j][k] + acc[i][j][8 + k]) + (acc[i][j][4 + k] + acc[i][j][12 + k]);
    // binary-counter merge: visits v and v ^ (1 << lev) pair at level lev
    bool carry = true;
#pragma unroll
    for (int lev = 0; lev < 4; ++lev) {
      if (carry) {
        if ((v >> lev) & 1) {
#pragma unroll
          for (int q = 0; q < TR * TT * 4; ++q) cur[q] = stack[lev][q] + cur[q];
        } else {
#pragma unroll
          for (int q = 0; q < TR * TT * 4; ++q) stack[lev][q] = cur[q];
          carry = false;
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < TR; ++i)
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      const int t = t0 + 16 * j + li;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = r0 + 16 * i + 4 * blk + k;
        if (r < a.out_dim && t < a.rows) {
          uint16_t o = spk::f2h(cur[(i * TT + j) * 4 + k]);
          if (a.R) o = spk::f2h(spk::h2f(a.R[(long long)t * a.ldy + r]) + spk::h2f(o));
          a.Y[(long long)t * a.ldy + r] = o;
        }
      }
    }
}

// Few output tiles (small projections, short prompts): the same leaves,
// order and tree as matvec_rows_mfma_kernel for one 16 x 16 tile, its 16
// leaves split over the workgroup's 4 waves.  Wave g takes visits v = 4g ..
// 4g+3, a whole subtree of the binary-counter merge, and merges them exactly
// as the one-wave kernel would; the four subtree sums are then combined as
// the counter's last two levels do, (g0 + g1) + (g2 + g3).  A quarter of the
// sequential chunk loads per wave.
template <int S>
__global__ __launch_bounds__(256) void matvec_rows_split_kernel(RowsArgs a, int n_tt) {
  __shared__ float part[4][4][64];  // [wave][k][lane]
  const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
  const int tile = blockIdx.x;
  const int r0 = (tile / n_tt) * 16, t0 = (tile % n_tt) * 16;
  const int blk = lane >> 4, li = lane & 15;
  constexpr int C = S / 8;  // 16-byte chunks per span
  const uint16_t* wrow = a.W + (size_t)min(r0 + li, a.out_dim - 1) * a.in_dim;
  const uint16_t* xrow = a.X + (size_t)min(t0 + li, a.rows - 1) * a.ldx;
  auto span_of = [&](int v) { return (int)(__builtin_bitreverse32((uint32_t)v) >> 28) + 16 * blk; };
  uint4 nw, nx;
  auto issue = [&](int v, int c) {
    const int off = span_of(v) * S + 8 * c;
    nw = *reinterpret_cast<const uint4*>(wrow + off);
    nx = *reinterpret_cast<const uint4*>(xrow + off);
  };
  float stack[2][4];
  float cur[4];
  issue(4 * g, 0);
#pragma unroll 1
  for (int m = 0; m < 4; ++m) {
    const int v = 4 * g + m;
    v16f acc = v16f{};
    for (int c = 0; c < C; ++c) {
      float wf[8], xf[8];
      unpack8h(nw, wf);
      unpack8h(nx, xf);
      if (c + 1 < C)
        issue(v, c + 1);
      else if (m + 1 < 4)
        issue(v + 1, 0);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x1f32(wf[e], xf[e], acc, 0, 0, 0);
    }
    // (P_l + P_{l+32}) + (P_{l+16} + P_{l+48})
#pragma unroll
    for (int k = 0; k < 4; ++k) cur[k] = (acc[k] + acc[8 + k]) + (acc[4 + k] + acc[12 + k]);
    // binary-counter merge inside the subtree (levels 0 and 1; m = v mod 4)
    bool carry = true;
#pragma unroll
    for (int lev = 0; lev < 2; ++lev) {
      if (carry) {
        if ((m >> lev) & 1) {
#pragma unroll
          for (int q = 0; q < 4; ++q) cur[q] = stack[lev][q] + cur[q];
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) stack[lev][q] = cur[q];
          carry = false;
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) part[g][k][lane] = cur[k];
  __syncthreads();
  if (g != 0) return;
  const int t = t0 + li;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float s = (part[0][k][lane] + part[1][k][lane]) + (part[2][k][lane] + part[3][k][lane]);
    const int r = r0 + 4 * blk + k;
    if (r < a.out_dim && t < a.rows) {
      uint16_t o = spk::f2h(s);
      if (a.R) o = spk::f2h(spk::h2f(a.R[(long long)t * a.ldy + r]) + spk::h2f(o));
      a.Y[(long long)t * a.ldy + r] = o;
    }
  }
}

// in_dim 2048 / 3584 (S = 32 / 56): the same leaves, order and tree as
// matvec_rows_mfma_kernel, with each leaf's operands staged through LDS by
// coalesced loads (a span is 64 / 112 contiguous bytes; the lanes of a load
// walk a span's 16-byte pieces, then the next block's span, then the next
// row) instead of per-lane loads from 64 separate rows, which saturate the
// vector-memory address pipe.  Workgroup tile: 16*WR W rows x 16*WT prompt
// rows, one 16 x 16 MFMA tile per wave; the next leaf's pieces are loaded into
// registers while the current leaf is multiplied.  LDS rows hold the 4 spans
// of a leaf (4*S halves) plus 8 halves of padding, so the 16-byte fragment
// reads of 16 consecutive rows fall in distinct banks.
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

template <int S, int WR, int WT>
__global__ __launch_bounds__(64 * WR * WT) void matvec_rows_lds_kernel(RowsArgs a) {
  constexpr int NT = 64 * WR * WT;
  constexpr int LD = 4 * S + 8;
  constexpr int PPS = S / 8;                              // 16-byte pieces per span
  constexpr int PPR = 4 * PPS;                            // pieces per staged row
  constexpr int NPW = 16 * WR * PPR, NP = NPW + 16 * WT * PPR;
  constexpr int P = (NP + NT - 1) / NT;                   // pieces per thread
  __shared__ __align__(16) uint16_t lds[(16 * WR + 16 * WT) * LD];  // W rows, then X rows
  auto Ws = reinterpret_cast<uint16_t(*)[LD]>(lds);
  auto Xs = reinterpret_cast<uint16_t(*)[LD]>(lds + 16 * WR * LD);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int blk = lane >> 4, li = lane & 15;
  const int wr = wave % WR, wt = wave / WR;
  const int r0 = blockIdx.x * 16 * WR, t0 = blockIdx.y * 16 * WT;
  // piece p of this thread: staged row, block, piece within the span
  const uint16_t* src[P];
  int dst[P];
#pragma unroll
  for (int k = 0; k < P; ++k) {
    const int pc = min(tid + NT * k, NP - 1);  // the tail re-stages the last piece
    const bool isw = pc < NPW;
    const int pr = isw ? pc : pc - NPW;
    const int row = pr / PPR, b = (pr % PPR) / PPS, q = pr % PPS;
    src[k] = isw ? a.W + (size_t)min(r0 + row, a.out_dim - 1) * a.in_dim + b * 16 * S + 8 * q
                 : a.X + (size_t)min(t0 + row, a.rows - 1) * a.ldx + b * 16 * S + 8 * q;
    dst[k] = (isw ? 0 : 16 * WR * LD) + row * LD + b * S + 8 * q;
  }
  // leaf v: span l = bitrev4(v) (+16 per block)
  auto span_off = [](int v) { return (int)(__builtin_bitreverse32((uint32_t)v) >> 28) * S; };
  v4u pv[P];  // a native vector type, which the compiler keeps in registers
#pragma unroll
  for (int k = 0; k < P; ++k) pv[k] = *reinterpret_cast<const v4u*>(src[k]);
  float stack[4][4];
  float cur[4];
#pragma unroll 1
  for (int v = 0; v < 16; ++v) {
    __syncthreads();  // the previous leaf's fragment reads are done
#pragma unroll
    for (int k = 0; k < P; ++k) *reinterpret_cast<v4u*>(lds + dst[k]) = pv[k];
    __syncthreads();
    const int noff = span_off(min(v + 1, 15));
#pragma unroll
    for (int k = 0; k < P; ++k) pv[k] = *reinterpret_cast<const v4u*>(src[k] + noff);
    v16f acc = v16f{};
#pragma unroll
    for (int c = 0; c < PPS; ++c) {
      float wf[8], xf[8];
      unpack8h(*reinterpret_cast<const uint4*>(&Ws[16 * wr + li][blk * S + 8 * c]), wf);
      unpack8h(*reinterpret_cast<const uint4*>(&Xs[16 * wt + li][blk * S + 8 * c]), xf);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x1f32(wf[e], xf[e], acc, 0, 0, 0);
    }
    // (P_l + P_{l+32}) + (P_{l+16} + P_{l+48})
#pragma unroll
    for (int k = 0; k < 4; ++k) cur[k] = (acc[k] + acc[8 + k]) + (acc[4 + k] + acc[12 + k]);
    // binary-counter merge: visits v and v ^ (1 << lev) pair at level lev
    bool carry = true;
#pragma unroll
    for (int lev = 0; lev < 4; ++lev) {
      if (carry) {
        if ((v >> lev) & 1) {
#pragma unroll
          for (int q = 0; q < 4; ++q) cur[q] = stack[lev][q] + cur[q];
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) stack[lev][q] = cur[q];
          carry = false;
        }
      }
    }
  }
  const int t = t0 + 16 * wt + li;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = r0 + 16 * wr + 4 * blk + k;
    if (r < a.out_dim && t < a.rows) {
      uint16_t o = spk::f2h(cur[k]);
      if (a.R) o = spk::f2h(spk::h2f(a.R[(long long)t * a.ldy + r]) + spk::h2f(o));
      a.Y[(long long)t * a.ldy + r] = o;
    }
  }
}

// in_dim == 1024 (S = 16, a span is 32 B): the same leaves and tree, with
// operands staged through LDS four leaves at a time.  Leaves v, v+4, v+8,
// v+12 (v < 4) are l = L..L+3 with L = bitrev4(v), i.e. spans L..L+3 (+16b
// per block): four whole 128-byte lines of every row, loaded coalesced.  The
// groups arrive in the order L = 0, 8, 4, 12 and are merged as the tree
// pairs them: s[m] + s[m+8] once L = 8 is in, s[4+m] + s[12+m] once L = 12 is
// in, then strides 4, 2, 1.  Workgroup tile: 64 W rows x 32 prompt rows, one
// 32 x 16 (2 x 1 MFMA tiles) per wave; three workgroups per CU.
constexpr int kGrpLd = 264;  // halves per LDS row: 4 blocks x 64 + 8 pad (row starts 4 banks apart)
constexpr int kGrpRows = 64, kGrpToks = 32;

__global__ __launch_bounds__(256, 3) void matvec_rows_grp_kernel(RowsArgs a) {
  __shared__ __align__(16) uint16_t Ws[kGrpRows][kGrpLd];
  __shared__ __align__(16) uint16_t Xs[kGrpToks][kGrpLd];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int blk = lane >> 4, li = lane & 15;
  const int r0 = blockIdx.x * kGrpRows, t0 = blockIdx.y * kGrpToks;
  const int wr = 32 * (wave & 1), wt = 16 * (wave >> 1);  // wave tile inside the workgroup tile
  float H[4][8], G[4][8];
#pragma unroll 1
  for (int g = 0; g < 4; ++g) {
    const int L = (int)(__builtin_bitreverse32((uint32_t)g) >> 28);
    __syncthreads();  // the previous group's operand reads are done
    // rows x 4 blocks x 8 pieces of 16 B: 8 W + 4 X pieces per thread
    uint4 pw[8], px[4];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int pc = tid + 256 * k;
      const int row = pc >> 5, b = (pc >> 3) & 3, q = pc & 7;
      pw[k] = *reinterpret_cast<const uint4*>(a.W + (size_t)min(r0 + row, a.out_dim - 1) * 1024 +
                                              (16 * b + L) * 16 + 8 * q);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int pc = tid + 256 * k;
      const int row = pc >> 5, b = (pc >> 3) & 3, q = pc & 7;
      px[k] = *reinterpret_cast<const uint4*>(a.X + (size_t)min(t0 + row, a.rows - 1) * a.ldx +
                                              (16 * b + L) * 16 + 8 * q);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int pc = tid + 256 * k;
      *reinterpret_cast<uint4*>(&Ws[pc >> 5][64 * ((pc >> 3) & 3) + 8 * (pc & 7)]) = pw[k];
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int pc = tid + 256 * k;
      *reinterpret_cast<uint4*>(&Xs[pc >> 5][64 * ((pc >> 3) & 3) + 8 * (pc & 7)]) = px[k];
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < 4; ++m) {  // leaf l = L + m: span L + m (+16 per block)
      v16f acc[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) acc[i] = v16f{};
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        float wf[2][8], xf[8];
#pragma unroll
        for (int i = 0; i < 2; ++i)
          unpack8h(*reinterpret_cast<const uint4*>(&Ws[wr + 16 * i + li][64 * blk + 16 * m + 8 * c]), wf[i]);
        unpack8h(*reinterpret_cast<const uint4*>(&Xs[wt + li][64 * blk + 16 * m + 8 * c]), xf);
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
          for (int i = 0; i < 2; ++i)
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x1f32(wf[i][e], xf[e], acc[i], 0, 0, 0);
      }
      float R[8];  // (P_l + P_{l+32}) + (P_{l+16} + P_{l+48})
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k)
          R[i * 4 + k] = (acc[i][k] + acc[i][8 + k]) + (acc[i][4 + k] + acc[i][12 + k]);
      if (g == 0) {
#pragma unroll
        for (int q = 0; q < 8; ++q) H[m][q] = R[q];  // s[m]
      } else if (g == 1) {
#pragma unroll
        for (int q = 0; q < 8; ++q) H[m][q] = H[m][q] + R[q];  // s[m] + s[m+8]
      } else if (g == 2) {
#pragma unroll
        for (int q = 0; q < 8; ++q) G[m][q] = R[q];  // s[4+m]
      } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) G[m][q] = G[m][q] + R[q];  // s[4+m] + s[12+m]
      }
    }
  }
  float out[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float b0 = H[0][q] + G[0][q], b1 = H[1][q] + G[1][q];  // stride 4
    const float b2 = H[2][q] + G[2][q], b3 = H[3][q] + G[3][q];
    out[q] = (b0 + b2) + (b1 + b3);  // strides 2, 1
  }
  const int t = t0 + wt + li;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = r0 + wr + 16 * i + 4 * blk + k;
      if (r < a.out_dim && t < a.rows) {
        uint16_t o = spk::f2h(out[i * 4 + k]);
        if (a.R) o = spk::f2h(spk::h2f(a.R[(long long)t * a.ldy + r]) + spk::h2f(o));
        a.Y[(long long)t * a.ldy + r] = o;
      }
    }
}

// ---------------------------------------------------------------------------
// spk_chunk_prefill_ordered
// ---------------------------------------------------------------------------
constexpr int kC = 64, kD = 128, kThreads = 512;

struct OrdArgs {
  int H, T, total;  // total = T rounded up to 64
  int l2, f16;
  float q_scale;
  const void* q;
  const void* k;
  const void* v;
  const float* g;
  const float* beta;
  const float* init;
  float* core;
  long long core_head_stride;
  float* state;
  float* ws;  // per head: qs, ks, vs [total][128]; solved, kcd, vnew, inter [64][128]
};

__device__ __forceinline__ float ld_in(const void* p, bool f16, long long i) {
  return f16 ? spk::h2f(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

// Per chunk, the state-independent results of the chunk body: solved (U)
// [64][128], kcd (W) [64][128], local (decayed QK^T) [64][64], eg [64],
// wlast [64].
constexpr int kChunkWs = 2 * kC * kD + kC * kC + 2 * kC;

// Per head: the padded, normalised and q-scaled qs, ks [total][128], then
// kChunkWs floats per chunk.
__host__ __device__ __forceinline__ size_t head_ws_floats(int total) {
  return (size_t)2 * total * kD + (size_t)(total / kC) * kChunkWs;
}

__device__ __forceinline__ float* head_ws(const OrdArgs& a, int h) {
  return a.ws + (size_t)h * head_ws_floats(a.total);
}

__device__ __forceinline__ float* chunk_ws(const OrdArgs& a, int h, int ci) {
  return head_ws(a, h) + (size_t)2 * a.total * kD + (size_t)ci * kChunkWs;
}

// Chunk body, part 1 (run_deltanet_chunk_rule's loops that do not read the
// state): one workgroup per (chunk, head), every chunk at once.  The chunk's
// q, k, v rows are loaded once into LDS, padded with zeros past T, optionally
// L2-normalised (deltanet_chunk.cpp:27-39, 78-85: sequential sum of squares,
// then x * (1 / sqrt(sum + 1e-6))) and q-scaled (:87-88); q and k are also
// written out for the state scan.  Each phase is split over its independent
// outputs; every reduction runs in the reference's sequential order.
constexpr int kRowLd = kD + 4;  // LDS row pitch: 16-byte reads, rows 4 banks apart

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

__global__ __launch_bounds__(kThreads) void ordered_chunk_prep_kernel(OrdArgs a) {
  __shared__ __align__(16) float qs[kC][kRowLd];
  __shared__ __align__(16) float ks[kC][kRowLd];
  __shared__ __align__(16) float vs[kC][kRowLd];
  __shared__ float gcum[kC], bc[kC], eg[kC], inv_q[kC], inv_k[kC];
  __shared__ float decay[kC][kC + 1], attn[kC][kC + 1];
  const int ci = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  float* w = head_ws(a, h);
  const int base = ci * kC;
  float* cw = chunk_ws(a, h, ci);
  float* solved = cw;
  float* kcd = cw + kC * kD;
  float* local = cw + 2 * kC * kD;
  float* egw = local + kC * kC;
  float* wlast = egw + kC;
  // q, k, v rows of the chunk: 4 elements per piece, every load issued before
  // any use (rows past T read row T-1 and stage zeros)
  {
    constexpr int kPieces = kC * kD / 4 / kThreads;  // 4
    float4 lq[kPieces], lk[kPieces], lv[kPieces];
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      const int pc = tid + kThreads * j, t = pc / (kD / 4), d = (pc % (kD / 4)) * 4;
      const long long src = ((long long)h * a.T + min(base + t, a.T - 1)) * kD + d;
      if (a.f16) {
        const uint2 uq = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.q) + src);
        const uint2 uk = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.k) + src);
        const uint2 uv = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(a.v) + src);
        lq[j] = make_float4(spk::h2f(uq.x & 0xffffu), spk::h2f(uq.x >> 16), spk::h2f(uq.y & 0xffffu), spk::h2f(uq.y >> 16));
        lk[j] = make_float4(spk::h2f(uk.x & 0xffffu), spk::h2f(uk.x >> 16), spk::h2f(uk.y & 0xffffu), spk::h2f(uk.y >> 16));
        lv[j] = make_float4(spk::h2f(uv.x & 0xffffu), spk::h2f(uv.x >> 16), spk::h2f(uv.y & 0xffffu), spk::h2f(uv.y >> 16));
      } else {
        lq[j] = ld4(static_cast<const float*>(a.q) + src);
        lk[j] = ld4(static_cast<const float*>(a.k) + src);
        lv[j] = ld4(static_cast<const float*>(a.v) + src);
      }
    }
#pragma unroll
    for (int j = 0; j < kPieces; ++j) {
      const int pc = tid + kThreads * j, t = pc / (kD / 4), d = (pc % (kD / 4)) * 4;
      const bool live = base + t < a.T;
      const float4 q = lq[j], k = lk[j], v = lv[j];
      *reinterpret_cast<float4*>(&qs[t][d]) =
          make_float4(live ? q.x : 0.0f, live ? q.y : 0.0f, live ? q.z : 0.0f, live ? q.w : 0.0f);
      *reinterpret_cast<float4*>(&ks[t][d]) =
          make_float4(live ? k.x : 0.0f, live ? k.y : 0.0f, live ? k.z : 0.0f, live ? k.w : 0.0f);
      *reinterpret_cast<float4*>(&vs[t][d]) =
          make_float4(live ? v.x : 0.0f, live ? v.y : 0.0f, live ? v.z : 0.0f, live ? v.w : 0.0f);
    }
  }
  if (tid < kC) {
    // :137-151: lane t of wave 0 adds g_0 .. g_t left to right (adding +0
    // past t), so its sum is rounded exactly as the reference's running sum;
    // g_j by readlane (no serial chain through LDS on one thread)
    const int tok = base + tid;
    const float gv = tok < a.T ? a.g[(size_t)h * a.T + tok] : 0.0f;
    bc[tid] = tok < a.T ? a.beta[(size_t)h * a.T + tok] : 0.0f;
    float running = 0.0f;
    const int gbits = __float_as_int(gv);
#pragma unroll
    for (int j = 0; j < kC; ++j) {
      const float gj = __int_as_float(__builtin_amdgcn_readlane(gbits, j));
      running = running + (j <= tid ? gj : 0.0f);
    }
    gcum[tid] = running;
  }
  __syncthreads();
  if (a.l2) {
    if (tid >= 64 && tid < 64 + 2 * kC) {  // waves 1, 2
      const int t = tid & (kC - 1);
      const float* x = tid < 128 ? qs[t] : ks[t];
      float sq = 0.0f;
      for (int d = 0; d < kD; d += 4) {
        const float4 v = ld4(x + d);
        sq = sq + v.x * v.x;
        sq = sq + v.y * v.y;
        sq = sq + v.z * v.z;
        sq = sq + v.w * v.w;
      }
      (tid < 128 ? inv_q : inv_k)[t] = 1.0f / __builtin_sqrtf(sq + 1e-6f);
    }
  }
  __syncthreads();
  for (int i = tid; i < kC * kD; i += kThreads) {
    const int t = i / kD, d = i % kD;
    float q = qs[t][d], k = ks[t][d];
    if (a.l2) {
      q = q * inv_q[t];
      k = k * inv_k[t];
    }
    q = q * a.q_scale;
    qs[t][d] = q;
    ks[t][d] = k;
    w[(size_t)(base + t) * kD + d] = q;
    w[(size_t)a.total * kD + (size_t)(base + t) * kD + d] = k;
  }
  if (tid < kC) {
    eg[tid] = spk::expf_det(gcum[tid]);
    egw[tid] = eg[tid];
    wlast[tid] = spk::expf_det(gcum[kC - 1] - gcum[tid]);
  }
  for (int i = tid; i < kC * kC; i += kThreads) {  // :153-159
    const int r = i / kC, c = i % kC;
    decay[r][c] = c <= r ? spk::expf_det(gcum[r] - gcum[c]) : 0.0f;
  }
  __syncthreads();
  // :161-170 (attn, strictly lower): lane = column c, wave-uniform rows, four
  // rows per pass; each d = 0..127 sum in order, 4 terms per 16-byte read.
  for (int r0 = 4 * wave; r0 < kC; r0 += 4 * (kThreads / 64)) {
    const int c = lane;
    float da[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int d = 0; d < kD; d += 4) {
      const float4 kc4 = ld4(&ks[c][d]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 kr = ld4(&ks[r0 + j][d]);
        const float br = bc[r0 + j];
        da[j] = da[j] + (kr.x * br) * kc4.x;
        da[j] = da[j] + (kr.y * br) * kc4.y;
        da[j] = da[j] + (kr.z * br) * kc4.z;
        da[j] = da[j] + (kr.w * br) * kc4.w;
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) attn[r0 + j][c] = c < r0 + j ? -da[j] * decay[r0 + j][c] : 0.0f;
  }
  __syncthreads();
  if (wave == 0) {
    // :171-181 forward substitution.  Row r is updated from its original
    // values (the reference's old_row) and rows < r already updated; lane c
    // keeps its column of the updated matrix in registers, so the original
    // rows stay in LDS untouched until the end and no barrier is needed
    // between rows.
    const int c = lane;
    float col[kC];
#pragma unroll
    for (int in = 0; in < kC; ++in) col[in] = attn[in][c];
#pragma unroll
    for (int r = 1; r < kC; ++r) {
      if (c < r) {
        float sum = col[r];
#pragma unroll
        for (int in = 0; in < r; ++in) sum = sum + attn[r][in] * col[in];
        col[r] = sum;
      }
    }
    // (one wave: its LDS reads above complete before the writes below)
#pragma unroll
    for (int in = 0; in < kC; ++in) attn[in][c] = in == c ? col[in] + 1.0f : col[in];  // :182-184 +I
  } else if (wave != 4) {
    // :204-213 (local, lower), meanwhile on the six waves that do not share
    // SIMD 0 with the solve (waves are dealt to SIMDs round-robin)
    const int lw = wave < 4 ? wave - 1 : wave - 2;  // 0..5
    for (int r0 = 4 * lw; r0 < kC; r0 += 4 * 6) {
      const int c = lane;
      float dl[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int d = 0; d < kD; d += 4) {
        const float4 kc4 = ld4(&ks[c][d]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float4 qr = ld4(&qs[r0 + j][d]);
          dl[j] = dl[j] + qr.x * kc4.x;
          dl[j] = dl[j] + qr.y * kc4.y;
          dl[j] = dl[j] + qr.z * kc4.z;
          dl[j] = dl[j] + qr.w * kc4.w;
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) local[(r0 + j) * kC + c] = c <= r0 + j ? dl[j] * decay[r0 + j][c] : 0.0f;
    }
  }
  __syncthreads();
  // :186-202.  The factors v*beta and (k*beta)*e^g depend on (c, d) only:
  // computed once, rounded as in the reference, in place of v and k.
  for (int i = tid; i < kC * kD; i += kThreads) {
    const int c = i / kD, d = i % kD;
    const float bcol = bc[c];
    vs[c][d] = vs[c][d] * bcol;
    ks[c][d] = (ks[c][d] * bcol) * eg[c];
  }
  __syncthreads();
  // thread = 4 rows x 4 consecutive d; c = 0..63 in order, zero coefficients
  // skipped per row as in the reference
  {
    const int r0 = (tid / (kD / 4)) * 4, d = (tid % (kD / 4)) * 4;
    float sv[4][4], sk[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) sv[j][e] = sk[j][e] = 0.0f;
    for (int c = 0; c < kC; ++c) {
      const float4 v4 = ld4(&vs[c][d]), k4 = ld4(&ks[c][d]);
      const float vv[4] = {v4.x, v4.y, v4.z, v4.w}, kk[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float coeff = attn[r0 + j][c];
        if (coeff == 0.0f) continue;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sv[j][e] = sv[j][e] + coeff * vv[e];
          sk[j][e] = sk[j][e] + coeff * kk[e];
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      *reinterpret_cast<float4*>(solved + (r0 + j) * kD + d) = make_float4(sv[j][0], sv[j][1], sv[j][2], sv[j][3]);
      *reinterpret_cast<float4*>(kcd + (r0 + j) * kD + d) = make_float4(sk[j][0], sk[j][1], sk[j][2], sk[j][3]);
    }
  }
}

// Chunk body, part 2 (the loops that read or write the state, :215-268): the
// state's value columns are independent, so one workgroup per (head, slice of
// kSlice columns) scans the chunks in order with its 128 x kSlice block of the
// state in LDS.  Each chunk's state-independent operands (kcd, q, k, local,
// the slice of solved, eg, wlast) are staged in LDS; the next chunk's are
// loaded into registers while the current one is computed.
constexpr int kSlice = 8;   // value columns per workgroup: 16 heads x 16 slices fill the chip
constexpr int kScanThreads = 512;
constexpr int kScanLd = kD + 4;

__global__ __launch_bounds__(kScanThreads) void ordered_chunk_scan_kernel(OrdArgs a) {
  __shared__ __align__(16) float Kc[kC][kScanLd];  // kcd (W)
  __shared__ __align__(16) float Qc[kC][kScanLd];  // scaled q
  __shared__ __align__(16) float Kk[kC][kScanLd];  // k
  __shared__ __align__(16) float Lc[kC][kC + 1];   // local
  __shared__ __align__(16) float Sol[kC][kSlice];  // solved (U), this slice
  __shared__ float Eg[kC], Wl[kC];
  __shared__ __align__(16) float Ss[kD][kSlice];   // the state slice
  __shared__ __align__(16) float vn[kC][kSlice];   // v_new, this slice
  const int h = blockIdx.x / (kD / kSlice);
  const int v0 = (blockIdx.x % (kD / kSlice)) * kSlice;
  const int tid = threadIdx.x;
  float* w = head_ws(a, h);
  const float* qs = w;
  const float* ks = w + (size_t)a.total * kD;
  float* S = a.state + (size_t)h * kD * kD;
  for (int i = tid; i < kD * kSlice; i += kScanThreads) {
    const int kd = i / kSlice, j = i % kSlice;
    Ss[kd][j] = a.init ? a.init[(size_t)h * kD * kD + kd * kD + v0 + j] : 0.0f;
  }
  // prefetch registers: kcd, q, k (4 float4 each), local (2 float4), the
  // solved slice (float2), eg or wlast (one float for tid < 128)
  float4 pk[4], pq[4], pkk[4], pl[2];
  float ps;
  float pe = 0.0f;
  auto prefetch = [&](int ci) {
    const float* cw = chunk_ws(a, h, ci);
    const float* kcd = cw + kC * kD;
    const float* loc = cw + 2 * kC * kD;
    const float* qc = qs + (size_t)ci * kC * kD;
    const float* kc = ks + (size_t)ci * kC * kD;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pc = tid + kScanThreads * j;  // float4 index in a [64][128] block
      pk[j] = ld4(kcd + 4 * pc);
      pq[j] = ld4(qc + 4 * pc);
      pkk[j] = ld4(kc + 4 * pc);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) pl[j] = ld4(loc + 4 * (tid + kScanThreads * j));
    ps = cw[(tid >> 3) * kD + v0 + (tid & 7)];
    if (tid < 2 * kC) pe = cw[2 * kC * kD + kC * kC + tid];  // eg[0..63], then wlast[0..63]
  };
  const int nchunks = a.total / kC;
  prefetch(0);
  for (int ci = 0; ci < nchunks; ++ci) {
    const int base = ci * kC;
    __syncthreads();  // the previous chunk's reads of the staged operands are done
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pc = tid + kScanThreads * j, r = pc / (kD / 4), d = (pc % (kD / 4)) * 4;
      *reinterpret_cast<float4*>(&Kc[r][d]) = pk[j];
      *reinterpret_cast<float4*>(&Qc[r][d]) = pq[j];
      *reinterpret_cast<float4*>(&Kk[r][d]) = pkk[j];
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int pc = tid + kScanThreads * j, r = pc / (kC / 4), c = (pc % (kC / 4)) * 4;
      Lc[r][c] = pl[j].x;
      Lc[r][c + 1] = pl[j].y;
      Lc[r][c + 2] = pl[j].z;
      Lc[r][c + 3] = pl[j].w;
    }
    Sol[tid >> 3][tid & 7] = ps;
    if (tid < kC)
      Eg[tid] = pe;
    else if (tid < 2 * kC)
      Wl[tid - kC] = pe;
    __syncthreads();
    if (ci + 1 < nchunks) prefetch(ci + 1);
    // A (:215-233): thread = row r, column cp of the slice
    const int r = tid >> 3, cp = tid & 7;
    float inter = 0.0f;
    {
      const float egr = Eg[r];
      float carry = 0.0f;
      for (int k4 = 0; k4 < kD; k4 += 4) {
        const float4 kw = ld4(&Kc[r][k4]);
        const float4 qw = ld4(&Qc[r][k4]);
        const float kk[4] = {kw.x, kw.y, kw.z, kw.w};
        const float qq[4] = {qw.x, qw.y, qw.z, qw.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float sv = Ss[k4 + e][cp];
          const float qe = qq[e] * egr;
          carry = carry + kk[e] * sv;
          inter = inter + qe * sv;
        }
      }
      vn[r][cp] = Sol[r][cp] - carry;
    }
    __syncthreads();
    // B (:235-244): core[r] = inter + sum_{c <= r} local[r][c] * vnew[c]
    {
      float s0 = inter;
      for (int c = 0; c <= r; ++c) s0 = s0 + Lc[r][c] * vn[c][cp];
      if (base + r < a.T) a.core[((size_t)h * a.core_head_stride + base + r) * kD + v0 + cp] = s0;
    }
    // C (:246-268): thread = state row kd, columns 2cq, 2cq+1 of the slice
    {
      const int kd = tid >> 2, cq = tid & 3;
      const float eglast = Eg[kC - 1];
      float upd[2] = {0.0f, 0.0f};
      for (int rr = 0; rr < kC; ++rr) {
        const float kw = Kk[rr][kd] * Wl[rr];
        const float2 v2 = *reinterpret_cast<const float2*>(&vn[rr][cq * 2]);
        upd[0] = upd[0] + kw * v2.x;
        upd[1] = upd[1] + kw * v2.y;
      }
      // Ss row kd was read by phase A (before the barrier above) and is
      // written here by this thread alone
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float ws = Ss[kd][cq * 2 + j] * eglast;
        Ss[kd][cq * 2 + j] = ws + upd[j];
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < kD * kSlice; i += kScanThreads) {
    const int k = i / kSlice, j = i % kSlice;
    S[(size_t)k * kD + v0 + j] = Ss[k][j];
  }
}

}  // namespace

extern "C" int spk_matvec_f16_rows(const uint16_t* W, const uint16_t* X, int64_t ldx, uint16_t* Y, int64_t ldy,
                                   const uint16_t* residual, int32_t rows, int32_t out_dim, int32_t in_dim,
                                   spk_stream_t stream) {
  if (!W || !X || !Y) return spk::fail(SPK_ERR_NULL, "spk_matvec_f16_rows: NULL pointer");
  if (rows <= 0 || out_dim <= 0 || in_dim <= 0 || in_dim % 64 != 0 || in_dim / 64 > 64)
    return spk::fail(SPK_ERR_SHAPE, "spk_matvec_f16_rows: rows %d out %d in %d (in a multiple of 64, <= 4096)", rows,
                     out_dim, in_dim);
  if (ldx < in_dim || ldy < out_dim) return spk::fail(SPK_ERR_SHAPE, "spk_matvec_f16_rows: leading dimensions");
  if (residual == X || Y == X) return spk::fail(SPK_ERR_ARG, "spk_matvec_f16_rows: output aliases the input");
  RowsArgs a{W, X, (long long)ldx, Y, (long long)ldy, residual, rows, out_dim, in_dim, in_dim / 64};
  hipStream_t s = spk::to_hip(stream);
  const int S = in_dim / 64;
  const bool vec_ok = spk::aligned(W, 16) && spk::aligned(X, 16) && ldx % 8 == 0;
  if (S == 16 && vec_ok && (long long)((out_dim + kGrpRows - 1) / kGrpRows) * ((rows + kGrpToks - 1) / kGrpToks) >= 256) {
    const dim3 grid((out_dim + kGrpRows - 1) / kGrpRows, (rows + kGrpToks - 1) / kGrpToks);
    hipLaunchKernelGGL(matvec_rows_grp_kernel, grid, dim3(256), 0, s, a);
    return spk::check_launch("spk_matvec_f16_rows");
  }
  if ((S == 32 || S == 56) && vec_ok && (long long)((out_dim + 31) / 32) * ((rows + 31) / 32) >= 256) {
    const dim3 grid((out_dim + 31) / 32, (rows + 31) / 32);
    if (S == 32)
      hipLaunchKernelGGL((matvec_rows_lds_kernel<32, 2, 2>), grid, dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((matvec_rows_lds_kernel<56, 2, 2>), grid, dim3(256), 0, s, a);
    return spk::check_launch("spk_matvec_f16_rows");
  }
  if ((S == 16 || S == 32 || S == 56) && vec_ok) {
    const int nt16 = (rows + 15) / 16;
    const long long tiles16 = (long long)((out_dim + 15) / 16) * nt16;
    if (tiles16 < 512) {  // one wave per tile would leave most of the chip idle
      if (S == 16)
        hipLaunchKernelGGL((matvec_rows_split_kernel<16>), dim3(tiles16), dim3(256), 0, s, a, nt16);
      else if (S == 32)
        hipLaunchKernelGGL((matvec_rows_split_kernel<32>), dim3(tiles16), dim3(256), 0, s, a, nt16);
      else
        hipLaunchKernelGGL((matvec_rows_split_kernel<56>), dim3(tiles16), dim3(256), 0, s, a, nt16);
      return spk::check_launch("spk_matvec_f16_rows");
    }
    // 2 x 2 tiles per wave unless that leaves SIMDs idle (1024 on the chip);
    // then 1 x 2, then 1 x 1 (two waves per SIMD hide more operand latency)
    const int n_rt32 = (out_dim + 31) / 32, n_rt16 = (out_dim + 15) / 16;
    const int n_tt32 = (rows + 31) / 32, n_tt16 = (rows + 15) / 16;
    int shape, n_rt, n_tt;
    if ((long long)n_rt32 * n_tt32 >= 1024) {
      shape = 0, n_rt = n_rt32, n_tt = n_tt32;
    } else if ((long long)n_rt16 * n_tt32 >= 2048) {
      shape = 1, n_rt = n_rt16, n_tt = n_tt32;
    } else {
      shape = 2, n_rt = n_rt16, n_tt = n_tt16;
    }
    const int n_tiles = n_rt * n_tt;
    const dim3 grid((n_tiles + 3) / 4);
#define SPK_MVR(s_, tr_, tt_) \
  hipLaunchKernelGGL((matvec_rows_mfma_kernel<s_, tr_, tt_>), grid, dim3(256), 0, s, a, n_tt, n_tiles)
#define SPK_MVR3(s_)        \
  if (shape == 0)           \
    SPK_MVR(s_, 2, 2);      \
  else if (shape == 1)      \
    SPK_MVR(s_, 1, 2);      \
  else                      \
    SPK_MVR(s_, 1, 1);
    if (S == 16) {
      SPK_MVR3(16)
    } else if (S == 32) {
      SPK_MVR3(32)
    } else {
      SPK_MVR3(56)
    }
#undef SPK_MVR3
#undef SPK_MVR
    return spk::check_launch("spk_matvec_f16_rows");
  }
  dim3 grid((out_dim + kTile - 1) / kTile, (rows + kTile - 1) / kTile);
  hipLaunchKernelGGL(matvec_rows_kernel, grid, dim3(256), 0, s, a);
  return spk::check_launch("spk_matvec_f16_rows");
}

extern "C" size_t spk_chunk_prefill_ordered_workspace_size(int32_t num_heads, int32_t total_tokens) {
  if (num_heads <= 0 || total_tokens <= 0) return 0;
  const size_t total = ((size_t)total_tokens + kC - 1) / kC * kC;
  return (size_t)num_heads * head_ws_floats((int)total) * sizeof(float);
}

extern "C" int spk_chunk_prefill_ordered(const SpkChunkArgs* p, spk_stream_t stream) {
  if (!p) return spk::fail(SPK_ERR_NULL, "spk_chunk_prefill_ordered: NULL args");
  if (p->num_heads <= 0 || p->total_tokens <= 0 || p->key_dim <= 0 || p->value_dim <= 0 || p->chunk_size <= 0)
    return spk::fail(SPK_ERR_SHAPE, "spk_chunk_prefill_ordered: DeltaNet chunk config fields must be non-zero");
  if (p->key_dim != kD || p->value_dim != kD || p->chunk_size != kC)
    return spk::fail(SPK_ERR_SHAPE, "spk_chunk_prefill_ordered: key_dim %d value_dim %d chunk %d (need 128/128/64)",
                     p->key_dim, p->value_dim, p->chunk_size);
  if (p->cu_seqlens || p->num_seqs > 1)
    return spk::fail(SPK_ERR_ARG, "spk_chunk_prefill_ordered: one sequence per call");
  if (!p->q || !p->k || !p->v || !p->g || !p->beta || !p->out_core || !p->out_state || !p->workspace)
    return spk::fail(SPK_ERR_NULL, "spk_chunk_prefill_ordered: NULL pointer");
  if (p->input_dtype != SPK_F32 && p->input_dtype != SPK_F16)
    return spk::fail(SPK_ERR_ARG, "spk_chunk_prefill_ordered: input_dtype %d", p->input_dtype);
  {
    const size_t vec = p->input_dtype == SPK_F16 ? 8 : 16;  // 4 elements per load
    if (!spk::aligned(p->q, vec) || !spk::aligned(p->k, vec) || !spk::aligned(p->v, vec) ||
        !spk::aligned(p->workspace, 16) || !spk::aligned(p->out_state, 4) || !spk::aligned(p->out_core, 4))
      return spk::fail(SPK_ERR_ALIGN, "spk_chunk_prefill_ordered: q/k/v must be %zu-byte aligned, workspace 16-byte",
                       vec);
  }
  if (p->workspace_bytes < spk_chunk_prefill_ordered_workspace_size(p->num_heads, p->total_tokens))
    return spk::fail(SPK_ERR_ARG, "spk_chunk_prefill_ordered: workspace %zu < %zu bytes", p->workspace_bytes,
                     spk_chunk_prefill_ordered_workspace_size(p->num_heads, p->total_tokens));
  const long long chs = p->core_head_stride ? p->core_head_stride : p->total_tokens;
  if (chs < p->total_tokens) return spk::fail(SPK_ERR_SHAPE, "spk_chunk_prefill_ordered: core_head_stride");
  if (p->initial_state == p->out_state && p->initial_state)
    return spk::fail(SPK_ERR_ARG, "spk_chunk_prefill_ordered: initial_state must not alias out_state");
  OrdArgs a;
  a.H = p->num_heads;
  a.T = p->total_tokens;
  a.total = (p->total_tokens + kC - 1) / kC * kC;
  a.l2 = p->use_qk_l2norm != 0;
  a.f16 = p->input_dtype == SPK_F16;
  a.q_scale = p->q_scale != 0.0f ? p->q_scale : 1.0f / sqrtf((float)p->key_dim);
  a.q = p->q;
  a.k = p->k;
  a.v = p->v;
  a.g = p->g;
  a.beta = p->beta;
  a.init = p->initial_state;
  a.core = p->out_core;
  a.core_head_stride = chs;
  a.state = p->out_state;
  a.ws = static_cast<float*>(p->workspace);
  hipStream_t s = spk::to_hip(stream);
  hipLaunchKernelGGL(ordered_chunk_prep_kernel, dim3(a.total / kC, a.H), dim3(kThreads), 0, s, a);
  int rc = spk::check_launch("spk_chunk_prefill_ordered (chunk prep)");
  if (rc) return rc;
  hipLaunchKernelGGL(ordered_chunk_scan_kernel, dim3(a.H * (kD / kSlice)), dim3(kScanThreads), 0, s, a);
  return spk::check_launch("spk_chunk_prefill_ordered (scan)");
}
