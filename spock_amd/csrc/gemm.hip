// gemm.hip -- prompt-length projections: C[M][N] = fp16(A[M][K] . W[N][K]^T),
// optionally fp16(R + fp16(A . W^T)) (the residual add after out_proj /
// o_proj / down_proj), fp16 operands, fp32 accumulation on the matrix cores
// (v_mfma_f32_32x32x16_f16, CDNA4's double-rate fp16 form).  This is the
// prefill form of every decode matvec (matvec_tiled.comp applied to all prompt
// tokens at once); both operands are K-contiguous, which is how the artifact
// stores weights.
//
// Tiling: each wave computes 32 rows x (32·TN) columns (TN 32x32 MFMA tiles);
// a workgroup holds WM x WN x KS waves, the KS groups splitting each staged
// K step and adding their partials in order at the end.  Shapes (chosen by a
// sweep of time per shape; see spk_gemm_f16):
//   32 x 64 with KS = 4 and K steps of 256 when 32 x 64 tiles number fewer
//     than 512 and K allows (the N <= 1024 projections of a 512-token prompt:
//     256 workgroups of 8 waves, a quarter of the K steps, so 4x the bytes in
//     flight per step of memory latency);
//   64 x 64 with KS = 4 up to 384 such tiles (N = 2048 at M = 512);
//   64 x 64 (2 x 2 waves) for wider outputs, 64 x 128 (TN = 2) only for
//   outputs large enough to fill the chip four times over.
// K in steps of BK staged through LDS, double-buffered: the next step's global
// loads are in flight while the current one is multiplied.  LDS rows are
// padded by 8 halves so the 16-byte fragment reads of 16 consecutive lanes
// (16 consecutive rows) fall in distinct banks.
#include "capi_common.hpp"
#include "numerics.hpp"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

template <int WM, int WN, int TN, int KS, int BK, bool RES>
__global__ __launch_bounds__(64 * WM * WN * KS) void gemm_nt_kernel(const uint16_t* __restrict__ A,
                                                                   const uint16_t* __restrict__ W, uint16_t* C,
                                                                   const uint16_t* R, int M, int N, int K,
                                                                   long long lda, long long ldw, long long ldc) {
  constexpr int BM = 32 * WM, BN = 32 * WN * TN, LDK = BK + 8;
  constexpr int NT = 64 * WM * WN * KS;
  constexpr int PPR = BK / 8;                     // 16-byte pieces per row per step
  constexpr int P = (BM + BN) * PPR / NT;         // pieces per thread per step
  constexpr int KW = BK / KS;                     // k values per wave per step
  static_assert((BM + BN) * PPR % NT == 0, "staging must divide evenly");
  static_assert(KW % 16 == 0, "a wave's k range is whole 32x32x16 steps");
  static_assert(KS == 1 || (KS - 1) * WM * WN * TN * 1024 * 4 <= 2 * (BM + BN) * LDK * 2,
                "the k-split partials fit in the staging buffers");
  __shared__ __align__(16) uint16_t smem[2 * (BM + BN) * LDK];
  auto As = reinterpret_cast<uint16_t(*)[BM][LDK]>(smem);
  auto Ws = reinterpret_cast<uint16_t(*)[BN][LDK]>(smem + 2 * BM * LDK);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int ks = wave / (WM * WN), wmn = wave % (WM * WN);
  const int wm = wmn / WN, wn = wmn % WN;

  // global -> register staging; rows past M / N read row 0 and stage zeros
  const uint16_t* src[P];
  bool ok[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const int idx = tid + NT * p, row = idx / PPR, col = (idx % PPR) * 8;
    if (row < BM) {
      ok[p] = m0 + row < M;
      src[p] = A + (long long)(ok[p] ? m0 + row : 0) * lda + col;
    } else {
      ok[p] = n0 + row - BM < N;
      src[p] = W + (long long)(ok[p] ? n0 + row - BM : 0) * ldw + col;
    }
  }
  uint4 reg[P];
  auto load = [&](int k0) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const uint4 v = *reinterpret_cast<const uint4*>(src[p] + k0);
      reg[p] = ok[p] ? v : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int idx = tid + NT * p, row = idx / PPR, col = (idx % PPR) * 8;
      if (row < BM)
        *reinterpret_cast<uint4*>(&As[buf][row][col]) = reg[p];
      else
        *reinterpret_cast<uint4*>(&Ws[buf][row - BM][col]) = reg[p];
    }
  };

  floatx16 acc[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;

  const int fr = lane & 31;        // fragment row (A) / column (B)
  const int fk = (lane >> 5) * 8;  // fragment k offset within a step of 16
  load(0);
  store(0);
  __syncthreads();
  const int nk = K / BK;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * BK);
#pragma unroll
    for (int i = 0; i < KW / 16; ++i) {
      const int kk = ks * KW + 16 * i;
      const half8_t a = *reinterpret_cast<const half8_t*>(&As[buf][wm * 32 + fr][kk + fk]);
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const half8_t b = *reinterpret_cast<const half8_t*>(&Ws[buf][(wn * TN + t) * 32 + fr][kk + fk]);
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[t], 0, 0, 0);
      }
    }
    if (kt + 1 < nk) {
      store(buf ^ 1);
      __syncthreads();
    }
  }
  if constexpr (KS > 1) {
    // k-split partials: waves ks > 0 park theirs in the staging buffers, the
    // ks = 0 waves add them in ks order
    float* red = reinterpret_cast<float*>(smem);
    __syncthreads();
    if (ks > 0) {
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) red[(((ks - 1) * (WM * WN) + wmn) * TN + t) * 1024 + r * 64 + lane] = acc[t][r];
    }
    __syncthreads();
    if (ks > 0) return;
    for (int j = 1; j < KS; ++j)
#pragma unroll
      for (int t = 0; t < TN; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] += red[(((j - 1) * (WM * WN) + wmn) * TN + t) * 1024 + r * 64 + lane];
  }
  // D[i][j]: lane j = lane%32, row i = 8*(r/4) + 4*(lane/32) + r%4
#pragma unroll
  for (int t = 0; t < TN; ++t) {
    const int col = n0 + (wn * TN + t) * 32 + fr;
    if (col >= N) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + wm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (row >= M) continue;
      uint16_t o = spk::f2h(acc[t][r]);
      if (RES) o = spk::f2h(spk::h2f(R[(long long)row * ldc + col]) + spk::h2f(o));
      C[(long long)row * ldc + col] = o;
    }
  }
}

template <int WM, int WN, int TN, int KS, int BK>
void launch_gemm(const uint16_t* A, const uint16_t* W, uint16_t* C, const uint16_t* R, int M, int N, int K,
                 long long lda, long long ldw, long long ldc, hipStream_t s) {
  constexpr int BM = 32 * WM, BN = 32 * WN * TN;
  const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  const dim3 block(64 * WM * WN * KS);
  if (R)
    hipLaunchKernelGGL((gemm_nt_kernel<WM, WN, TN, KS, BK, true>), grid, block, 0, s, A, W, C, R, M, N, K, lda, ldw,
                       ldc);
  else
    hipLaunchKernelGGL((gemm_nt_kernel<WM, WN, TN, KS, BK, false>), grid, block, 0, s, A, W, C, R, M, N, K, lda,
                       ldw, ldc);
}

}  // namespace

extern "C" int spk_gemm_f16(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw, uint16_t* C, int64_t ldc,
                            const uint16_t* residual, int32_t M, int32_t N, int32_t K, spk_stream_t stream) {
  if (!A || !W || !C) return spk::fail(SPK_ERR_NULL, "spk_gemm_f16: NULL pointer");
  if (M <= 0 || N <= 0 || K <= 0 || K % 32 != 0)
    return spk::fail(SPK_ERR_SHAPE, "spk_gemm_f16: M %d N %d K %d (K must be a positive multiple of 32)", M, N, K);
  if (lda < K || ldw < K || ldc < N || lda % 8 || ldw % 8)
    return spk::fail(SPK_ERR_SHAPE, "spk_gemm_f16: leading dimensions (lda %lld ldw %lld ldc %lld)", (long long)lda,
                     (long long)ldw, (long long)ldc);
  if (!spk::aligned(A, 16) || !spk::aligned(W, 16))
    return spk::fail(SPK_ERR_ALIGN, "spk_gemm_f16: A and W must be 16-byte aligned");
  if (residual == A || residual == W || C == A || C == W)
    return spk::fail(SPK_ERR_ARG, "spk_gemm_f16: the output or residual aliases an operand");
  hipStream_t s = spk::to_hip(stream);
  // tile shape by measured time on MI355X at the config-4 prompt shapes
  // (M = 512, K = 1024/2048/3584): k-split 32 x 64 tiles while they number
  // fewer than 512, k-split 64 x 64 up to 384 tiles, plain 64 x 64 above and
  // 64 x 128 only when its tiles alone fill four waves of workgroups per CU
  const long long t32x64 = (long long)((N + 63) / 64) * ((M + 31) / 32);
  const long long t64x64 = (long long)((N + 63) / 64) * ((M + 63) / 64);
  const long long t64x128 = (long long)((N + 127) / 128) * ((M + 63) / 64);
  if (K % 256 == 0 && t32x64 < 512)
    launch_gemm<1, 2, 1, 4, 256>(A, W, C, residual, M, N, K, lda, ldw, ldc, s);
  else if (K % 256 == 0 && t64x64 < 384)
    launch_gemm<2, 2, 1, 4, 256>(A, W, C, residual, M, N, K, lda, ldw, ldc, s);
  else if (K % 64 == 0 && t64x128 >= 1024)
    launch_gemm<2, 2, 2, 1, 64>(A, W, C, residual, M, N, K, lda, ldw, ldc, s);
  else if (K % 64 == 0)
    launch_gemm<2, 2, 1, 1, 64>(A, W, C, residual, M, N, K, lda, ldw, ldc, s);
  else
    launch_gemm<2, 2, 1, 1, 32>(A, W, C, residual, M, N, K, lda, ldw, ldc, s);
  return spk::check_launch("spk_gemm_f16");
}
