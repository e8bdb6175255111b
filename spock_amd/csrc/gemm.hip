// gemm.hip -- prompt-length projections: C[M][N] = fp16(A[M][K] . W[N][K]^T),
// optionally fp16(R + fp16(A . W^T)) (the residual add after out_proj /
// o_proj / down_proj), fp16 operands, fp32 accumulation on the matrix cores
// (v_mfma_f32_32x32x8_f16).  This is the prefill form of every decode matvec
// (matvec_tiled.comp applied to all prompt tokens at once); both operands are
// K-contiguous, which is how the artifact stores weights.
//
// Tiling: each wave computes 32 rows x (32·TN) columns (TN 32x32 MFMA tiles);
// a workgroup holds WM x WN waves.  Two shapes: 64 x 128 (2 x 2 waves, TN = 2)
// when that gives at least 256 workgroups, else 32 x 64 (1 x 2 waves, TN = 1)
// so the N = 1024 projections of a 512-token prompt still fill the chip.  K in
// steps of BK (64 when K allows, else 32) staged through LDS, double-buffered:
// the next step's global loads are in flight while the current one is
// multiplied.  LDS rows are padded by 8 halves so the 8-byte fragment reads of
// one MFMA spread over the banks.
#include "capi_common.hpp"
#include "numerics.hpp"

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

template <int WM, int WN, int TN, int BK, bool RES>
__global__ __launch_bounds__(64 * WM * WN) void gemm_nt_kernel(const uint16_t* __restrict__ A,
                                                              const uint16_t* __restrict__ W,
                                                              uint16_t* __restrict__ C,
                                                              const uint16_t* __restrict__ R, int M, int N, int K,
                                                              long long lda, long long ldw, long long ldc) {
  constexpr int BM = 32 * WM, BN = 32 * WN * TN, LDK = BK + 8;
  constexpr int NT = 64 * WM * WN;
  constexpr int PPR = BK / 8;                     // 16-byte pieces per row per step
  constexpr int P = (BM + BN) * PPR / NT;         // pieces per thread per step
  static_assert((BM + BN) * PPR % NT == 0, "staging must divide evenly");
  __shared__ __align__(16) uint16_t As[2][BM][LDK];
  __shared__ __align__(16) uint16_t Ws[2][BN][LDK];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int wm = wave / WN, wn = wave % WN;

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
  const int fk = (lane >> 5) * 4;  // fragment k offset within a step of 8
  load(0);
  store(0);
  __syncthreads();
  const int nk = K / BK;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 8) {
      const half4_t a = *reinterpret_cast<const half4_t*>(&As[buf][wm * 32 + fr][kk + fk]);
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const half4_t b = *reinterpret_cast<const half4_t*>(&Ws[buf][(wn * TN + t) * 32 + fr][kk + fk]);
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x8f16(a, b, acc[t], 0, 0, 0);
      }
    }
    if (kt + 1 < nk) {
      store(buf ^ 1);
      __syncthreads();
    }
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

template <int WM, int WN, int TN, int BK>
void launch_gemm(const uint16_t* A, const uint16_t* W, uint16_t* C, const uint16_t* R, int M, int N, int K,
                 long long lda, long long ldw, long long ldc, hipStream_t s) {
  constexpr int BM = 32 * WM, BN = 32 * WN * TN;
  const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  if (R)
    hipLaunchKernelGGL((gemm_nt_kernel<WM, WN, TN, BK, true>), grid, dim3(64 * WM * WN), 0, s, A, W, C, R, M, N, K,
                       lda, ldw, ldc);
  else
    hipLaunchKernelGGL((gemm_nt_kernel<WM, WN, TN, BK, false>), grid, dim3(64 * WM * WN), 0, s, A, W, C, R, M, N,
                       K, lda, ldw, ldc);
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
  const bool big = (long long)((N + 127) / 128) * ((M + 63) / 64) >= 256;
  if (K % 64 == 0) {
    if (big)
      launch_gemm<2, 2, 2, 64>(A, W, C, residual, M, N, K, lda, ldw, ldc, s);
    else
      launch_gemm<1, 2, 1, 64>(A, W, C, residual, M, N, K, lda, ldw, ldc, s);
  } else {
    if (big)
      launch_gemm<2, 2, 2, 32>(A, W, C, residual, M, N, K, lda, ldw, ldc, s);
    else
      launch_gemm<1, 2, 1, 32>(A, W, C, residual, M, N, K, lda, ldw, ldc, s);
  }
  return spk::check_launch("spk_gemm_f16");
}
