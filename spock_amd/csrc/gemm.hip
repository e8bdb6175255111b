// gemm.hip -- prompt-length projections: C[M][N] = fp16(A[M][K] . W[N][K]^T),
// optionally fp16(R + fp16(A . W^T)) (the residual add after out_proj /
// o_proj / down_proj), fp16 operands, fp32 accumulation on the matrix cores
// (v_mfma_f32_32x32x8_f16).  This is the prefill form of every decode matvec
// (matvec_tiled.comp applied to all prompt tokens at once); both operands are
// K-contiguous, which is how the artifact stores weights.
//
// Tiling: 64 x 128 output tile per 256-thread workgroup (4 waves in 2 x 2,
// each 32 x 64 = two 32x32 MFMA tiles), K in steps of 32 staged through LDS
// (double-buffered; the next step's global loads are in flight while the
// current one is multiplied).  LDS rows are padded to 40 halves so the
// 8-byte fragment reads of one MFMA spread over the banks.
#include "capi_common.hpp"
#include "numerics.hpp"

namespace {

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BM = 64;
constexpr int BN = 128;
constexpr int BK = 32;
constexpr int LDSK = 40;  // padded row length (halves)

template <bool RES>
__global__ __launch_bounds__(256) void gemm_nt_kernel(const uint16_t* __restrict__ A, const uint16_t* __restrict__ W,
                                                      uint16_t* __restrict__ C, const uint16_t* __restrict__ R, int M,
                                                      int N, int K, long long lda, long long ldw, long long ldc) {
  __shared__ __align__(16) uint16_t As[2][BM][LDSK];
  __shared__ __align__(16) uint16_t Ws[2][BN][LDSK];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int m0 = blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int wm = wave >> 1, wn = wave & 1;

  // global -> register staging: A 64x32 (one 16-byte piece per thread), W 128x32 (two)
  const int ar = tid >> 2, ak = (tid & 3) * 8;
  const bool a_ok = m0 + ar < M;
  const bool w0_ok = n0 + ar < N, w1_ok = n0 + 64 + ar < N;
  const uint16_t* a_src = A + (long long)(a_ok ? m0 + ar : 0) * lda + ak;
  const uint16_t* w0_src = W + (long long)(w0_ok ? n0 + ar : 0) * ldw + ak;
  const uint16_t* w1_src = W + (long long)(w1_ok ? n0 + 64 + ar : 0) * ldw + ak;
  uint4 ra, rw0, rw1;
  auto load = [&](int k0) {
    const uint4 z = make_uint4(0, 0, 0, 0);
    ra = a_ok ? *reinterpret_cast<const uint4*>(a_src + k0) : z;
    rw0 = w0_ok ? *reinterpret_cast<const uint4*>(w0_src + k0) : z;
    rw1 = w1_ok ? *reinterpret_cast<const uint4*>(w1_src + k0) : z;
  };
  auto store = [&](int buf) {
    *reinterpret_cast<uint4*>(&As[buf][ar][ak]) = ra;
    *reinterpret_cast<uint4*>(&Ws[buf][ar][ak]) = rw0;
    *reinterpret_cast<uint4*>(&Ws[buf][64 + ar][ak]) = rw1;
  };

  floatx16 acc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
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
      for (int t = 0; t < 2; ++t) {
        const half4_t b = *reinterpret_cast<const half4_t*>(&Ws[buf][wn * 64 + t * 32 + fr][kk + fk]);
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
  for (int t = 0; t < 2; ++t) {
    const int col = n0 + wn * 64 + t * 32 + fr;
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

}  // namespace

extern "C" int spk_gemm_f16(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw, uint16_t* C, int64_t ldc,
                            const uint16_t* residual, int32_t M, int32_t N, int32_t K, spk_stream_t stream) {
  if (!A || !W || !C) return spk::fail(SPK_ERR_NULL, "spk_gemm_f16: NULL pointer");
  if (M <= 0 || N <= 0 || K <= 0 || K % BK != 0)
    return spk::fail(SPK_ERR_SHAPE, "spk_gemm_f16: M %d N %d K %d (K must be a positive multiple of %d)", M, N, K, BK);
  if (lda < K || ldw < K || ldc < N || lda % 8 || ldw % 8)
    return spk::fail(SPK_ERR_SHAPE, "spk_gemm_f16: leading dimensions (lda %lld ldw %lld ldc %lld)", (long long)lda,
                     (long long)ldw, (long long)ldc);
  if (!spk::aligned(A, 16) || !spk::aligned(W, 16))
    return spk::fail(SPK_ERR_ALIGN, "spk_gemm_f16: A and W must be 16-byte aligned");
  if (residual == A || residual == W || C == A || C == W)
    return spk::fail(SPK_ERR_ARG, "spk_gemm_f16: the output or residual aliases an operand");
  dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
  hipStream_t s = spk::to_hip(stream);
  if (residual)
    hipLaunchKernelGGL(gemm_nt_kernel<true>, grid, dim3(256), 0, s, A, W, C, residual, M, N, K, (long long)lda,
                       (long long)ldw, (long long)ldc);
  else
    hipLaunchKernelGGL(gemm_nt_kernel<false>, grid, dim3(256), 0, s, A, W, C, residual, M, N, K, (long long)lda,
                       (long long)ldw, (long long)ldc);
  return spk::check_launch("spk_gemm_f16");
}
