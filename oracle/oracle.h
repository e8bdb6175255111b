/*
 * oracle.h -- CPU restatement of the Spock hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker.  The product (spock_amd/) never
 * links it and has no CPU fallback.
 *
 * Every function cites the reference file:line it restates (paths are relative
 * to the Alexintosh/spock checkout).  Pinning of each function (what checks it
 * beyond its own formula) is listed next to it:
 *
 *   orc_h2f / orc_f2h_rne       exhaustive round trip over all 65536 halves and
 *                               numpy float16 casts (tests/test_oracle_numerics.py)
 *   orc_f2h_trunc               bit rules of vk_session.cpp:69-89; hand cases
 *   orc_expf / orc_logf         against float64 exp/log over 2^20 points (<=2 ulp)
 *   orc_chunk_rule              bit-exact against the reference's own compiled
 *                               deltanet_chunk.cpp (oracle/_ref) and against an
 *                               fp64 token-sequential recurrence; special cases
 *                               (C=1, beta=0, padding, orthonormal overwrite)
 *   orc_delta_recurrence_f64    closed form of the gated delta rule; brute force
 *   orc_recurrent               reference GPU capture tests/data/layer0_step1_* of
 *                               deltanet_recurrent.comp (<=2 fp16 ulp)
 *   orc_conv_l2_qk              T decode steps against torch's depthwise
 *                               conv1d (HF's causal-conv formulation) + SiLU +
 *                               fp16 + per-head L2 in fp64; one-hot taps select
 *                               the lagged input (tests/test_oracle_decode_pins.py)
 *   orc_gbeta                   g at a + dt_bias = 0 equals -e^{A_log} ln 2;
 *                               torch softplus / sigmoid in fp64 below softplus's
 *                               threshold; the shader's large-argument limits
 *   orc_norm_gate_f16 / orc_norm_gate_row  the reference GPU captures
 *                               layer0_step1_dn_core + dn_z -> dn_gated: a norm
 *                               weight fitted with each head held out reproduces
 *                               it within 1 fp16 ulp (2 for head 0, whose core is
 *                               subnormal); wrong variants (sigmoid gate, sum
 *                               instead of mean, one norm across heads, eps
 *                               outside the root) miss by > 100 ulp; the fused
 *                               row equals the unfused form
 *   orc_recurrent_gbeta_norm_gate  composed of orc_gbeta, the recurrence (as
 *                               orc_recurrent) and orc_norm_gate_row, each pinned
 *                               above; beta also by the layer0 g_beta capture
 *   orc_matvec_f16 / orc_lm_head  fp64 dot products -> one RNE rounding (<=1 ulp)
 *   orc_matvec_f16_strided / _serial  the same fp64 bound, and cancellation rows
 *                               (+L and -L placed in one lane's chain, x = 1,
 *                               small exact terms elsewhere) whose exact sum
 *                               only the named order keeps: the other orders
 *                               absorb small terms into L first
 *   orc_argmax_f16              brute-force emulation of argmax.comp's lane/tree
 *                               order on crafted tie patterns
 */
#ifndef SPOCK_ORACLE_H
#define SPOCK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 helpers (vk_session.cpp:28-55, :69-89) ---------------------- */
float orc_h2f(uint16_t h);
uint16_t orc_f2h_rne(float f);
uint16_t orc_f2h_trunc(float f);
void orc_h2f_array(const uint16_t* in, float* out, size_t n);
void orc_f2h_rne_array(const float* in, uint16_t* out, size_t n);

/* ---- deterministic transcendental functions --------------------------- */
float orc_expf(float x);
float orc_logf(float x);
float orc_rsqrtf(float x);
void orc_expf_array(const float* in, float* out, size_t n);
void orc_logf_array(const float* in, float* out, size_t n);

/* ---- chunk rule (src/runtime/deltanet_chunk.cpp:53-284) ---------------- */
/* Returns 0 on success, -1 on a zero config field (deltanet_chunk.cpp:55-58).
 * q,k: [H][T][dk]; v: [H][T][dv]; g,beta: [H][T]; init: [H][dk][dv] or NULL;
 * out_core: [H][T][dv]; out_state: [H][dk][dv]. */
int orc_chunk_rule(size_t H, size_t T, size_t dk, size_t dv, size_t C,
                   int use_qk_l2norm, const float* q, const float* k,
                   const float* v, const float* g, const float* beta,
                   const float* init, float* out_core, float* out_state);

/* orc_chunk_rule with every exp evaluated by orc_expf (the deterministic exp
 * the GPU kernels share) instead of the C library's expf: the chunk rule of the
 * full-model restatement (model.h) and of spk_chunk_prefill_ordered. */
int orc_chunk_rule_det(size_t H, size_t T, size_t dk, size_t dv, size_t C,
                       int use_qk_l2norm, const float* q, const float* k,
                       const float* v, const float* g, const float* beta,
                       const float* init, float* out_core, float* out_state);

/* Packed varlen form: q/k/v are [H][N][d] with sequence s on tokens
 * [cu[s], cu[s+1]); each sequence is chunked from its own start.
 * init (nullable) and out_state are [S][H][dk][dv]; out_core is [H][N][dv]. */
int orc_chunk_rule_varlen(size_t H, size_t N, size_t dk, size_t dv, size_t C,
                          int use_qk_l2norm, const int32_t* cu_seqlens,
                          size_t num_seqs, const float* q, const float* k,
                          const float* v, const float* g, const float* beta,
                          const float* init, float* out_core, float* out_state);

/* fp64 token-by-token gated delta rule (the closed form the chunk rule equals):
 * S_t = e^{g_t} S_{t-1} + k_t (beta_t (v_t - e^{g_t} S_{t-1}^T k_t))^T,
 * o_t = S_t^T (q_t * scale).  Same layouts as orc_chunk_rule, doubles. */
void orc_delta_recurrence_f64(size_t H, size_t T, size_t dk, size_t dv,
                              int use_qk_l2norm, const double* q,
                              const double* k, const double* v,
                              const double* g, const double* beta,
                              const double* init, double* out_core,
                              double* out_state);

/* ---- prefill collect / last-token hand-off ----------------------------- */
/* deltanet_prefill_collect.comp:75-108 (one token) */
void orc_prefill_collect(size_t H, size_t T, size_t token_idx, size_t dk,
                         size_t dv, const uint16_t* dn_qkv, const float* g_beta,
                         float* q_out, float* k_out, float* v_out,
                         float* g_out, float* beta_out);
/* deltanet_chunk_last_to_fp16.comp:37-77: dst[h*dv+d] = trunc16(src[(h*total+T-1)*dv+d]) */
void orc_chunk_last_to_fp16(size_t H, size_t dv, size_t T, size_t total_seq,
                            const float* src, uint16_t* dst);

/* ---- decode step -------------------------------------------------------- */
/* deltanet_conv_l2_qk.comp:41-111 for one sequence.  qkv [conv_dim] fp16 in/out,
 * conv_state [conv_dim][ks] fp16 in/out (channel-major), conv_w [conv_dim][ks]. */
void orc_conv_l2_qk(size_t conv_dim, size_t ks, size_t key_total,
                    size_t num_heads, uint16_t* qkv, uint16_t* conv_state,
                    const uint16_t* conv_w);

/* deltanet_recurrent_gbeta_norm_gate.comp:91-225 for one sequence, head-block
 * of 128 (k_dim == v_dim == 128).  qkv: [Q nh*128 | K nh*128 | V nh*128] fp16,
 * V section overwritten with the gated output.  state [nh][128][128] fp32. */
void orc_recurrent_gbeta_norm_gate(size_t num_heads, size_t layer_idx,
                                   float q_scale, float eps, const uint16_t* a,
                                   const uint16_t* b, const float* a_log_bias,
                                   uint16_t* qkv, float* state,
                                   const uint16_t* z, const float* norm_w);

/* g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b) for one head
 * (deltanet_recurrent_gbeta_norm_gate.comp:102-116). */
void orc_gbeta(float a, float b, float a_log, float dt_bias, float* g, float* beta);

/* Gated RMSNorm of one fp32 head row of 128 (the fused shader's :182-224):
 * out = fp16(fp16(w * o * r) * silu(z)), r = 1/sqrt(tree128(o^2)/128 + eps). */
void orc_norm_gate_row(const float* o, const uint16_t* z, const float* norm_w,
                       float eps, uint16_t* out);

/* deltanet_norm_gate.comp:80-105 (unfused, fp16 input): io [nh][128] fp16 in
 * place, z [nh][128] fp16, norm_w [128] fp32. */
void orc_norm_gate_f16(size_t num_heads, float eps, uint16_t* io, const uint16_t* z,
                       const float* norm_w);

/* deltanet_recurrent.comp (unfused): g/beta read from the state tail
 * state[nh*128*128 + h] / state[nh*128*128 + nh + h]; output fp16 into V. */
void orc_recurrent(size_t num_heads, float q_scale, uint16_t* qkv, float* state);

/* Fused decode step for B sequences (conv_l2_qk then recurrent_gbeta_norm_gate),
 * strides in elements. */
void orc_decode_step(size_t B, size_t num_heads, size_t layer_idx, float q_scale,
                     float eps, uint16_t* qkv, size_t qkv_stride,
                     uint16_t* conv_state, size_t conv_stride,
                     const uint16_t* conv_w, const uint16_t* a,
                     const uint16_t* b, size_t ab_stride,
                     const float* a_log_bias, float* state, size_t state_stride,
                     const uint16_t* z, size_t z_stride, const float* norm_w);

/* ---- matvec / lm_head / argmax ----------------------------------------- */
/* y[r] = fp16(sum_j W[r][j]*x[j]) in lm_head_tiled.comp:40-87 order: lane l of 64
 * sums the contiguous span [l*in/64, (l+1)*in/64) sequentially, then the
 * 64-lane tree with strides 32..1.  Requires in % 64 == 0 (lm_head_tiled.comp:46). */
int orc_matvec_f16(const uint16_t* W, const uint16_t* x, uint16_t* y,
                   size_t out_dim, size_t in_dim);
/* matvec_tiled.comp:41-84 order: lane l sums j = l, l+64, ... sequentially,
 * then the 32..1 tree; any in_dim > 0. */
int orc_matvec_f16_strided(const uint16_t* W, const uint16_t* x, uint16_t* y,
                           size_t out_dim, size_t in_dim);
/* matvec.comp:28-41 order: one sequential sum over j; any in_dim > 0. */
int orc_matvec_f16_serial(const uint16_t* W, const uint16_t* x, uint16_t* y,
                          size_t out_dim, size_t in_dim);
/* argmax.comp:27-63 exactly (256 lanes, contiguous blocks, strict-greater tree) */
uint32_t orc_argmax_f16(const uint16_t* vals, size_t n);
/* lm_head logits (matvec) + argmax; logits may be NULL */
uint32_t orc_lm_head_argmax(const uint16_t* W, const uint16_t* x, size_t vocab,
                            size_t hidden, uint16_t* logits);

#ifdef __cplusplus
}
#endif
#endif
