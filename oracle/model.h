/*
 * model.h -- CPU restatement of the full Qwen3.5-0.8B-shaped text model
 * (24 layers: gated DeltaNet x3 then full attention, repeated), the forward
 * that Spock's DecodeSession runs (src/runtime/vk_session.cpp decode loop
 * :2560-3400, final norm + lm_head + argmax :3533-3563).  TEST INFRASTRUCTURE
 * ONLY (same rules as oracle.h: tests/, smoke() and bench.py's cpu_baseline may
 * use it, only as the checker).
 *
 * Numerics.  Every decode-path operation is a fixed IEEE fp32 sequence that
 * the HIP kernels evaluate identically, so a decode step from identical state
 * gives identical bits:
 *   RMSNorm(1+w) over 1024 (rms_norm.comp): 256 partials p_t = fma chain of
 *     x^2 over elements 4t..4t+3, tree s[t] += s[t+stride] (stride 128..1),
 *     nf = 1/sqrt(sum/1024 + 1e-6), y = fp16((x*nf)*(1+w)).
 *   per-head RMSNorm(1+w) over 256 (rms_norm_per_head.comp): p_t = x_t^2, same
 *     tree, nf = 1/sqrt(sum/256 + 1e-6).
 *   GEMV: orc_matvec_f16's order (64 contiguous spans, then a 32..1 tree).
 *   residual (residual_add.comp): fp16(a + b).
 *   SiLU gate (silu_gate.comp): fp16((g / (1 + exp(-g))) * u).
 *   sigmoid gate (sigmoid_gate.comp): fp16(v * (1 / (1 + exp(-g)))).
 *   RoPE (rope_apply.comp): pairs (i, i+32) of the first 64 dims,
 *     y_i = fp16(x_i c - x_{i+32} s), y_{i+32} = fp16(x_{i+32} c + x_i s);
 *     table c/s = float(cos/sin(pos * 1e7^(-2i/64))) evaluated in double.
 *   attention (attention_decode.comp's softmax(q.K^T/16) V, evaluated over
 *     blocks of 64 positions): score_p = (sequential fma dot over d) * 1/16;
 *     per block m_b = max, w_p = exp(score_p - m_b), S_b = 64-lane tree of w_p,
 *     O_b[d] = fma chain over p ascending; then M = max_b m_b,
 *     c_b = exp(m_b - M), tot = sum_b S_b*c_b and O[d] = sum_b O_b[d]*c_b in
 *     block order, out = fp16(O[d] * (1 / (tot + 1e-30))).
 *   DeltaNet layer: orc_conv_l2_qk + orc_recurrent_gbeta_norm_gate.
 *   exp/log: orc_expf/orc_logf.
 * Prefill (HF semantics, modeling_qwen3_5.py:519-530): layer-major over the
 * prompt; every per-token operation is the decode one, except that the
 * DeltaNet recurrence over the prompt is the chunk rule (orc_chunk_rule_det:
 * run_deltanet_chunk_rule's loops with orc_expf; C = 64, q/k already
 * L2-normalised in fp16, initial state = the layer's state) and the
 * norm-gate uses its fp32 core output.
 */
#ifndef SPOCK_ORACLE_MODEL_H
#define SPOCK_ORACLE_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_MAX_LAYERS 64
#define ORC_HIDDEN 1024
#define ORC_INTER 3584
#define ORC_DN_HEADS 16
#define ORC_DN_DIM 128
#define ORC_CONV_DIM 6144
#define ORC_Q_HEADS 8
#define ORC_KV_HEADS 2
#define ORC_HEAD_DIM 256
#define ORC_ROT_DIM 64
#define ORC_KV_ROW 1024 /* K 2x256 | V 2x256 fp16 per cached position */

typedef struct OrcLayer {
  int32_t kind; /* 0 gated DeltaNet, 1 full attention */
  int32_t sub_idx; /* index among layers of the same kind */
  const uint16_t *input_norm, *post_norm, *mlp_gate, *mlp_up, *mlp_down;
  /* DeltaNet: in_proj_qkv [6144][1024], z [2048][1024], a/b [16][1024],
   * conv [6144][4], out_proj [1024][2048], dt_bias fp16 [16]; A_log, norm fp32 */
  const uint16_t *dn_qkv, *dn_z, *dn_a, *dn_b, *dn_conv, *dn_out, *dn_dt_bias;
  const float *dn_a_log, *dn_norm;
  /* attention: q [4096][1024] (per head: 256 query rows then 256 gate rows),
   * k/v [512][1024], o [1024][2048], q_norm/k_norm fp16 [256] */
  const uint16_t *attn_q, *attn_k, *attn_v, *attn_o, *attn_q_norm, *attn_k_norm;
} OrcLayer;

typedef struct OrcModel {
  int32_t n_layers;
  int32_t vocab;
  int32_t max_seq;
  int32_t n_dn;
  int32_t n_attn;
  int32_t pad_;
  const uint16_t* embed;      /* [vocab][1024], tied lm_head */
  const uint16_t* final_norm; /* [1024] */
  OrcLayer layers[ORC_MAX_LAYERS];
} OrcModel;

typedef struct OrcModelState {
  float* dn_state;      /* [n_dn][16][128][128] */
  uint16_t* conv_state; /* [n_dn][6144][4] */
  uint16_t* kv_cache;   /* [n_attn][max_seq][1024] */
  float* a_log_bias;    /* [n_dn][16][2], filled by orc_model_init_state */
  float* rope;          /* [max_seq][64] (cos, sin) pairs */
  int32_t pos;
} OrcModelState;

/* RoPE table [max_seq][64]: [2i] = cos, [2i+1] = sin of pos*1e7^(-2i/64). */
void orc_rope_table(int32_t max_seq, float* out);

/* Zeroes the state, fills a_log_bias and rope; pos = 0. */
void orc_model_init_state(const OrcModel* m, OrcModelState* st);

/* Prefill T prompt tokens at positions st->pos.. (layer-major, chunk rule for
 * DeltaNet).  Writes the fp16 logits of the last token (nullable) and the
 * last token's final hidden state before the final norm (nullable, fp16
 * [1024]).  Returns the greedy token. */
uint32_t orc_model_prefill(const OrcModel* m, OrcModelState* st, const int32_t* tokens,
                           int32_t T, uint16_t* last_logits, uint16_t* last_hidden);

/* One decode step of `token` at position st->pos. */
uint32_t orc_model_decode(const OrcModel* m, OrcModelState* st, int32_t token,
                          uint16_t* logits, uint16_t* hidden);

/* prefill + (n_new - 1) decode steps; out_tokens[n_new]. */
void orc_model_generate(const OrcModel* m, OrcModelState* st, const int32_t* prompt,
                        int32_t T, int32_t n_new, int32_t* out_tokens);

/* Experiment switches (robustness of the greedy tokens to prefill rounding):
 * gemm_f64 != 0 evaluates prefill projections as fp64 dots rounded once;
 * chunk_f64 != 0 replaces the chunk rule by the fp64 recurrence. */
void orc_model_set_variant(int32_t gemm_f64, int32_t chunk_f64);

/* single operations, exposed for per-kernel parity tests */
void orc_rmsnorm1024(const uint16_t* x, const uint16_t* w, uint16_t* y);
void orc_head_rmsnorm256(const uint16_t* x, const uint16_t* w, uint16_t* y);
void orc_rope_apply(uint16_t* x, int32_t num_heads, const float* cos_sin_pos);
void orc_attend(const uint16_t* q, const uint16_t* kv_layer, int32_t kv_head,
                int32_t npos, uint16_t* out);
void orc_silu_gate(const uint16_t* g, const uint16_t* u, uint16_t* y, size_t n);
void orc_sigmoid_gate(const uint16_t* v, const uint16_t* g, uint16_t* y, size_t n);
void orc_residual_add(const uint16_t* a, const uint16_t* b, uint16_t* y, size_t n);
/* Y[t][r] = GEMV order dot of W row r with X row t, for T rows at once. */
void orc_matmul_rows(const uint16_t* W, const uint16_t* X, uint16_t* Y, size_t out_dim,
                     size_t in_dim, size_t T);

#ifdef __cplusplus
}
#endif
#endif
