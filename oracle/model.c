/*
 * model.c -- CPU restatement of the Qwen3.5-0.8B-shaped text model forward
 * (Spock DecodeSession decode loop, src/runtime/vk_session.cpp:2560-3400, and
 * the HF prefill semantics of modeling_qwen3_5.py:519-530 / :740-795).
 * TEST INFRASTRUCTURE ONLY; see model.h for the operation order it pins.
 */
#include "model.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static int g_gemm_f64 = 0;
static int g_chunk_f64 = 0;

void orc_model_set_variant(int32_t gemm_f64, int32_t chunk_f64) {
  g_gemm_f64 = gemm_f64;
  g_chunk_f64 = chunk_f64;
}

#define H2F orc_h2f
#define F2H orc_f2h_rne

static float tree_pow2(float* s, size_t n) {
  for (size_t stride = n / 2; stride > 0; stride >>= 1)
    for (size_t l = 0; l < stride; ++l) s[l] = s[l] + s[l + stride];
  return s[0];
}

static inline float silu_f(float x) { return x / (1.0f + orc_expf(-x)); }

/* ---- element-wise operations ------------------------------------------- */

/* rms_norm.comp:40-78 with 256 lanes of 4 contiguous elements. */
void orc_rmsnorm1024(const uint16_t* x, const uint16_t* w, uint16_t* y) {
  float p[256];
  for (size_t t = 0; t < 256; ++t) {
    float acc = 0.0f;
    for (size_t i = 0; i < 4; ++i) {
      const float v = H2F(x[4 * t + i]);
      acc = fmaf(v, v, acc);
    }
    p[t] = acc;
  }
  const float sum = tree_pow2(p, 256);
  const float nf = 1.0f / sqrtf(sum / 1024.0f + 1e-6f);
  for (size_t i = 0; i < ORC_HIDDEN; ++i)
    y[i] = F2H((H2F(x[i]) * nf) * (1.0f + H2F(w[i])));
}

/* rms_norm_per_head.comp:35-70 (head_dim 256, one element per lane). */
void orc_head_rmsnorm256(const uint16_t* x, const uint16_t* w, uint16_t* y) {
  float p[256], v[256];
  for (size_t t = 0; t < 256; ++t) {
    v[t] = H2F(x[t]);
    p[t] = v[t] * v[t];
  }
  const float sum = tree_pow2(p, 256);
  const float nf = 1.0f / sqrtf(sum / 256.0f + 1e-6f);
  for (size_t t = 0; t < 256; ++t) y[t] = F2H((v[t] * nf) * (1.0f + H2F(w[t])));
}

/* rope_apply.comp:30-62: rotary pairs (i, i+32) of the first 64 dims. */
void orc_rope_apply(uint16_t* x, int32_t num_heads, const float* cs) {
  for (int32_t h = 0; h < num_heads; ++h) {
    uint16_t* b = x + (size_t)h * ORC_HEAD_DIM;
    for (size_t i = 0; i < ORC_ROT_DIM / 2; ++i) {
      const float c = cs[2 * i], s = cs[2 * i + 1];
      const float v0 = H2F(b[i]), v1 = H2F(b[i + 32]);
      b[i] = F2H(v0 * c - v1 * s);
      b[i + 32] = F2H(v1 * c + v0 * s);
    }
  }
}

/* vk_session.cpp:332-346's table, evaluated in double and rounded once. */
void orc_rope_table(int32_t max_seq, float* out) {
  for (int32_t pos = 0; pos < max_seq; ++pos)
    for (int32_t i = 0; i < ORC_ROT_DIM / 2; ++i) {
      const double inv_freq = pow(1.0e7, -(2.0 * i) / (double)ORC_ROT_DIM);
      const double ang = (double)pos * inv_freq;
      out[(size_t)pos * ORC_ROT_DIM + 2 * i] = (float)cos(ang);
      out[(size_t)pos * ORC_ROT_DIM + 2 * i + 1] = (float)sin(ang);
    }
}

/* attention_decode.comp:45-119 (softmax(q K^T / 16) V for one query head),
 * evaluated over blocks of 64 positions in the order stated in model.h. */
void orc_attend(const uint16_t* q, const uint16_t* kv, int32_t kv_head, int32_t npos,
                uint16_t* out) {
  const int32_t nb = (npos + 63) / 64;
  float* mb = (float*)malloc(sizeof(float) * nb);
  float* sb = (float*)malloc(sizeof(float) * nb);
  float* ob = (float*)malloc(sizeof(float) * nb * ORC_HEAD_DIM);
  float qf[ORC_HEAD_DIM];
  for (size_t d = 0; d < ORC_HEAD_DIM; ++d) qf[d] = H2F(q[d]);
  for (int32_t b = 0; b < nb; ++b) {
    float sc[64], w[64];
    float m = -INFINITY;
    for (int32_t l = 0; l < 64; ++l) {
      const int32_t p = 64 * b + l;
      if (p >= npos) break;
      const uint16_t* kp = kv + (size_t)p * ORC_KV_ROW + (size_t)kv_head * ORC_HEAD_DIM;
      float dot = 0.0f;
      for (size_t d = 0; d < ORC_HEAD_DIM; ++d) dot = fmaf(qf[d], H2F(kp[d]), dot);
      sc[l] = dot * 0.0625f;
      m = fmaxf(m, sc[l]);
    }
    for (int32_t l = 0; l < 64; ++l) w[l] = (64 * b + l < npos) ? orc_expf(sc[l] - m) : 0.0f;
    float tw[64];
    memcpy(tw, w, sizeof(tw));
    mb[b] = m;
    sb[b] = tree_pow2(tw, 64);
    for (size_t d = 0; d < ORC_HEAD_DIM; ++d) {
      float acc = 0.0f;
      for (int32_t l = 0; l < 64; ++l) {
        const int32_t p = 64 * b + l;
        if (p >= npos) break;
        const uint16_t* vp = kv + (size_t)p * ORC_KV_ROW + 512 + (size_t)kv_head * ORC_HEAD_DIM;
        acc = fmaf(w[l], H2F(vp[d]), acc);
      }
      ob[(size_t)b * ORC_HEAD_DIM + d] = acc;
    }
  }
  float M = -INFINITY;
  for (int32_t b = 0; b < nb; ++b) M = fmaxf(M, mb[b]);
  float tot = 0.0f;
  for (int32_t b = 0; b < nb; ++b) {
    mb[b] = orc_expf(mb[b] - M); /* now the block's rescale factor */
    tot = tot + sb[b] * mb[b];
  }
  const float inv = 1.0f / (tot + 1e-30f);
  for (size_t d = 0; d < ORC_HEAD_DIM; ++d) {
    float o = 0.0f;
    for (int32_t b = 0; b < nb; ++b) o = o + ob[(size_t)b * ORC_HEAD_DIM + d] * mb[b];
    out[d] = F2H(o * inv);
  }
  free(mb);
  free(sb);
  free(ob);
}

/* silu_gate.comp:28-39 */
void orc_silu_gate(const uint16_t* g, const uint16_t* u, uint16_t* y, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float gv = H2F(g[i]);
    y[i] = F2H((gv / (1.0f + orc_expf(-gv))) * H2F(u[i]));
  }
}

/* sigmoid_gate.comp:28-39 */
void orc_sigmoid_gate(const uint16_t* v, const uint16_t* g, uint16_t* y, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float sig = 1.0f / (1.0f + orc_expf(-H2F(g[i])));
    y[i] = F2H(H2F(v[i]) * sig);
  }
}

/* residual_add.comp:28-37 */
void orc_residual_add(const uint16_t* a, const uint16_t* b, uint16_t* y, size_t n) {
  for (size_t i = 0; i < n; ++i) y[i] = F2H(H2F(a[i]) + H2F(b[i]));
}

/* ---- projections ----------------------------------------------------------- */

static void matmul_impl(const uint16_t* W, const uint16_t* X, uint16_t* Y, size_t out_dim,
                        size_t in_dim, size_t T, int f64) {
  const size_t span = in_dim / 64;
  float* XT = (float*)malloc(sizeof(float) * in_dim * T);
  for (size_t t = 0; t < T; ++t)
    for (size_t j = 0; j < in_dim; ++j) XT[j * T + t] = H2F(X[t * in_dim + j]);
#pragma omp parallel
  {
    float* part = (float*)malloc(sizeof(float) * 64 * T);
    double* dpart = f64 ? (double*)malloc(sizeof(double) * T) : NULL;
    float* wr = (float*)malloc(sizeof(float) * in_dim);
#pragma omp for schedule(static)
    for (size_t r = 0; r < out_dim; ++r) {
      const uint16_t* row = W + r * in_dim;
      for (size_t j = 0; j < in_dim; ++j) wr[j] = H2F(row[j]);
      if (f64) {
        for (size_t t = 0; t < T; ++t) dpart[t] = 0.0;
        for (size_t j = 0; j < in_dim; ++j) {
          const double w = wr[j];
          const float* xr = XT + j * T;
          for (size_t t = 0; t < T; ++t) dpart[t] += w * (double)xr[t];
        }
        for (size_t t = 0; t < T; ++t) Y[t * out_dim + r] = F2H((float)dpart[t]);
        continue;
      }
      for (size_t l = 0; l < 64; ++l) {
        float* pl = part + l * T;
        for (size_t t = 0; t < T; ++t) pl[t] = 0.0f;
        for (size_t j = l * span; j < (l + 1) * span; ++j) {
          const float w = wr[j];
          const float* xr = XT + j * T;
          for (size_t t = 0; t < T; ++t) pl[t] = fmaf(w, xr[t], pl[t]);
        }
      }
      for (size_t stride = 32; stride > 0; stride >>= 1)
        for (size_t l = 0; l < stride; ++l) {
          float* a = part + l * T;
          const float* b = part + (l + stride) * T;
          for (size_t t = 0; t < T; ++t) a[t] = a[t] + b[t];
        }
      for (size_t t = 0; t < T; ++t) Y[t * out_dim + r] = F2H(part[t]);
    }
    free(part);
    free(dpart);
    free(wr);
  }
  free(XT);
}

void orc_matmul_rows(const uint16_t* W, const uint16_t* X, uint16_t* Y, size_t out_dim,
                     size_t in_dim, size_t T) {
  matmul_impl(W, X, Y, out_dim, in_dim, T, 0);
}

/* ---- model ----------------------------------------------------------------- */

void orc_model_init_state(const OrcModel* m, OrcModelState* st) {
  memset(st->dn_state, 0, sizeof(float) * (size_t)m->n_dn * ORC_DN_HEADS * 128 * 128);
  memset(st->conv_state, 0, 2 * (size_t)m->n_dn * ORC_CONV_DIM * 4);
  memset(st->kv_cache, 0, 2 * (size_t)m->n_attn * m->max_seq * ORC_KV_ROW);
  for (int32_t L = 0; L < m->n_layers; ++L) {
    const OrcLayer* ly = &m->layers[L];
    if (ly->kind != 0) continue;
    for (int32_t h = 0; h < ORC_DN_HEADS; ++h) {
      st->a_log_bias[((size_t)ly->sub_idx * ORC_DN_HEADS + h) * 2] = ly->dn_a_log[h];
      st->a_log_bias[((size_t)ly->sub_idx * ORC_DN_HEADS + h) * 2 + 1] = H2F(ly->dn_dt_bias[h]);
    }
  }
  orc_rope_table(m->max_seq, st->rope);
  st->pos = 0;
}

static float dn_q_scale(void) { return 1.0f / sqrtf(128.0f); }

/* Attention token mixer for T consecutive tokens at positions p0.. of one
 * layer (the decode sequence of vk_session.cpp:2676-2790 per token). */
static void attn_mixer(const OrcModel* m, OrcModelState* st, const OrcLayer* ly, const uint16_t* XN,
                       int32_t T, int32_t p0, uint16_t* MIX) {
  uint16_t* QG = (uint16_t*)malloc(2 * (size_t)T * 4096);
  uint16_t* K = (uint16_t*)malloc(2 * (size_t)T * 512);
  uint16_t* V = (uint16_t*)malloc(2 * (size_t)T * 512);
  uint16_t* Q = (uint16_t*)malloc(2 * (size_t)T * 2048);
  uint16_t* G = (uint16_t*)malloc(2 * (size_t)T * 2048);
  const int f64 = g_gemm_f64 && T > 1;
  matmul_impl(ly->attn_q, XN, QG, 4096, ORC_HIDDEN, T, f64);
  matmul_impl(ly->attn_k, XN, K, 512, ORC_HIDDEN, T, f64);
  matmul_impl(ly->attn_v, XN, V, 512, ORC_HIDDEN, T, f64);
  uint16_t* kv = st->kv_cache + (size_t)ly->sub_idx * m->max_seq * ORC_KV_ROW;
  for (int32_t t = 0; t < T; ++t) {
    const int32_t pos = p0 + t;
    uint16_t* q = Q + (size_t)t * 2048;
    uint16_t* k = K + (size_t)t * 512;
    for (int32_t h = 0; h < ORC_Q_HEADS; ++h) {  /* split_q_gate.comp:27-45 */
      memcpy(q + h * 256, QG + (size_t)t * 4096 + h * 512, 512);
      orc_head_rmsnorm256(q + h * 256, ly->attn_q_norm, q + h * 256);
    }
    for (int32_t h = 0; h < ORC_KV_HEADS; ++h) orc_head_rmsnorm256(k + h * 256, ly->attn_k_norm, k + h * 256);
    orc_rope_apply(q, ORC_Q_HEADS, st->rope + (size_t)pos * ORC_ROT_DIM);
    orc_rope_apply(k, ORC_KV_HEADS, st->rope + (size_t)pos * ORC_ROT_DIM);
    uint16_t* row = kv + (size_t)pos * ORC_KV_ROW;  /* kv_cache_store.comp:27-48 */
    memcpy(row, k, 1024);
    memcpy(row + 512, V + (size_t)t * 512, 1024);
  }
#pragma omp parallel for schedule(dynamic) collapse(2)
  for (int32_t t = 0; t < T; ++t)
    for (int32_t h = 0; h < ORC_Q_HEADS; ++h) {
      uint16_t att[256];
      orc_attend(Q + (size_t)t * 2048 + h * 256, kv, h / (ORC_Q_HEADS / ORC_KV_HEADS), p0 + t + 1, att);
      orc_sigmoid_gate(att, QG + (size_t)t * 4096 + h * 512 + 256, G + (size_t)t * 2048 + h * 256, 256);
    }
  matmul_impl(ly->attn_o, G, MIX, ORC_HIDDEN, 2048, T, f64);
  free(QG); free(K); free(V); free(Q); free(G);
}

/* DeltaNet token mixer for T tokens: per-token conv/L2 and g/beta of the fused
 * decode shaders, then the chunk rule over the span (T > 1) or the fused
 * recurrence (T == 1). */
static void dn_mixer(const OrcModel* m, OrcModelState* st, const OrcLayer* ly, const uint16_t* XN,
                     int32_t T, uint16_t* MIX) {
  (void)m;
  const int f64 = g_gemm_f64 && T > 1;
  uint16_t* QKV = (uint16_t*)malloc(2 * (size_t)T * ORC_CONV_DIM);
  uint16_t* Z = (uint16_t*)malloc(2 * (size_t)T * 2048);
  uint16_t* A = (uint16_t*)malloc(2 * (size_t)T * 16);
  uint16_t* B = (uint16_t*)malloc(2 * (size_t)T * 16);
  matmul_impl(ly->dn_qkv, XN, QKV, ORC_CONV_DIM, ORC_HIDDEN, T, f64);
  matmul_impl(ly->dn_z, XN, Z, 2048, ORC_HIDDEN, T, f64);
  matmul_impl(ly->dn_a, XN, A, 16, ORC_HIDDEN, T, f64);
  matmul_impl(ly->dn_b, XN, B, 16, ORC_HIDDEN, T, f64);
  float* S = st->dn_state + (size_t)ly->sub_idx * ORC_DN_HEADS * 128 * 128;
  uint16_t* cs = st->conv_state + (size_t)ly->sub_idx * ORC_CONV_DIM * 4;
  const float eps = 1e-6f;
  if (T == 1) {
    orc_conv_l2_qk(ORC_CONV_DIM, 4, 2048, ORC_DN_HEADS, QKV, cs, ly->dn_conv);
    orc_recurrent_gbeta_norm_gate(ORC_DN_HEADS, (size_t)ly->sub_idx, dn_q_scale(), eps, A, B,
                                  st->a_log_bias, QKV, S, Z, ly->dn_norm);
    matmul_impl(ly->dn_out, QKV + 4096, MIX, ORC_HIDDEN, 2048, 1, 0);
  } else {
    for (int32_t t = 0; t < T; ++t)
      orc_conv_l2_qk(ORC_CONV_DIM, 4, 2048, ORC_DN_HEADS, QKV + (size_t)t * ORC_CONV_DIM, cs, ly->dn_conv);
    const size_t HT = (size_t)ORC_DN_HEADS * T;
    float* q = (float*)malloc(sizeof(float) * HT * 128);
    float* k = (float*)malloc(sizeof(float) * HT * 128);
    float* v = (float*)malloc(sizeof(float) * HT * 128);
    float* g = (float*)malloc(sizeof(float) * HT);
    float* beta = (float*)malloc(sizeof(float) * HT);
    float* core = (float*)malloc(sizeof(float) * HT * 128);
    float* init = (float*)malloc(sizeof(float) * ORC_DN_HEADS * 128 * 128);
    memcpy(init, S, sizeof(float) * ORC_DN_HEADS * 128 * 128);
    for (int32_t t = 0; t < T; ++t) {
      const uint16_t* row = QKV + (size_t)t * ORC_CONV_DIM;
      for (int32_t h = 0; h < ORC_DN_HEADS; ++h) {
        for (size_t d = 0; d < 128; ++d) {
          q[((size_t)h * T + t) * 128 + d] = H2F(row[h * 128 + d]);
          k[((size_t)h * T + t) * 128 + d] = H2F(row[2048 + h * 128 + d]);
          v[((size_t)h * T + t) * 128 + d] = H2F(row[4096 + h * 128 + d]);
        }
        orc_gbeta(H2F(A[(size_t)t * 16 + h]), H2F(B[(size_t)t * 16 + h]),
                  st->a_log_bias[((size_t)ly->sub_idx * 16 + h) * 2],
                  st->a_log_bias[((size_t)ly->sub_idx * 16 + h) * 2 + 1],
                  &g[(size_t)h * T + t], &beta[(size_t)h * T + t]);
      }
    }
    if (!g_chunk_f64) {
#pragma omp parallel for schedule(static)
      for (int32_t h = 0; h < ORC_DN_HEADS; ++h) {
        const size_t o = (size_t)h * T;
        orc_chunk_rule_det(1, (size_t)T, 128, 128, 64, 0, q + o * 128, k + o * 128, v + o * 128, g + o,
                           beta + o, init + (size_t)h * 128 * 128, core + o * 128, S + (size_t)h * 128 * 128);
      }
    } else {
#pragma omp parallel for schedule(static)
      for (int32_t h = 0; h < ORC_DN_HEADS; ++h) {
        const size_t o = (size_t)h * T, nt = (size_t)T * 128;
        double* dq = (double*)malloc(sizeof(double) * nt);
        double* dk = (double*)malloc(sizeof(double) * nt);
        double* dv = (double*)malloc(sizeof(double) * nt);
        double* dg = (double*)malloc(sizeof(double) * T);
        double* db = (double*)malloc(sizeof(double) * T);
        double* di = (double*)malloc(sizeof(double) * 128 * 128);
        double* dc = (double*)malloc(sizeof(double) * nt);
        double* ds = (double*)malloc(sizeof(double) * 128 * 128);
        for (size_t i = 0; i < nt; ++i) { dq[i] = q[o * 128 + i]; dk[i] = k[o * 128 + i]; dv[i] = v[o * 128 + i]; }
        for (int32_t t = 0; t < T; ++t) { dg[t] = g[o + t]; db[t] = beta[o + t]; }
        for (size_t i = 0; i < 128 * 128; ++i) di[i] = init[(size_t)h * 128 * 128 + i];
        orc_delta_recurrence_f64(1, (size_t)T, 128, 128, 0, dq, dk, dv, dg, db, di, dc, ds);
        for (size_t i = 0; i < nt; ++i) core[o * 128 + i] = (float)dc[i];
        for (size_t i = 0; i < 128 * 128; ++i) S[(size_t)h * 128 * 128 + i] = (float)ds[i];
        free(dq); free(dk); free(dv); free(dg); free(db); free(di); free(dc); free(ds);
      }
    }
    /* norm-gate of deltanet_recurrent_gbeta_norm_gate.comp:182-224 on the fp32 core */
    uint16_t* Gt = (uint16_t*)malloc(2 * (size_t)T * 2048);
#pragma omp parallel for schedule(static)
    for (int32_t t = 0; t < T; ++t)
      for (int32_t h = 0; h < ORC_DN_HEADS; ++h)
        orc_norm_gate_row(core + ((size_t)h * T + t) * 128, Z + (size_t)t * 2048 + h * 128,
                          ly->dn_norm, eps, Gt + (size_t)t * 2048 + h * 128);
    matmul_impl(ly->dn_out, Gt, MIX, ORC_HIDDEN, 2048, T, f64);
    free(q); free(k); free(v); free(g); free(beta); free(core); free(init); free(Gt);
  }
  free(QKV); free(Z); free(A); free(B);
}

/* Runs T tokens (rows of H, fp16 [T][1024]) through every layer in place. */
static void forward_layers(const OrcModel* m, OrcModelState* st, uint16_t* H, int32_t T) {
  const int32_t p0 = st->pos;
  uint16_t* XN = (uint16_t*)malloc(2 * (size_t)T * ORC_HIDDEN);
  uint16_t* MIX = (uint16_t*)malloc(2 * (size_t)T * ORC_HIDDEN);
  uint16_t* GA = (uint16_t*)malloc(2 * (size_t)T * ORC_INTER);
  uint16_t* UP = (uint16_t*)malloc(2 * (size_t)T * ORC_INTER);
  const int f64 = g_gemm_f64 && T > 1;
  for (int32_t L = 0; L < m->n_layers; ++L) {
    const OrcLayer* ly = &m->layers[L];
    for (int32_t t = 0; t < T; ++t)
      orc_rmsnorm1024(H + (size_t)t * ORC_HIDDEN, ly->input_norm, XN + (size_t)t * ORC_HIDDEN);
    if (ly->kind == 0)
      dn_mixer(m, st, ly, XN, T, MIX);
    else
      attn_mixer(m, st, ly, XN, T, p0, MIX);
    for (int32_t t = 0; t < T; ++t) {
      uint16_t* h = H + (size_t)t * ORC_HIDDEN;
      orc_residual_add(h, MIX + (size_t)t * ORC_HIDDEN, h, ORC_HIDDEN);
      orc_rmsnorm1024(h, ly->post_norm, XN + (size_t)t * ORC_HIDDEN);
    }
    matmul_impl(ly->mlp_gate, XN, GA, ORC_INTER, ORC_HIDDEN, T, f64);
    matmul_impl(ly->mlp_up, XN, UP, ORC_INTER, ORC_HIDDEN, T, f64);
    for (int32_t t = 0; t < T; ++t)
      orc_silu_gate(GA + (size_t)t * ORC_INTER, UP + (size_t)t * ORC_INTER, GA + (size_t)t * ORC_INTER, ORC_INTER);
    matmul_impl(ly->mlp_down, GA, MIX, ORC_HIDDEN, ORC_INTER, T, f64);
    for (int32_t t = 0; t < T; ++t)
      orc_residual_add(H + (size_t)t * ORC_HIDDEN, MIX + (size_t)t * ORC_HIDDEN, H + (size_t)t * ORC_HIDDEN,
                       ORC_HIDDEN);
  }
  free(XN); free(MIX); free(GA); free(UP);
  st->pos += T;
}

static uint32_t head_out(const OrcModel* m, const uint16_t* h, uint16_t* logits, uint16_t* hidden) {
  uint16_t hn[ORC_HIDDEN];
  if (hidden) memcpy(hidden, h, 2 * ORC_HIDDEN);
  orc_rmsnorm1024(h, m->final_norm, hn);
  uint16_t* lg = logits ? logits : (uint16_t*)malloc(2 * (size_t)m->vocab);
  matmul_impl(m->embed, hn, lg, (size_t)m->vocab, ORC_HIDDEN, 1, 0);
  const uint32_t idx = orc_argmax_f16(lg, (size_t)m->vocab);
  if (!logits) free(lg);
  return idx;
}

uint32_t orc_model_prefill(const OrcModel* m, OrcModelState* st, const int32_t* tokens, int32_t T,
                           uint16_t* last_logits, uint16_t* last_hidden) {
  if (T <= 0 || st->pos + T > m->max_seq) {
    fprintf(stderr, "orc_model_prefill: %d tokens at position %d exceed max_seq %d\n", T, st->pos, m->max_seq);
    abort();
  }
  uint16_t* H = (uint16_t*)malloc(2 * (size_t)T * ORC_HIDDEN);
  for (int32_t t = 0; t < T; ++t)  /* embedding_lookup.comp */
    memcpy(H + (size_t)t * ORC_HIDDEN, m->embed + (size_t)tokens[t] * ORC_HIDDEN, 2 * ORC_HIDDEN);
  forward_layers(m, st, H, T);
  const uint32_t idx = head_out(m, H + (size_t)(T - 1) * ORC_HIDDEN, last_logits, last_hidden);
  free(H);
  return idx;
}

uint32_t orc_model_decode(const OrcModel* m, OrcModelState* st, int32_t token, uint16_t* logits,
                          uint16_t* hidden) {
  if (st->pos + 1 > m->max_seq) {
    fprintf(stderr, "orc_model_decode: position %d exceeds max_seq %d\n", st->pos, m->max_seq);
    abort();
  }
  uint16_t h[ORC_HIDDEN];
  memcpy(h, m->embed + (size_t)token * ORC_HIDDEN, 2 * ORC_HIDDEN);
  forward_layers(m, st, h, 1);
  return head_out(m, h, logits, hidden);
}

void orc_model_generate(const OrcModel* m, OrcModelState* st, const int32_t* prompt, int32_t T,
                        int32_t n_new, int32_t* out) {
  if (n_new <= 0) return;
  uint32_t tok = orc_model_prefill(m, st, prompt, T, NULL, NULL);
  out[0] = (int32_t)tok;
  for (int32_t i = 1; i < n_new; ++i) {
    tok = orc_model_decode(m, st, (int32_t)tok, NULL, NULL);
    out[i] = (int32_t)tok;
  }
}
