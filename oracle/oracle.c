/*
 * oracle.c -- CPU restatement of the Spock hot path.  TEST INFRASTRUCTURE ONLY
 * (see oracle.h for who may load it and how each function is pinned).
 *
 * Build: -O2 -ffp-contract=off so that every a*b+c below rounds twice unless
 * fmaf() is written explicitly; the GPU kernels in spock_amd/csrc are built the
 * same way and follow the same operation order where bit-exactness is claimed
 * (decode step, matvec, lm_head, argmax).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* fp16 helpers                                                              */
/* ------------------------------------------------------------------------ */

static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Exact half -> float, subnormals included (vk_session.cpp:28-55). */
float orc_h2f(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) & 1u;
  uint32_t exponent = (uint32_t)(h >> 10) & 0x1fu;
  uint32_t mantissa = (uint32_t)h & 0x3ffu;
  uint32_t f;
  if (exponent == 0) {
    if (mantissa == 0) {
      f = sign << 31;
    } else {
      /* normalise the subnormal: value = mantissa * 2^-24 */
      int e = -14;
      while ((mantissa & 0x400u) == 0) { mantissa <<= 1; e -= 1; }
      mantissa &= 0x3ffu;
      f = (sign << 31) | ((uint32_t)(e + 127) << 23) | (mantissa << 13);
    }
  } else if (exponent == 31) {
    f = (sign << 31) | (0xffu << 23) | (mantissa << 13);
  } else {
    f = (sign << 31) | ((exponent + 127 - 15) << 23) | (mantissa << 13);
  }
  return bits_f(f);
}

/* IEEE float -> half, round to nearest even, with fp16 subnormals, overflow to
 * inf and NaN kept quiet.  This is what a GLSL float16_t(x) conversion does on
 * AMD hardware (v_cvt_f16_f32) and what the reference repacker's
 * fp32_to_fp16_bits (apps/spock-repack-text.cpp:62-89) aims at. */
uint16_t orc_f2h_rne(float f) {
  uint32_t x = f_bits(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) {                     /* inf or NaN */
    if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
  }
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
  if (ax < 0x38800000u) {                      /* below 2^-14: fp16 subnormal */
    /* value = ax as float; q = round(value * 2^24) */
    if (ax < 0x33000000u) {                    /* < 2^-25: rounds to 0 ... */
      return (uint16_t)sign;                   /* (2^-25 exactly ties to 0) */
    }
    uint32_t e = ax >> 23;                     /* biased exp, 102..112 */
    uint32_t m = (ax & 0x7fffffu) | 0x800000u; /* 24-bit significand */
    uint32_t shift = 126u - e;                 /* value*2^24 = m * 2^(e-150+24) */
    /* q = m >> (126 - e) with RNE */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
  }
  /* normal range */
  uint32_t e = (ax >> 23) - 127u + 15u;
  uint32_t m = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u; /* may carry into exp */
  return (uint16_t)(sign | h);
}

/* Truncating float -> half with flush to zero (vk_session.cpp:69-89,
 * deltanet_chunk_last_to_fp16.comp:45-74). */
uint16_t orc_f2h_trunc(float f) {
  uint32_t bits = f_bits(f);
  uint32_t sign = (bits >> 31) & 1u;
  uint32_t exponent = (bits >> 23) & 0xffu;
  uint32_t mantissa = bits & 0x7fffffu;
  uint16_t h_sign = (uint16_t)(sign << 15);
  if (exponent == 0) return h_sign;
  if (exponent == 0xff) return (uint16_t)(h_sign | 0x7c00u | (mantissa ? 0x200u : 0u));
  int32_t new_exp = (int32_t)exponent - 127 + 15;
  if (new_exp <= 0) return h_sign;
  if (new_exp >= 31) return (uint16_t)(h_sign | 0x7c00u);
  return (uint16_t)(h_sign | ((uint32_t)new_exp << 10) | (mantissa >> 13));
}

void orc_h2f_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_h2f(in[i]);
}
void orc_f2h_rne_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_f2h_rne(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Deterministic exp / log.                                                 */
/*                                                                          */
/* The reference uses GLSL exp/log (driver-defined accuracy) and std::exp.  */
/* For bit-exact GPU/CPU agreement both sides evaluate the same IEEE        */
/* operation sequence: Cody-Waite reduction by ln2 split in two parts, then */
/* the Taylor polynomial of e^r to degree 7 (|r| <= ln2/2, truncation error */
/* below 4e-9 relative) and an exact ldexp.  log uses m in [sqrt(1/2),      */
/* sqrt(2)), s = (m-1)/(m+1) and log(m) = 2 atanh(s) to s^11.               */
/* ------------------------------------------------------------------------ */

#define ORC_LN2_HI 0.693145751953125f          /* 0x3F317200, 15 significant bits */
#define ORC_LN2_LO 1.42860677e-06f             /* ln2 - ln2_hi */
#define ORC_LOG2E 1.44269504f

float orc_expf(float x) {
  if (x != x) return x;
  if (x > 88.7228394f) return INFINITY;
  if (x < -103.972084f) return 0.0f;
  float t = x * ORC_LOG2E;
  float kf = rintf(t);
  float r = fmaf(-kf, ORC_LN2_HI, x);
  r = fmaf(-kf, ORC_LN2_LO, r);
  float p = 1.98412698e-4f;            /* 1/7! */
  p = fmaf(p, r, 1.38888889e-3f);      /* 1/6! */
  p = fmaf(p, r, 8.33333333e-3f);      /* 1/5! */
  p = fmaf(p, r, 4.16666667e-2f);      /* 1/4! */
  p = fmaf(p, r, 1.66666667e-1f);      /* 1/3! */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)kf);
}

float orc_logf(float x) {
  if (x != x) return x;
  if (x < 0.0f) return NAN;
  if (x == 0.0f) return -INFINITY;
  if (x == INFINITY) return x;
  int e;
  float m = frexpf(x, &e);             /* x = m 2^e, m in [0.5, 1) */
  if (m < 0.707106781f) { m = m * 2.0f; e -= 1; }
  float s = (m - 1.0f) / (m + 1.0f);
  float s2 = s * s;
  float p = 9.09090909e-2f;            /* 1/11 */
  p = fmaf(p, s2, 1.11111111e-1f);     /* 1/9 */
  p = fmaf(p, s2, 1.42857143e-1f);     /* 1/7 */
  p = fmaf(p, s2, 2.0e-1f);            /* 1/5 */
  p = fmaf(p, s2, 3.33333333e-1f);     /* 1/3 */
  float ls = 2.0f * s;
  float lm = fmaf(ls * s2, p, ls);
  float ef = (float)e;
  return fmaf(ef, ORC_LN2_HI, fmaf(ef, ORC_LN2_LO, lm));
}

/* 1/sqrt(x) as two correctly rounded IEEE operations. */
float orc_rsqrtf(float x) { return 1.0f / sqrtf(x); }

void orc_expf_array(const float* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_expf(in[i]);
}
void orc_logf_array(const float* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = orc_logf(in[i]);
}

/* ------------------------------------------------------------------------ */
/* Chunk rule: deltanet_chunk.cpp:53-284, same loop nests and operation     */
/* order; std::exp(float) is exp_fn: the C library's expf reproduces the    */
/* compiled reference bit for bit under -ffp-contract=off, orc_expf gives   */
/* the variant the GPU evaluates identically.                               */
/* ------------------------------------------------------------------------ */

static inline size_t qkv_index(size_t head, size_t token, size_t dim, size_t seq, size_t width) {
  return ((head * seq) + token) * width + dim;
}

/* deltanet_chunk.cpp:27-39 */
static void l2_norm_token(float* values, size_t head, size_t token, size_t seq, size_t width) {
  const float eps = 1e-6f;
  float ss = 0.0f;
  for (size_t d = 0; d < width; ++d) {
    const float x = values[qkv_index(head, token, d, seq, width)];
    ss += x * x;
  }
  const float inv_norm = 1.0f / sqrtf(ss + eps);
  for (size_t d = 0; d < width; ++d) values[qkv_index(head, token, d, seq, width)] *= inv_norm;
}

static int chunk_rule_impl(size_t heads, size_t seq, size_t k_dim, size_t v_dim, size_t chunk,
                           int use_qk_l2norm, const float* q_in, const float* k_in,
                           const float* v_in, const float* g_in, const float* beta_in,
                           const float* init, float* out_core, float* out_state,
                           float (*exp_fn)(float)) {
  if (heads == 0 || seq == 0 || k_dim == 0 || v_dim == 0 || chunk == 0) return -1;

  float* query = (float*)malloc(heads * seq * k_dim * sizeof(float));
  float* key = (float*)malloc(heads * seq * k_dim * sizeof(float));
  memcpy(query, q_in, heads * seq * k_dim * sizeof(float));
  memcpy(key, k_in, heads * seq * k_dim * sizeof(float));
  float* state = out_state;
  if (init) memcpy(state, init, heads * k_dim * v_dim * sizeof(float));
  else memset(state, 0, heads * k_dim * v_dim * sizeof(float));

  /* :78-85 */
  if (use_qk_l2norm) {
    for (size_t h = 0; h < heads; ++h)
      for (size_t t = 0; t < seq; ++t) {
        l2_norm_token(query, h, t, seq, k_dim);
        l2_norm_token(key, h, t, seq, k_dim);
      }
  }
  /* :87-88 */
  const float q_scale = 1.0f / sqrtf((float)k_dim);
  for (size_t i = 0; i < heads * seq * k_dim; ++i) query[i] *= q_scale;

  /* :90-113 zero padding to a multiple of the chunk */
  const size_t pad = (chunk - (seq % chunk)) % chunk;
  const size_t total = seq + pad;
  float* qp = (float*)calloc(heads * total * k_dim, sizeof(float));
  float* kp = (float*)calloc(heads * total * k_dim, sizeof(float));
  float* vp = (float*)calloc(heads * total * v_dim, sizeof(float));
  float* gp = (float*)calloc(heads * total, sizeof(float));
  float* bp = (float*)calloc(heads * total, sizeof(float));
  for (size_t h = 0; h < heads; ++h)
    for (size_t t = 0; t < seq; ++t) {
      memcpy(&qp[qkv_index(h, t, 0, total, k_dim)], &query[qkv_index(h, t, 0, seq, k_dim)], k_dim * 4);
      memcpy(&kp[qkv_index(h, t, 0, total, k_dim)], &key[qkv_index(h, t, 0, seq, k_dim)], k_dim * 4);
      memcpy(&vp[qkv_index(h, t, 0, total, v_dim)], &v_in[qkv_index(h, t, 0, seq, v_dim)], v_dim * 4);
      gp[h * total + t] = g_in[h * seq + t];
      bp[h * total + t] = beta_in[h * seq + t];
    }

  float* core = (float*)calloc(heads * total * v_dim, sizeof(float));
  const size_t nchunks = total / chunk;
  float* decay = (float*)malloc(chunk * chunk * 4);
  float* attn = (float*)malloc(chunk * chunk * 4);
  float* solved = (float*)malloc(chunk * v_dim * 4);
  float* kcd = (float*)malloc(chunk * k_dim * 4);
  float* qc = (float*)malloc(chunk * k_dim * 4);
  float* kc = (float*)malloc(chunk * k_dim * 4);
  float* vc = (float*)malloc(chunk * v_dim * 4);
  float* gcum = (float*)malloc(chunk * 4);
  float* bc = (float*)malloc(chunk * 4);
  float* wstate = (float*)malloc(k_dim * v_dim * 4);
  float* local = (float*)malloc(chunk * chunk * 4);
  float* vnew = (float*)malloc(chunk * v_dim * 4);
  float* inter = (float*)malloc(chunk * v_dim * 4);
  float* upd = (float*)malloc(k_dim * v_dim * 4);
  float* old_row = (float*)malloc(chunk * 4);

  for (size_t h = 0; h < heads; ++h) {
    float* S = state + h * k_dim * v_dim;
    for (size_t ci = 0; ci < nchunks; ++ci) {
      const size_t base = ci * chunk;
      float running = 0.0f;                                   /* :137-151 */
      for (size_t t = 0; t < chunk; ++t) {
        gcum[t] = running + gp[h * total + base + t];
        running = gcum[t];
        bc[t] = bp[h * total + base + t];
        memcpy(&qc[t * k_dim], &qp[qkv_index(h, base + t, 0, total, k_dim)], k_dim * 4);
        memcpy(&kc[t * k_dim], &kp[qkv_index(h, base + t, 0, total, k_dim)], k_dim * 4);
        memcpy(&vc[t * v_dim], &vp[qkv_index(h, base + t, 0, total, v_dim)], v_dim * 4);
      }
      memset(decay, 0, chunk * chunk * 4);                    /* :153-159 */
      memset(attn, 0, chunk * chunk * 4);
      for (size_t r = 0; r < chunk; ++r)
        for (size_t c = 0; c <= r; ++c) decay[r * chunk + c] = exp_fn(gcum[r] - gcum[c]);
      for (size_t r = 0; r < chunk; ++r)                      /* :161-170 */
        for (size_t c = 0; c < r; ++c) {
          float dot = 0.0f;
          for (size_t d = 0; d < k_dim; ++d) dot += (kc[r * k_dim + d] * bc[r]) * kc[c * k_dim + d];
          attn[r * chunk + c] = -dot * decay[r * chunk + c];
        }
      for (size_t r = 1; r < chunk; ++r) {                    /* :171-181 */
        for (size_t c = 0; c < r; ++c) old_row[c] = attn[r * chunk + c];
        for (size_t c = 0; c < r; ++c) {
          float sum = old_row[c];
          for (size_t in = 0; in < r; ++in) sum += old_row[in] * attn[in * chunk + c];
          attn[r * chunk + c] = sum;
        }
      }
      for (size_t d = 0; d < chunk; ++d) attn[d * chunk + d] += 1.0f; /* :182-184 */

      memset(solved, 0, chunk * v_dim * 4);                   /* :186-202 */
      memset(kcd, 0, chunk * k_dim * 4);
      for (size_t r = 0; r < chunk; ++r)
        for (size_t c = 0; c < chunk; ++c) {
          const float coeff = attn[r * chunk + c];
          if (coeff == 0.0f) continue;
          const float bcol = bc[c];
          const float egc = exp_fn(gcum[c]);
          for (size_t vd = 0; vd < v_dim; ++vd) solved[r * v_dim + vd] += coeff * (vc[c * v_dim + vd] * bcol);
          for (size_t kd = 0; kd < k_dim; ++kd) kcd[r * k_dim + kd] += coeff * (kc[c * k_dim + kd] * bcol * egc);
        }
      memset(local, 0, chunk * chunk * 4);                    /* :204-213 */
      for (size_t r = 0; r < chunk; ++r)
        for (size_t c = 0; c <= r; ++c) {
          float dot = 0.0f;
          for (size_t d = 0; d < k_dim; ++d) dot += qc[r * k_dim + d] * kc[c * k_dim + d];
          local[r * chunk + c] = dot * decay[r * chunk + c];
        }
      for (size_t r = 0; r < chunk; ++r) {                    /* :215-233 */
        const float egr = exp_fn(gcum[r]);
        for (size_t vd = 0; vd < v_dim; ++vd) {
          float carry = 0.0f, it = 0.0f;
          for (size_t kd = 0; kd < k_dim; ++kd) {
            carry += kcd[r * k_dim + kd] * S[kd * v_dim + vd];
            it += (qc[r * k_dim + kd] * egr) * S[kd * v_dim + vd];
          }
          vnew[r * v_dim + vd] = solved[r * v_dim + vd] - carry;
          inter[r * v_dim + vd] = it;
        }
      }
      for (size_t r = 0; r < chunk; ++r)                      /* :235-244 */
        for (size_t vd = 0; vd < v_dim; ++vd) {
          float sum = inter[r * v_dim + vd];
          for (size_t c = 0; c <= r; ++c) sum += local[r * chunk + c] * vnew[c * v_dim + vd];
          core[qkv_index(h, base + r, vd, total, v_dim)] = sum;
        }
      const float eglast = exp_fn(gcum[chunk - 1]);             /* :246-268 */
      for (size_t i = 0; i < k_dim * v_dim; ++i) wstate[i] = S[i] * eglast;
      memset(upd, 0, k_dim * v_dim * 4);
      for (size_t r = 0; r < chunk; ++r) {
        const float w = exp_fn(gcum[chunk - 1] - gcum[r]);
        for (size_t kd = 0; kd < k_dim; ++kd) {
          const float sk = kc[r * k_dim + kd] * w;
          for (size_t vd = 0; vd < v_dim; ++vd) upd[kd * v_dim + vd] += sk * vnew[r * v_dim + vd];
        }
      }
      for (size_t i = 0; i < k_dim * v_dim; ++i) S[i] = wstate[i] + upd[i];
    }
  }
  for (size_t h = 0; h < heads; ++h)                          /* :272-283 trim */
    for (size_t t = 0; t < seq; ++t)
      memcpy(&out_core[qkv_index(h, t, 0, seq, v_dim)], &core[qkv_index(h, t, 0, total, v_dim)], v_dim * 4);

  free(query); free(key); free(qp); free(kp); free(vp); free(gp); free(bp); free(core);
  free(decay); free(attn); free(solved); free(kcd); free(qc); free(kc); free(vc); free(gcum);
  free(bc); free(wstate); free(local); free(vnew); free(inter); free(upd); free(old_row);
  return 0;
}

int orc_chunk_rule(size_t heads, size_t seq, size_t k_dim, size_t v_dim, size_t chunk,
                   int use_qk_l2norm, const float* q_in, const float* k_in,
                   const float* v_in, const float* g_in, const float* beta_in,
                   const float* init, float* out_core, float* out_state) {
  return chunk_rule_impl(heads, seq, k_dim, v_dim, chunk, use_qk_l2norm, q_in, k_in, v_in, g_in,
                         beta_in, init, out_core, out_state, expf);
}

/* The same loops with orc_expf in place of the C library's expf. */
int orc_chunk_rule_det(size_t heads, size_t seq, size_t k_dim, size_t v_dim, size_t chunk,
                       int use_qk_l2norm, const float* q_in, const float* k_in,
                       const float* v_in, const float* g_in, const float* beta_in,
                       const float* init, float* out_core, float* out_state) {
  return chunk_rule_impl(heads, seq, k_dim, v_dim, chunk, use_qk_l2norm, q_in, k_in, v_in, g_in,
                         beta_in, init, out_core, out_state, orc_expf);
}

int orc_chunk_rule_varlen(size_t H, size_t N, size_t dk, size_t dv, size_t C,
                          int use_qk_l2norm, const int32_t* cu, size_t S,
                          const float* q, const float* k, const float* v,
                          const float* g, const float* beta, const float* init,
                          float* out_core, float* out_state) {
  if (cu[0] != 0 || (size_t)cu[S] != N) return -2;
  for (size_t s = 0; s < S; ++s) {
    const size_t t0 = (size_t)cu[s];
    const size_t L = (size_t)(cu[s + 1] - cu[s]);
    if (L == 0) {                       /* empty sequence: state passes through */
      float* st = out_state + s * H * dk * dv;
      if (init) memcpy(st, init + s * H * dk * dv, H * dk * dv * 4);
      else memset(st, 0, H * dk * dv * 4);
      continue;
    }
    float* qs = (float*)malloc(H * L * dk * 4);
    float* ks = (float*)malloc(H * L * dk * 4);
    float* vs = (float*)malloc(H * L * dv * 4);
    float* gs = (float*)malloc(H * L * 4);
    float* bs = (float*)malloc(H * L * 4);
    float* os = (float*)malloc(H * L * dv * 4);
    for (size_t h = 0; h < H; ++h) {
      memcpy(qs + h * L * dk, q + (h * N + t0) * dk, L * dk * 4);
      memcpy(ks + h * L * dk, k + (h * N + t0) * dk, L * dk * 4);
      memcpy(vs + h * L * dv, v + (h * N + t0) * dv, L * dv * 4);
      memcpy(gs + h * L, g + h * N + t0, L * 4);
      memcpy(bs + h * L, beta + h * N + t0, L * 4);
    }
    int rc = orc_chunk_rule(H, L, dk, dv, C, use_qk_l2norm, qs, ks, vs, gs, bs,
                            init ? init + s * H * dk * dv : NULL, os,
                            out_state + s * H * dk * dv);
    for (size_t h = 0; h < H; ++h) memcpy(out_core + (h * N + t0) * dv, os + h * L * dv, L * dv * 4);
    free(qs); free(ks); free(vs); free(gs); free(bs); free(os);
    if (rc) return rc;
  }
  return 0;
}

void orc_delta_recurrence_f64(size_t H, size_t T, size_t dk, size_t dv, int l2,
                              const double* q, const double* k, const double* v,
                              const double* g, const double* beta, const double* init,
                              double* out_core, double* out_state) {
  const double scale = 1.0 / sqrt((double)dk);
  double* qn = (double*)malloc(dk * sizeof(double));
  double* kn = (double*)malloc(dk * sizeof(double));
  double* kv = (double*)malloc(dv * sizeof(double));
  for (size_t h = 0; h < H; ++h) {
    double* S = out_state + h * dk * dv;
    if (init) memcpy(S, init + h * dk * dv, dk * dv * sizeof(double));
    else memset(S, 0, dk * dv * sizeof(double));
    for (size_t t = 0; t < T; ++t) {
      const double* qt = q + (h * T + t) * dk;
      const double* kt = k + (h * T + t) * dk;
      const double* vt = v + (h * T + t) * dv;
      double nq = 1.0, nk = 1.0;
      if (l2) {
        double sq = 0, sk = 0;
        for (size_t d = 0; d < dk; ++d) { sq += qt[d] * qt[d]; sk += kt[d] * kt[d]; }
        nq = 1.0 / sqrt(sq + 1e-6); nk = 1.0 / sqrt(sk + 1e-6);
      }
      for (size_t d = 0; d < dk; ++d) { qn[d] = qt[d] * nq * scale; kn[d] = kt[d] * nk; }
      const double eg = exp(g[h * T + t]);
      for (size_t i = 0; i < dk * dv; ++i) S[i] *= eg;
      for (size_t j = 0; j < dv; ++j) {
        double acc = 0;
        for (size_t i = 0; i < dk; ++i) acc += S[i * dv + j] * kn[i];
        kv[j] = (vt[j] - acc) * beta[h * T + t];
      }
      for (size_t i = 0; i < dk; ++i)
        for (size_t j = 0; j < dv; ++j) S[i * dv + j] += kn[i] * kv[j];
      for (size_t j = 0; j < dv; ++j) {
        double acc = 0;
        for (size_t i = 0; i < dk; ++i) acc += S[i * dv + j] * qn[i];
        out_core[(h * T + t) * dv + j] = acc;
      }
    }
  }
  free(qn); free(kn); free(kv);
}

/* ------------------------------------------------------------------------ */
/* Collect / last-token hand-off                                            */
/* ------------------------------------------------------------------------ */

void orc_prefill_collect(size_t H, size_t T, size_t tok, size_t dk, size_t dv,
                         const uint16_t* qkv, const float* gb, float* qo, float* ko,
                         float* vo, float* go, float* bo) {
  for (size_t h = 0; h < H; ++h) {
    for (size_t d = 0; d < dk; ++d) {
      qo[(h * T + tok) * dk + d] = orc_h2f(qkv[h * dk + d]);
      ko[(h * T + tok) * dk + d] = orc_h2f(qkv[H * dk + h * dk + d]);
    }
    for (size_t d = 0; d < dv; ++d) vo[(h * T + tok) * dv + d] = orc_h2f(qkv[2 * H * dk + h * dv + d]);
    go[h * T + tok] = gb[h];
    bo[h * T + tok] = gb[H + h];
  }
}

void orc_chunk_last_to_fp16(size_t H, size_t dv, size_t T, size_t total, const float* src,
                            uint16_t* dst) {
  for (size_t h = 0; h < H; ++h)
    for (size_t d = 0; d < dv; ++d) dst[h * dv + d] = orc_f2h_trunc(src[(h * total + T - 1) * dv + d]);
}

/* ------------------------------------------------------------------------ */
/* Decode step.  The arithmetic is the reference shaders'; where a shader    */
/* leaves the order of a reduction to one thread's loop, the order below is */
/* the one the HIP kernel uses (stated at each site) so the two agree       */
/* bit for bit.                                                              */
/* ------------------------------------------------------------------------ */

/* 128-wide pairwise tree: s[l] += s[l+stride] for stride 64,32,...,1
 * (deltanet_conv_l2_qk.comp:97-103, deltanet_recurrent_gbeta_norm_gate.comp:313-318) */
static float tree128(float* s) {
  for (size_t stride = 64; stride > 0; stride >>= 1)
    for (size_t l = 0; l < stride; ++l) s[l] = s[l] + s[l + stride];
  return s[0];
}

static inline float silu_f(float x) { return x / (1.0f + orc_expf(-x)); }

void orc_conv_l2_qk(size_t conv_dim, size_t ks, size_t key_total, size_t num_heads,
                    uint16_t* qkv, uint16_t* cs, const uint16_t* w) {
  (void)key_total;
  /* phase 1: shift left, insert (conv_l2_qk.comp:48-58) */
  for (size_t ch = 0; ch < conv_dim; ++ch) {
    for (size_t i = 0; i + 1 < ks; ++i) cs[ch * ks + i] = cs[ch * ks + i + 1];
    cs[ch * ks + ks - 1] = qkv[ch];
  }
  /* phase 2: depthwise conv + SiLU, taps summed in order i = 0..ks-1 (:62-75).
   * Each product of two halves is exact in fp32. */
  for (size_t ch = 0; ch < conv_dim; ++ch) {
    float sum = 0.0f;
    for (size_t i = 0; i < ks; ++i) sum = sum + orc_h2f(cs[ch * ks + i]) * orc_h2f(w[ch * ks + i]);
    qkv[ch] = orc_f2h_rne(silu_f(sum));
  }
  /* phase 3: L2 of each Q and K head block (:79-110) */
  float s[128];
  for (size_t blk = 0; blk < 2 * num_heads; ++blk) {
    uint16_t* y = qkv + blk * 128;
    for (size_t l = 0; l < 128; ++l) { float t = orc_h2f(y[l]); s[l] = t * t; }
    const float inv = orc_rsqrtf(tree128(s) + 1e-6f);
    for (size_t l = 0; l < 128; ++l) y[l] = orc_f2h_rne(orc_h2f(y[l]) * inv);
  }
}

/* Column reduction used by the HIP decode kernel: rows split in 32 contiguous
 * groups of 4, fma-accumulated from 0 in row order, then a balanced pairwise
 * tree over the 32 partials, adjacent pairs first. */
static float col_dot128(const float* S, size_t j, const float* x) {
  float p[32];
  for (size_t gi = 0; gi < 32; ++gi) {
    float acc = 0.0f;
    for (size_t i = gi * 4; i < gi * 4 + 4; ++i) acc = fmaf(S[i * 128 + j], x[i], acc);
    p[gi] = acc;
  }
  for (size_t n = 32; n > 1; n >>= 1)
    for (size_t i = 0; i < n / 2; ++i) p[i] = p[2 * i] + p[2 * i + 1];
  return p[0];
}

/* One head of the recurrence (deltanet_recurrent_gbeta_norm_gate.comp:243-291):
 * decay, kv_mem = S^T k, delta, rank-1 update (fma), o = S^T q. */
static void recur_head(float* S, const float* qf, const float* kf, const float* vf,
                       float g, float beta, float* o) {
  const float eg = orc_expf(g);
  float kv[128], delta[128];
  for (size_t i = 0; i < 128 * 128; ++i) S[i] = S[i] * eg;
  for (size_t j = 0; j < 128; ++j) kv[j] = col_dot128(S, j, kf);
  for (size_t j = 0; j < 128; ++j) delta[j] = (vf[j] - kv[j]) * beta;
  for (size_t i = 0; i < 128; ++i)
    for (size_t j = 0; j < 128; ++j) S[i * 128 + j] = fmaf(kf[i], delta[j], S[i * 128 + j]);
  for (size_t j = 0; j < 128; ++j) o[j] = col_dot128(S, j, qf);
}

/* g and beta of one head (deltanet_recurrent_gbeta_norm_gate.comp:102-116):
 * g = -exp(A_log) * log(1 + exp(a + dt_bias)) (softplus with no overflow
 * threshold), beta = 1 / (1 + exp(-b)). */
void orc_gbeta(float a, float b, float a_log, float dt_bias, float* g, float* beta) {
  const float sp = orc_logf(1.0f + orc_expf(a + dt_bias));
  *g = -orc_expf(a_log) * sp;
  *beta = 1.0f / (1.0f + orc_expf(-b));
}

/* Gated RMSNorm of one 128-wide head row o (fp32):
 * r = 1/sqrt(tree128(o^2)/128 + eps), out = fp16(fp16(w * (o*r)) * silu(z))
 * (deltanet_recurrent_gbeta_norm_gate.comp:182-224, deltanet_norm_gate.comp:80-105). */
void orc_norm_gate_row(const float* o, const uint16_t* z, const float* nw, float eps,
                       uint16_t* out) {
  float s[128];
  for (size_t l = 0; l < 128; ++l) s[l] = o[l] * o[l];
  const float r = orc_rsqrtf(tree128(s) / 128.0f + eps);
  for (size_t l = 0; l < 128; ++l) {
    const float normed = o[l] * r;
    const float weighted = orc_h2f(orc_f2h_rne(nw[l] * normed));
    out[l] = orc_f2h_rne(weighted * silu_f(orc_h2f(z[l])));
  }
}

/* deltanet_norm_gate.comp:80-105, the unfused norm-gate over fp16 input rows
 * (dispatch vk_session.cpp:1743-1756, :3245-3257): io [nh][128] in place.
 * The shader's 256-lane tree adds 128 zero partials at its first level
 * (exact), so the sum is tree128 of the squares. */
void orc_norm_gate_f16(size_t nh, float eps, uint16_t* io, const uint16_t* z,
                       const float* nw) {
  float o[128];
  for (size_t h = 0; h < nh; ++h) {
    for (size_t l = 0; l < 128; ++l) o[l] = orc_h2f(io[h * 128 + l]);
    orc_norm_gate_row(o, z + h * 128, nw, eps, io + h * 128);
  }
}

void orc_recurrent_gbeta_norm_gate(size_t nh, size_t layer, float q_scale, float eps,
                                   const uint16_t* a, const uint16_t* b,
                                   const float* alb, uint16_t* qkv, float* state,
                                   const uint16_t* z, const float* nw) {
  float qf[128], kf[128], vf[128], o[128];
  for (size_t h = 0; h < nh; ++h) {
    float g, beta;
    orc_gbeta(orc_h2f(a[h]), orc_h2f(b[h]), alb[(layer * nh + h) * 2],
              alb[(layer * nh + h) * 2 + 1], &g, &beta);
    /* :233-241 */
    for (size_t l = 0; l < 128; ++l) {
      qf[l] = orc_h2f(qkv[h * 128 + l]) * q_scale;
      kf[l] = orc_h2f(qkv[nh * 128 + h * 128 + l]);
      vf[l] = orc_h2f(qkv[2 * nh * 128 + h * 128 + l]);
    }
    recur_head(state + h * 128 * 128, qf, kf, vf, g, beta, o);
    orc_norm_gate_row(o, z + h * 128, nw, eps, qkv + 2 * nh * 128 + h * 128);
  }
}

void orc_recurrent(size_t nh, float q_scale, uint16_t* qkv, float* state) {
  float qf[128], kf[128], vf[128], o[128];
  const size_t tail = nh * 128 * 128;
  for (size_t h = 0; h < nh; ++h) {
    for (size_t l = 0; l < 128; ++l) {
      qf[l] = orc_h2f(qkv[h * 128 + l]) * q_scale;
      kf[l] = orc_h2f(qkv[nh * 128 + h * 128 + l]);
      vf[l] = orc_h2f(qkv[2 * nh * 128 + h * 128 + l]);
    }
    recur_head(state + h * 128 * 128, qf, kf, vf, state[tail + h], state[tail + nh + h], o);
    for (size_t l = 0; l < 128; ++l) qkv[2 * nh * 128 + h * 128 + l] = orc_f2h_rne(o[l]);
  }
}

void orc_decode_step(size_t B, size_t nh, size_t layer, float q_scale, float eps,
                     uint16_t* qkv, size_t qkv_stride, uint16_t* cs, size_t cs_stride,
                     const uint16_t* cw, const uint16_t* a, const uint16_t* b,
                     size_t ab_stride, const float* alb, float* state, size_t st_stride,
                     const uint16_t* z, size_t z_stride, const float* nw) {
  const size_t conv_dim = 3 * nh * 128;
  for (size_t s = 0; s < B; ++s) {
    orc_conv_l2_qk(conv_dim, 4, nh * 128, nh, qkv + s * qkv_stride, cs + s * cs_stride, cw);
    orc_recurrent_gbeta_norm_gate(nh, layer, q_scale, eps, a + s * ab_stride, b + s * ab_stride,
                                  alb, qkv + s * qkv_stride, state + s * st_stride,
                                  z + s * z_stride, nw);
  }
}

/* ------------------------------------------------------------------------ */
/* matvec / lm_head / argmax                                                 */
/* ------------------------------------------------------------------------ */

int orc_matvec_f16(const uint16_t* W, const uint16_t* x, uint16_t* y, size_t out_dim,
                   size_t in_dim) {
  if (in_dim % 64 != 0) return -1;
  const size_t span = in_dim / 64;
  float* xf = (float*)malloc(in_dim * 4);
  orc_h2f_array(x, xf, in_dim);
  float part[64];
  for (size_t r = 0; r < out_dim; ++r) {
    const uint16_t* row = W + r * in_dim;
    for (size_t l = 0; l < 64; ++l) {
      float acc = 0.0f;
      for (size_t j = l * span; j < (l + 1) * span; ++j) acc = fmaf(orc_h2f(row[j]), xf[j], acc);
      part[l] = acc;
    }
    for (size_t stride = 32; stride > 0; stride >>= 1)
      for (size_t l = 0; l < stride; ++l) part[l] = part[l] + part[l + stride];
    y[r] = orc_f2h_rne(part[0]);
  }
  free(xf);
  return 0;
}

/* matvec_tiled.comp:41-84: lane l of 64 sums j = l, l+64, ... < in_dim
 * (:54-58, fp32 from 0), then s[l] += s[l+stride] for stride 32..1 (:66-73),
 * fp16 store (:80).  Any in_dim. */
int orc_matvec_f16_strided(const uint16_t* W, const uint16_t* x, uint16_t* y, size_t out_dim,
                           size_t in_dim) {
  if (in_dim == 0) return -1;
  float* xf = (float*)malloc(in_dim * 4);
  orc_h2f_array(x, xf, in_dim);
  float part[64];
  for (size_t r = 0; r < out_dim; ++r) {
    const uint16_t* row = W + r * in_dim;
    for (size_t l = 0; l < 64; ++l) {
      float acc = 0.0f;
      for (size_t j = l; j < in_dim; j += 64) acc = fmaf(orc_h2f(row[j]), xf[j], acc);
      part[l] = acc;
    }
    for (size_t stride = 32; stride > 0; stride >>= 1)
      for (size_t l = 0; l < stride; ++l) part[l] = part[l] + part[l + stride];
    y[r] = orc_f2h_rne(part[0]);
  }
  free(xf);
  return 0;
}

/* matvec.comp:28-41: one invocation per row, sum over j = 0 .. in_dim-1 in
 * order (:35-38, fp32 from 0), fp16 store (:40).  Any in_dim. */
int orc_matvec_f16_serial(const uint16_t* W, const uint16_t* x, uint16_t* y, size_t out_dim,
                          size_t in_dim) {
  if (in_dim == 0) return -1;
  float* xf = (float*)malloc(in_dim * 4);
  orc_h2f_array(x, xf, in_dim);
  for (size_t r = 0; r < out_dim; ++r) {
    const uint16_t* row = W + r * in_dim;
    float acc = 0.0f;
    for (size_t j = 0; j < in_dim; ++j) acc = fmaf(orc_h2f(row[j]), xf[j], acc);
    y[r] = orc_f2h_rne(acc);
  }
  free(xf);
  return 0;
}

uint32_t orc_argmax_f16(const uint16_t* vals, size_t n) {
  const size_t E = (n + 255) / 256;
  float mv[256];
  uint32_t mi[256];
  for (size_t l = 0; l < 256; ++l) {                 /* argmax.comp:243-258 */
    float lm = -3.402823466e+38f;
    uint32_t li = 0;
    for (size_t i = 0; i < E; ++i) {
      const size_t idx = l * E + i;
      if (idx < n) {
        const float v = orc_h2f(vals[idx]);
        if (v > lm) { lm = v; li = (uint32_t)idx; }
      }
    }
    mv[l] = lm; mi[l] = li;
  }
  for (size_t stride = 128; stride > 0; stride >>= 1) /* :261-270 */
    for (size_t l = 0; l < stride; ++l)
      if (mv[l + stride] > mv[l]) { mv[l] = mv[l + stride]; mi[l] = mi[l + stride]; }
  return mi[0];
}

uint32_t orc_lm_head_argmax(const uint16_t* W, const uint16_t* x, size_t vocab,
                            size_t hidden, uint16_t* logits) {
  uint16_t* lg = logits ? logits : (uint16_t*)malloc(vocab * 2);
  orc_matvec_f16(W, x, lg, vocab, hidden);
  const uint32_t idx = orc_argmax_f16(lg, vocab);
  if (!logits) free(lg);
  return idx;
}
