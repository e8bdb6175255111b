/*
 * spock_hip.h -- C ABI of the MI355X (gfx950) DeltaNet hot path.
 *
 * Drop-in replacement for the Vulkan dispatches of Alexintosh/spock's
 * DecodeSession on three sub-paths: gated-DeltaNet chunk prefill, the fused
 * DeltaNet recurrent decode step, and the fp16 decode GEMV / lm_head + argmax.
 *
 * Conventions (every entry point):
 *   - returns SPK_OK (0) or a negative SPK_ERR_* code; no exception crosses the
 *     ABI; spk_last_error() gives a message for the calling thread;
 *   - all tensor pointers are caller-owned DEVICE memory (hipMalloc'd), plain
 *     pointers plus sizes; fp16 tensors are passed as uint16_t bit patterns;
 *   - calls are stream-ordered and asynchronous on `stream` (NULL = default
 *     stream); nothing is allocated inside a call except where stated;
 *   - re-entrant per stream: concurrent calls on different streams must not
 *     share output or workspace buffers.
 * Layouts and numerics follow the reference shaders cited per entry point
 * (paths relative to the Alexintosh/spock checkout).
 */
#ifndef SPOCK_HIP_H
#define SPOCK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* spk_stream_t; /* == hipStream_t */

enum {
  SPK_OK = 0,
  SPK_ERR_NULL = -1,      /* a required pointer is NULL */
  SPK_ERR_SHAPE = -2,     /* unsupported or inconsistent shape */
  SPK_ERR_HIP = -3,       /* the HIP runtime reported an error */
  SPK_ERR_ALIGN = -4,     /* a pointer or stride breaks the alignment contract */
  SPK_ERR_ARG = -5        /* any other invalid argument */
};

enum { SPK_F32 = 0, SPK_F16 = 1 };

/* Message for the last non-zero status returned on this thread. */
const char* spk_last_error(void);
/* ABI version: (major << 16) | minor. */
uint32_t spk_abi_version(void);

/* ------------------------------------------------------------------------
 * Gated-DeltaNet chunk prefill (WY/UT chunk rule).
 *
 * Replaces: run_deltanet_chunk_rule (src/runtime/deltanet_chunk.hpp:39-40,
 * deltanet_chunk.cpp:53-284) and the tiled dispatch of
 * shaders/deltanet_chunk_prefill_tiled.comp:53-273 issued by
 * DecodeSession::gpu_chunk_prefill_from_gpu_collect (vk_session.cpp:4466-4828,
 * dispatch at :4573) and gpu_chunk_prefill (:4192-4465).
 *
 * Inputs are head-major as the reference collects them
 * (deltanet_prefill_collect.comp): q,k [H][N][dk], v [H][N][dv] (fp32 or fp16
 * per `input_dtype`), g and beta fp32 [H][N].  With cu_seqlens == NULL there is
 * one sequence of N tokens; otherwise sequence s owns tokens
 * [cu_seqlens[s], cu_seqlens[s+1]) (device int32, num_seqs+1 entries, host
 * copy in cu_seqlens_host) and is chunked from its own start and zero padded
 * independently.  Precondition: the device copy holds the same values as
 * cu_seqlens_host when the kernels run.  The call validates and sizes the
 * launch from the host copy (and, for up to 32 sequences, builds the
 * kernels' sequence tables from it, never reading the device copy); for
 * larger packs the kernels read the device copy and treat a span outside
 * [0, total_tokens], or one whose chunks would exceed the workspace sized
 * from the host copy, as empty -- a differing device copy gives wrong
 * results, but no access outside the caller's buffers.
 * initial_state (nullable = zeros, which is what the tiled shader assumes,
 * :66-71) and out_state are [num_seqs][H][dk][dv] fp32.
 * out_core row (h, t) starts at out_core + (h*core_head_stride + t)*dv, so the
 * reference's single output buffer [H*total_seq*dv | H*dk*dv] is addressed by
 * core_head_stride = total_seq and out_state = out_core + H*total_seq*dv.
 * Supported shape: dk == dv == 128, chunk_size == 64.
 * workspace: device buffer of spk_chunk_prefill_workspace_size() bytes,
 * 256-byte aligned, contents ignored.
 * ---------------------------------------------------------------------- */
typedef struct SpkChunkArgs {
  int32_t num_heads;
  int32_t total_tokens;      /* N: tokens of all sequences (sequence_length) */
  int32_t key_dim;           /* 128 */
  int32_t value_dim;         /* 128 */
  int32_t chunk_size;        /* 64 */
  int32_t use_qk_l2norm;     /* deltanet_chunk.cpp:78-85 */
  float q_scale;             /* 0 => 1/sqrt(key_dim) (deltanet_chunk.cpp:87) */
  int32_t input_dtype;       /* SPK_F32 or SPK_F16, for q/k/v */
  const void* q;
  const void* k;
  const void* v;
  const float* g;
  const float* beta;
  const float* initial_state;
  float* out_core;
  int64_t core_head_stride;  /* tokens per head row block; 0 => total_tokens */
  float* out_state;
  const int32_t* cu_seqlens;       /* device, nullable */
  const int32_t* cu_seqlens_host;  /* host, required when cu_seqlens != NULL */
  int32_t num_seqs;                /* 1 when cu_seqlens == NULL */
  void* workspace;
  size_t workspace_bytes;
} SpkChunkArgs;

size_t spk_chunk_prefill_workspace_size(int32_t num_heads, int32_t total_tokens,
                                        int32_t num_seqs, int32_t chunk_size);
int spk_chunk_prefill(const SpkChunkArgs* args, spk_stream_t stream);

/* Prefill collect for one token: shaders/deltanet_prefill_collect.comp:75-108
 * (dispatch vk_session.cpp:1632-1670).  dn_qkv fp16 [Q H*dk | K H*dk | V H*dv],
 * g_beta fp32 [g H | beta H]; outputs head-major fp32 with row stride seq_len. */
int spk_prefill_collect(const uint16_t* dn_qkv, const float* g_beta, float* q_out,
                        float* k_out, float* v_out, float* g_out, float* beta_out,
                        int32_t num_heads, int32_t seq_len, int32_t token_idx,
                        int32_t key_dim, int32_t value_dim, spk_stream_t stream);

/* Last-token core_attn_out -> fp16 with the reference's truncating, flushing
 * conversion: shaders/deltanet_chunk_last_to_fp16.comp:37-77 (dispatch
 * vk_session.cpp:4628).  dst[h*dv+d] = trunc16(src[(h*total_seq+seq_len-1)*dv+d]). */
int spk_chunk_last_to_fp16(const float* src, uint16_t* dst, int32_t num_heads,
                           int32_t value_dim, int32_t seq_len, int32_t total_seq,
                           spk_stream_t stream);

/* ------------------------------------------------------------------------
 * DeltaNet recurrent decode step, batched over B independent sequences.
 *
 * Per sequence the buffers are the reference's per-layer buffers
 * (vk_session.cpp:350-371): qkv fp16 [Q H*128 | K H*128 | V H*128]
 * (conv output written back; the gated output overwrites V), conv_state fp16
 * channel-major [conv_dim][4], state fp32 [H][128][128] (+ optional g/beta
 * tail, see spk_deltanet_recurrent), z fp16 [H*128], a and b fp16 [H].
 * Shared: conv_weight fp16 [conv_dim][4], a_log_bias fp32 [layers][H][2] =
 * (A_log, dt_bias) (vk_session.cpp:486-495), norm_weight fp32 [128].
 * Strides are in elements between consecutive sequences.  H == 16 heads of
 * key_dim == value_dim == 128 (conv_dim = 6144).  state must be 16-byte
 * aligned with state_stride % 4 == 0.
 * ---------------------------------------------------------------------- */
typedef struct SpkDecodeArgs {
  int32_t batch;
  int32_t num_heads;        /* 16 */
  int32_t layer_idx;        /* row of a_log_bias */
  float q_scale;            /* 0 => 1/sqrt(128) */
  float rms_eps;            /* 0 => 1e-6 */
  uint16_t* qkv;            int64_t qkv_stride;
  uint16_t* conv_state;     int64_t conv_state_stride;
  const uint16_t* conv_weight;
  const uint16_t* a;
  const uint16_t* b;        int64_t ab_stride;
  const float* a_log_bias;
  float* state;             int64_t state_stride;
  const uint16_t* z;        int64_t z_stride;
  const float* norm_weight;
} SpkDecodeArgs;

/* Fused: deltanet_conv_l2_qk.comp:41-111 followed by
 * deltanet_recurrent_gbeta_norm_gate.comp:91-225 (dispatches
 * vk_session.cpp:2876-2884 and :3212-3219), one kernel, state read once. */
int spk_deltanet_decode_step(const SpkDecodeArgs* args, spk_stream_t stream);
/* deltanet_conv_l2_qk.comp alone (uses qkv, conv_state, conv_weight). */
int spk_deltanet_conv_l2_qk(const SpkDecodeArgs* args, spk_stream_t stream);
/* deltanet_recurrent_gbeta_norm_gate.comp alone (qkv already convolved). */
int spk_deltanet_recurrent_gbeta_norm_gate(const SpkDecodeArgs* args, spk_stream_t stream);
/* Unfused deltanet_recurrent.comp (prefill path vk_session.cpp:1717-1742):
 * g and beta are read from the state tail state[H*128*128 + h] and
 * state[H*128*128 + H + h]; the raw output is rounded to fp16 into V.
 * Uses qkv, state (stride must include the tail) and q_scale. */
int spk_deltanet_recurrent(const SpkDecodeArgs* args, spk_stream_t stream);

/* ------------------------------------------------------------------------
 * fp16 decode GEMV, lm_head and argmax.
 * ---------------------------------------------------------------------- */

/* y[r] = fp16(sum_j W[r][j] x[j]), fp32 accumulation.  Replaces matvec.comp:28-41
 * and matvec_tiled.comp:41-84 (bind/dispatch vk_session.cpp:2247-2256); the
 * summation order is lm_head_tiled.comp's (64 lanes x contiguous spans, then a
 * 32..1 tree).  W row-major [out_dim][in_dim]; in_dim % 64 == 0. */
int spk_matvec_f16(const uint16_t* W, const uint16_t* x, uint16_t* y, int32_t out_dim,
                   int32_t in_dim, spk_stream_t stream);

/* The same GEMV in the summation order of a chosen reference shader (the
 * session's pipeline selection, vk_session.cpp:2228-2256 and :3533-3545):
 *   SPK_MATVEC_ORDER_SPANS    lm_head_tiled.comp:40-87 (= spk_matvec_f16;
 *                             in_dim % 64 == 0)
 *   SPK_MATVEC_ORDER_STRIDED  matvec_tiled.comp:41-84 (SPOCK_GPU_MATVEC_TILED):
 *                             lane l of 64 sums j = l, l+64, ... sequentially,
 *                             then the 32..1 tree; any in_dim > 0
 *   SPK_MATVEC_ORDER_SERIAL   matvec.comp:28-41 (the session's default): one
 *                             sequential sum over j = 0 .. in_dim-1; any in_dim > 0
 * fp32 accumulation from 0 (fp16 x fp16 products are exact, so fma and
 * mul+add agree), one RNE rounding to fp16.  SPK_ERR_ARG for another order. */
enum { SPK_MATVEC_ORDER_SPANS = 0, SPK_MATVEC_ORDER_STRIDED = 1, SPK_MATVEC_ORDER_SERIAL = 2 };
int spk_matvec_f16_order(const uint16_t* W, const uint16_t* x, uint16_t* y, int32_t out_dim,
                         int32_t in_dim, int32_t order, spk_stream_t stream);

/* Several independent GEMVs, up to 4 per launch (the decode projections). */
typedef struct SpkMatvecDesc {
  const uint16_t* W;
  const uint16_t* x;
  uint16_t* y;
  int32_t out_dim;
  int32_t in_dim;
} SpkMatvecDesc;
int spk_matvec_f16_batched(const SpkMatvecDesc* descs, int32_t count, spk_stream_t stream);

/* argmax over fp16 values with argmax.comp:27-63's exact tie rule (256 lanes
 * over contiguous blocks, first strict maximum per lane, strictly-greater tree;
 * NaN and -inf never win; all-invalid gives 0).  Dispatch vk_session.cpp:3558-3563. */
int spk_argmax_f16(const uint16_t* vals, int32_t n, uint32_t* out_index, spk_stream_t stream);

/* Tied lm_head (lm_head_tiled.comp:40-87, dispatch vk_session.cpp:3533-3547)
 * fused with argmax (same tie rule as spk_argmax_f16 over the fp16 logits).
 * logits (nullable) receives the fp16 logits.  workspace: device buffer of
 * spk_lm_head_workspace_size(vocab) bytes, contents ignored. */
size_t spk_lm_head_workspace_size(int32_t vocab);
int spk_lm_head_argmax(const uint16_t* W, const uint16_t* x, int32_t vocab, int32_t hidden,
                       uint16_t* logits, uint32_t* out_index, void* workspace,
                       size_t workspace_bytes, spk_stream_t stream);

/* spk_lm_head_argmax without a workspace argument.  No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * per-workgroup partial keys live in a static device array of
 * SPK_LM_HEAD_NOALLOC_MAX_VOCAB / 16 keys (128 KiB), one copy per device held
 * until the process ends; the call allocates nothing.  vocab above
 * SPK_LM_HEAD_NOALLOC_MAX_VOCAB is rejected with SPK_ERR_SHAPE.  Calls that
 * overlap on one device (concurrent streams or threads) race on that array:
 * serialise them. */
#define SPK_LM_HEAD_NOALLOC_MAX_VOCAB 262144
int spk_lm_head_argmax_noalloc(const uint16_t* W, const uint16_t* x, int32_t vocab, int32_t hidden,
                               uint16_t* logits, uint32_t* out_index, spk_stream_t stream);

/* ------------------------------------------------------------------------
 * Qwen3.5 text model: the rest of the per-token decode loop and the prefill
 * element-wise operations (DecodeSession::decode, vk_session.cpp:2560-3400).
 * Results are bit-identical to the CPU restatement; every operation's order
 * is stated in oracle/model.h.  Hidden size 1024; attention 8 query heads,
 * 2 KV heads, head_dim 256, rotary dim 64; KV cache per layer
 * [max_seq][K 2x256 | V 2x256] fp16 (vk_session.cpp:322-328).
 * ---------------------------------------------------------------------- */

enum { SPK_GEMV_IN_PLAIN = 0, SPK_GEMV_IN_RMSNORM = 1, SPK_GEMV_IN_SILU_GATE = 2 };

/* Input of a fused projection, computed once per workgroup:
 *   PLAIN      x                                         (matvec_tiled.comp)
 *   RMSNORM    fp16(RMSNorm(h) * (1 + x2)), in_dim 1024  (rms_norm.comp before
 *              the projection, vk_session.cpp:2606-2613, :3283-3289);
 *              h = x, or row token[0] of x when token != NULL (the embedding
 *              lookup of embedding_lookup.comp, token read on the device;
 *              ids outside [0, token_rows) select row 0), in which case
 *              h_out (nullable) receives that row: the residual stream
 *   SILU_GATE  fp16(silu(x) * x2)                        (silu_gate.comp) */
typedef struct SpkGemvInput {
  int32_t kind;
  int32_t in_dim;          /* multiple of 512, <= 4096 */
  const uint16_t* x;
  const uint16_t* x2;
  const int32_t* token;
  int32_t token_rows;
  uint16_t* h_out;
} SpkGemvInput;

/* y = fp16(W . x), or fp16(residual + fp16(W . x)) (residual_add.comp after
 * the projection) when residual != NULL; y may equal residual (in-place update
 * of the stream) but must not alias the input vectors.  With W_up != NULL the
 * output is the SiLU-gated pair of the MLP (gate/up matvecs then
 * silu_gate.comp): y = fp16(silu(fp16(W . x)) * fp16(W_up . x)); a launch
 * holds either only pairs or only single projections. */
typedef struct SpkGemvOutput {
  const uint16_t* W;         /* [out_dim][in_dim] fp16, 16-byte aligned */
  uint16_t* y;
  const uint16_t* residual;
  int32_t out_dim;
  const uint16_t* W_up;      /* nullable, [out_dim][in_dim] */
} SpkGemvOutput;

/* Up to 8 projections of one input (one launch per 4 outputs).  Replaces the
 * rms_norm + matvec (+ residual_add / silu_gate) dispatch runs of
 * vk_session.cpp:2606-2870 and :3276-3360. */
int spk_gemv_fused(const SpkGemvInput* in, const SpkGemvOutput* outs, int32_t count,
                   spk_stream_t stream);

/* A batch-1 DeltaNet layer's input in one launch: spk_gemv_fused with the
 * RMSNorm input and the four outputs qkv (6144 rows), z (2048), a (16), b (16),
 * then spk_deltanet_decode_step (d: batch 1, 16 heads, its qkv/z/a/b the
 * outputs' y).  No single counterpart in the reference: it replaces the
 * dispatch runs of vk_session.cpp:2606-2870 (projections) and :2876-2884
 * (conv + recurrence + norm-gate) for a session that runs them back to back.
 * The workgroups that form one head's rows count their arrival in
 * arrive[64 * head], and the last runs that head's step; arrive is 1,024 device
 * ints (4 KiB), zero before the first call, and every call leaves them zero.  Calls that
 * overlap on one `arrive` race.  Same outputs, bit for bit, as the two calls. */
int spk_deltanet_inproj_step(const SpkGemvInput* in, const SpkGemvOutput* outs, const SpkDecodeArgs* d,
                             int32_t* arrive, spk_stream_t stream);

/* Full-attention token mixer: split_q_gate.comp, rms_norm_per_head.comp (q and
 * k, weights applied as 1 + w), rope_apply.comp (pairs (i, i+32) of the first
 * 64 dims, table rope[pos][64] = (cos, sin) pairs), kv_cache_store.comp,
 * attention_decode.comp (softmax(q.K^T / 16) V, GQA 4:1) and sigmoid_gate.comp
 * (dispatches vk_session.cpp:2676-2790). */
typedef struct SpkAttnArgs {
  const uint16_t* qg;        /* q_proj output per token [8][256 query | 256 gate] */
  const uint16_t* k;         /* k_proj output per token [2][256] */
  const uint16_t* v;         /* v_proj output per token [2][256] */
  const uint16_t* q_norm_w;  /* [256] */
  const uint16_t* k_norm_w;  /* [256] */
  const float* rope;         /* [max_seq][64] */
  uint16_t* kv_cache;        /* this layer's [max_seq][1024] */
  int32_t max_seq;
  const int32_t* pos_dev;    /* decode: device int32 position of the token */
  uint16_t* out;             /* gated output per token [2048] */
  void* workspace;
  size_t workspace_bytes;
} SpkAttnArgs;

/* Workspace bytes for `tokens` queries over positions [0, positions). */
size_t spk_attention_workspace_size(int32_t positions, int32_t tokens);
/* The attention layer's projections (spk_gemv_fused with the RMSNorm input
 * and outs = {q|gate [4096], k [512], v [512]}, vk_session.cpp:2606-2675)
 * for a session that runs spk_attention_decode(_oproj) right after: the
 * launch also reads the layer's cached K/V rows 0 .. *attn->pos_dev (at most
 * attn->max_seq; up to 2.5 MiB) and drops them, so that the attention launch
 * finds them in the caches instead of at HBM latency.  attn->qg/k/v must be
 * the three outputs; attn->kv_cache and pos_dev are read, nothing of attn is
 * written.  Same outputs, bit for bit, as spk_gemv_fused. */
int spk_attention_inproj(const SpkGemvInput* in, const SpkGemvOutput* outs, const SpkAttnArgs* attn,
                         spk_stream_t stream);
/* One token at position *pos_dev (< max_seq; read on the device, so the call
 * can be recorded once and replayed); workspace for (max_seq, 1). */
int spk_attention_decode(const SpkAttnArgs* args, spk_stream_t stream);
/* spk_attention_decode followed by the o_proj projection (+ residual):
 * attention_decode.comp, sigmoid_gate.comp, the o_proj matvec and
 * residual_add.comp (vk_session.cpp:2676-2830) in two launches instead of
 * three.  The second stage -- blocks combined in order, normalised,
 * sigmoid-gated into args->out -- runs in the last-finishing block workgroup
 * of each KV head, found by an arrival count in the last 512 bytes of the
 * workspace: they must be zero before the first call, and every call leaves
 * them zero (calls that overlap on one workspace race).  o_proj: W
 * [out_dim][2048], y, residual as in spk_gemv_fused (W_up must be NULL; y and
 * residual must not be args->out).  Same bits as spk_attention_decode then
 * spk_gemv_fused (PLAIN input over args->out). */
int spk_attention_decode_oproj(const SpkAttnArgs* args, const SpkGemvOutput* o_proj, spk_stream_t stream);
/* `tokens` consecutive tokens at positions pos0.. (rows of qg/k/v/out are
 * per token); workspace for (pos0 + tokens, tokens). */
int spk_attention_prefill(const SpkAttnArgs* args, int32_t pos0, int32_t tokens,
                          spk_stream_t stream);

/* RMSNorm(1 + w) of `rows` rows of n = 1024 (rms_norm.comp) or n = 256
 * (rms_norm_per_head.comp). */
int spk_rmsnorm_f16(const uint16_t* x, const uint16_t* w, uint16_t* y, int32_t rows, int32_t n,
                    spk_stream_t stream);
/* silu_gate.comp: y = fp16(silu(g) * u) */
int spk_silu_gate_f16(const uint16_t* g, const uint16_t* u, uint16_t* y, int64_t n,
                      spk_stream_t stream);
/* residual_add.comp: y = fp16(a + b) */
int spk_residual_add_f16(const uint16_t* a, const uint16_t* b, uint16_t* y, int64_t n,
                         spk_stream_t stream);
/* embedding_lookup.comp for n_tokens device token ids (rows of 1024; ids
 * outside [0, vocab) give zero rows). */
int spk_embedding_f16(const uint16_t* E, const int32_t* tokens, int32_t n_tokens, int32_t vocab,
                      uint16_t* y, spk_stream_t stream);
/* Final RMSNorm(1+w) (rms_norm.comp; skipped when norm_w is NULL, else
 * hidden == 1024), tied lm_head (lm_head_tiled.comp's order, as
 * spk_lm_head_argmax) and argmax.comp's winner, in one launch: every
 * workgroup folds its best 64-bit key into one of SPK_ARGMAX_KEY_WORDS device
 * words with a device-scope atomic max.  key: SPK_ARGMAX_KEY_WORDS words
 * (512 bytes) of device memory that hold 0 before the call;
 * spk_argmax_key_take reduces them and sets them back to 0.  The final norm,
 * lm_head, argmax and record-token dispatches of vk_session.cpp:3533-3563
 * become this call and the take. */
#define SPK_ARGMAX_KEY_WORDS 64
int spk_lm_head_argmax_key(const uint16_t* W, const uint16_t* x, const uint16_t* norm_w, int32_t vocab,
                           int32_t hidden, uint16_t* logits, uint64_t* key, spk_stream_t stream);
/* *out_index = argmax.comp's index for the key words left by
 * spk_lm_head_argmax_key over `vocab` rows; the words are set to 0.  With pos != NULL the token is also
 * recorded as spk_record_token does (history[*count] = index when *count <
 * capacity, *count += 1, *pos += 1). */
int spk_argmax_key_take(uint64_t* key, int32_t vocab, uint32_t* out_index, int32_t* pos, int32_t* count,
                        int32_t* history, int32_t capacity, spk_stream_t stream);
/* spk_lm_head_argmax_key and spk_argmax_key_take in one launch (the final
 * norm, lm_head, argmax and record-token dispatches of vk_session.cpp:3533-3563
 * as one kernel): each workgroup of the lm_head writes its 64-bit key to a
 * slot of its own, and one extra workgroup polls the slots until all are
 * written, reduces them with argmax.comp's tie rule, sets them back to 0 and
 * writes *out_index (and the bookkeeping of spk_argmax_key_take when pos !=
 * NULL).  slots: slot_words >= spk_lm_head_take_slots(vocab) 64-bit words of
 * device memory that hold 0 before the call (the call leaves them at 0);
 * calls that overlap on one slot array race.  The poll is bounded, so the
 * kernel always ends: if the slots are not all written within seconds (the
 * lm_head workgroups held off the GPU that long), *out_index is 0xffffffff,
 * and slots written after the give-up stay set: zero the array again before
 * the next call. */
size_t spk_lm_head_take_slots(int32_t vocab);
int spk_lm_head_argmax_take(const uint16_t* W, const uint16_t* x, const uint16_t* norm_w, int32_t vocab,
                            int32_t hidden, uint16_t* logits, uint64_t* slots, size_t slot_words,
                            uint32_t* out_index, int32_t* pos, int32_t* count, int32_t* history,
                            int32_t capacity, spk_stream_t stream);
/* *p += delta on the device (advances a device position counter). */
int spk_add_i32(int32_t* p, int32_t delta, spk_stream_t stream);

/* ---- prompt-length (prefill) forms ------------------------------------- */

/* C[M][N] = fp16(A[M][K] . W[N][K]^T), or fp16(residual + fp16(...)) when
 * residual != NULL (may equal C; must not alias A or W); fp16 operands, fp32
 * accumulation on the matrix cores.  The prompt-wide form of every decode
 * matvec (matvec_tiled.comp over all prompt tokens).  K % 32 == 0; A, W
 * 16-byte aligned with lda, ldw multiples of 8.  Not bit-identical to the
 * matvec's summation order. */
int spk_gemm_f16(const uint16_t* A, int64_t lda, const uint16_t* W, int64_t ldw, uint16_t* C,
                 int64_t ldc, const uint16_t* residual, int32_t M, int32_t N, int32_t K,
                 spk_stream_t stream);

/* DeltaNet prompt conv: for every token t of qkv [tokens][ld] (raw in_proj_qkv
 * output, fp16), the deltanet_conv_l2_qk.comp operations of decode (window of
 * the raw inputs t-3..t, earlier ones from conv_state [6144][4]; SiLU; fp16;
 * L2 of each Q/K head block), written head-major for the chunk rule: q_hm,
 * k_hm, v_hm [16][tokens][128] fp16.  conv_state then holds the last 4 raw
 * inputs.  Replaces the per-token collect loop of vk_session.cpp:1464-1716. */
int spk_deltanet_prefill_conv(const uint16_t* qkv, int64_t ld, uint16_t* conv_state,
                              const uint16_t* conv_weight, int32_t tokens, uint16_t* q_hm,
                              uint16_t* k_hm, uint16_t* v_hm, spk_stream_t stream);
/* g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b) for every token
 * (deltanet_recurrent_gbeta_norm_gate.comp:102-116); a, b [tokens][ld] fp16;
 * g, beta head-major [16][tokens] fp32. */
int spk_deltanet_prefill_gbeta(const uint16_t* a, const uint16_t* b, int64_t ld,
                               const float* a_log_bias, int32_t layer_idx, int32_t tokens,
                               float* g, float* beta, spk_stream_t stream);
/* Gated RMSNorm of the chunk rule's fp32 output (the fused decode shader's
 * :182-224 on every token): core row (h, t) at core + (h*core_head_stride +
 * t)*128, z [tokens][z_ld] fp16, out [tokens][out_ld] fp16. */
int spk_deltanet_norm_gate(const float* core, int64_t core_head_stride, const uint16_t* z,
                           int64_t z_ld, const float* norm_weight, float eps, int32_t tokens,
                           uint16_t* out, int64_t out_ld, spk_stream_t stream);
/* The unfused decode norm-gate, deltanet_norm_gate.comp:80-105 (dispatched
 * after deltanet_recurrent.comp at vk_session.cpp:1743-1756 and :3245-3257,
 * push constants {num_heads, head_dim, eps, output_offset = 0}): per head h,
 * io[h*128 .. +127] (fp16, in place) <- fp16(fp16(w * RMSNorm(io)) *
 * SiLU(z)), z [num_heads][128] fp16, norm_weight [128] fp32.  head_dim must
 * be 128. */
int spk_deltanet_norm_gate_f16(uint16_t* io, const uint16_t* z, const float* norm_weight,
                               int32_t num_heads, int32_t head_dim, float eps, spk_stream_t stream);
/* history[*count] = *token (when *count < capacity), *count += 1, *pos += 1:
 * the greedy loop's bookkeeping, kept on the device so one recorded decode
 * step serves every token. */
int spk_record_token(const int32_t* token, int32_t* pos, int32_t* count, int32_t* history,
                     int32_t capacity, spk_stream_t stream);

/* ---- prompt-wide kernels in the CPU restatement's operation order -------
 * The parity forms of spk_gemm_f16 and spk_chunk_prefill: bit-identical to
 * the oracle, so a prompt prefilled with them leaves exactly the state (and
 * greedy tokens) of the CPU path.  They keep the reference's sequential
 * reduction orders: the matvec runs on fp32 matrix cores one product per
 * instruction (exact for fp16 operands), the chunk rule on the vector ALUs. */

/* Y[t][r] (+ residual as in spk_gemm_f16) for every row t of X: each output
 * bit-identical to spk_matvec_f16 of X's row t (the matvec_tiled /
 * lm_head_tiled order).  in_dim % 64 == 0, in_dim <= 4096. */
int spk_matvec_f16_rows(const uint16_t* W, const uint16_t* X, int64_t ldx, uint16_t* Y,
                        int64_t ldy, const uint16_t* residual, int32_t rows, int32_t out_dim,
                        int32_t in_dim, spk_stream_t stream);

/* run_deltanet_chunk_rule (deltanet_chunk.cpp:53-284) with the reference's
 * loop nests and sequential reductions, exp = the library's deterministic exp;
 * one sequence (cu_seqlens NULL), dk == dv == 128, chunk_size == 64;
 * initial_state must not alias out_state.  Same argument struct and
 * alignment rules as spk_chunk_prefill (q/k/v 16-byte aligned for fp32, 8 for
 * fp16; workspace 16); workspace of spk_chunk_prefill_ordered_workspace_size(). */
size_t spk_chunk_prefill_ordered_workspace_size(int32_t num_heads, int32_t total_tokens);
int spk_chunk_prefill_ordered(const SpkChunkArgs* args, spk_stream_t stream);

/* ------------------------------------------------------------------------
 * Diagnostics (no reference counterpart).
 * ---------------------------------------------------------------------- */

/* Evaluates the device scalar numerics used by the bit-exact kernels on x[n]
 * and writes six planes of n floats to out: exp, log, 1/sqrt, SiLU,
 * float(half_rne(x)), and the bits of the truncating half in the low 16 bits. */
int spk_selftest_numerics(const float* x, int32_t n, float* out, spk_stream_t stream);

/* Measured ceilings beside the datasheet peaks.  spk_selftest_mfma_peak runs
 * `blocks` workgroups of 4 wavefronts, each issuing 8 independent chains of
 * `iters` v_mfma_f32_16x16x4_f32 (2048 FLOP each); out holds blocks * 256
 * floats.  spk_selftest_stream_read reads `bytes` (16-byte multiple, 16-byte
 * aligned) once with `blocks` workgroups of 256 threads; mode bit 0: plain
 * cached loads (else non-temporal), bit 1: the grid walks the whole buffer in
 * strides (else each workgroup reads its own contiguous share); out holds
 * `blocks` words (almost never written). */
int spk_selftest_mfma_peak(int32_t blocks, int32_t iters, float* out, spk_stream_t stream);
/* out[i] = the XCD (XCC) that ran workgroup i of a `blocks`-workgroup launch.
 * spk_deltanet_inproj_step and spk_attention_decode_oproj hand rows from one
 * workgroup to another through the L2 they share, which holds when
 * workgroup ids are dealt to the XCDs round-robin: (id + s) mod 8 on
 * MI355X, where the start s continues the rotation of earlier dispatches, so
 * ids congruent mod 8 share an XCD; the GPU tests check that with this call. */
int spk_selftest_xcc_ids(int32_t blocks, int32_t* out, spk_stream_t stream);
int spk_selftest_stream_read(const void* p, size_t bytes, int32_t blocks, int32_t mode, uint32_t* out,
                             spk_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif
