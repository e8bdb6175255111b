/*
 * spock_model.h -- C ABI of the MI355X Qwen3.5-0.8B-shaped decode session
 * (libspock_hip_host.so).
 *
 * Replaces the reference's session entry points: DecodeSession(repack_dir,
 * verbose), DecodeSession::decode(prompt_tokens, max_new_tokens) ->
 * DecodeResult and DecodeSession::reset() (src/runtime/vk_session.hpp:22-46,
 * vk_decode.hpp:10-44), over the repacked artifact of
 * src/runtime/weight_loader.hpp:22-54 (text_repack_manifest.json +
 * text_weights.bin).  Prefill follows the HF semantics (chunk rule over the
 * whole prompt for every DeltaNet layer, causal attention over the prompt);
 * decode runs one device-resident step per token (the token id and position
 * stay on the GPU, so the step is recorded once as a HIP graph and replayed).
 *
 * Conventions: int status (0 = ok, negative = error; spk_model_last_error()
 * gives the message for the calling thread); host pointers; one session is
 * used by one host thread at a time (as the reference's DecodeSession).
 */
#ifndef SPOCK_MODEL_H
#define SPOCK_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct SpkModel SpkModel;

/* Timings of one spk_model_generate call (DecodeResult's prefill_ms,
 * decode_ms, gpu_decode_us; vk_decode.hpp:10-24). */
typedef struct SpkGenerateStats {
  double prefill_ms;      /* host wall clock, prompt upload .. first token ready */
  double decode_ms;       /* host wall clock of the decode steps */
  double gpu_prefill_ms;  /* HIP events around the prefill on the session stream */
  double gpu_decode_ms;   /* HIP events around the decode steps */
  int32_t decode_steps;
  int32_t used_graph;
} SpkGenerateStats;

const char* spk_model_last_error(void);

/* spk_model_open flags */
enum {
  SPK_MODEL_NO_GRAPH = 1,        /* launch the decode step's kernels one by one */
  SPK_MODEL_MATRIX_PREFILL = 2,  /* prompt on the matrix cores (spk_gemm_f16, MFMA
                                    chunk rule) instead of the default order of
                                    the CPU restatement (bit-identical prefill) */
  SPK_MODEL_GPU_TIMESTAMPS = 4,  /* GPU time of every decode step (the reference's
                                    SPOCK_GPU_TIMESTAMPS, vk_session.cpp:2188-2201):
                                    a HIP event before each step, graph kept */
  SPK_MODEL_GPU_REGIONS = 8,     /* also GPU time per region of the step
                                    (SPOCK_GPU_BLOCK_TIMESTAMPS, vk_session.cpp:
                                    2204-2218): events after each layer, lm_head and
                                    argmax; the step's kernels are then launched one
                                    by one, since a recorded graph holds no events */
  SPK_MODEL_LMHEAD_ONE_LAUNCH = 16, /* accepted, no effect: the final norm +
                                    lm_head + argmax run as one launch
                                    (spk_lm_head_argmax_take) by default */
  SPK_MODEL_SPLIT_DN_STEP = 32,     /* each DeltaNet layer's input projections and
                                    decode step as two launches (spk_gemv_fused,
                                    spk_deltanet_decode_step) instead of one
                                    (spk_deltanet_inproj_step); same tokens,
                                    about 19 us per token slower */
  SPK_MODEL_LMHEAD_KEY_TAKE = 64    /* the final norm + lm_head with the atomic
                                    argmax key, then the take, as two launches
                                    (spk_lm_head_argmax_key, spk_argmax_key_take)
                                    instead of one; same tokens, about 10 us per
                                    token slower */
};

/* Opens <repack_dir>, uploads every tensor, allocates the per-layer state for
 * max_seq positions (<= 0: 2048, the reference's MAX_SEQ).  By default the
 * decode step is replayed as a HIP graph and the prompt is prefilled in the
 * CPU restatement's order.  NULL on error. */
SpkModel* spk_model_open(const char* repack_dir, int32_t max_seq, int32_t flags);
void spk_model_close(SpkModel* m);

/* Model shape as read from the artifact. */
int spk_model_info(const SpkModel* m, int32_t* layers, int32_t* vocab, int32_t* max_seq);

/* DecodeSession::reset(): zero DeltaNet state, conv state and KV cache. */
int spk_model_reset(SpkModel* m);

/* DecodeSession::decode(): reset, prefill `prompt`, then greedy-generate
 * max_new tokens (the first from the prefill logits).  out_tokens[max_new]. */
int spk_model_generate(SpkModel* m, const int32_t* prompt, int32_t prompt_len, int32_t max_new,
                       int32_t* out_tokens, SpkGenerateStats* stats);

/* GPU timings of the last spk_model_generate call's decode steps (sessions
 * opened with SPK_MODEL_GPU_TIMESTAMPS or SPK_MODEL_GPU_REGIONS; otherwise
 * empty).  DecodeResult::per_token_gpu_us (vk_decode.hpp:19): writes
 * min(*count, capacity) microseconds, one per step; *count = steps. */
int spk_model_gpu_token_us(const SpkModel* m, double* us, int32_t capacity, int32_t* count);
/* DecodeResult::gpu_region_us (vk_decode.hpp:20, filled at vk_session.cpp:
 * 4139-4176), SPK_MODEL_GPU_REGIONS only: microseconds per region summed over
 * the steps, in step order: "layer_0" .. "layer_<n-1>" ("layer_0" includes the
 * embedding gather, which its input norm reads directly, so there is no
 * "embedding" region), "lm_head" (final norm, lm_head and the argmax key in
 * one launch, so no separate "final_norm"; with SPK_MODEL_LMHEAD_ONE_LAUNCH
 * the whole argmax), "argmax" (the take that records the token; empty with
 * SPK_MODEL_LMHEAD_ONE_LAUNCH).  *name stays valid until the next
 * spk_model_generate call. */
int spk_model_gpu_region_count(const SpkModel* m, int32_t* count);
int spk_model_gpu_region(const SpkModel* m, int32_t index, const char** name, double* us);

/* Lower-level steps (the same work as spk_model_generate):
 * prefill at the current position (no reset) -> greedy token;
 * n_steps greedy decode steps continuing from the last token. */
int spk_model_prefill(SpkModel* m, const int32_t* prompt, int32_t prompt_len, int32_t* out_token);
int spk_model_decode(SpkModel* m, int32_t n_steps, int32_t* out_tokens);

/* State exchange (parity tests start a decode from a state computed
 * elsewhere).  Layouts: dn_state [n_dn][16][128][128] fp32, conv
 * [n_dn][6144][4] fp16, kv [n_attn][max_seq][1024] fp16; `pos` is the next
 * position, `last_token` the token the next decode step consumes. */
int spk_model_state_sizes(const SpkModel* m, size_t* dn_state_bytes, size_t* conv_bytes,
                          size_t* kv_bytes);
int spk_model_get_state(SpkModel* m, void* dn_state, void* conv, void* kv, int32_t* pos,
                        int32_t* last_token);
int spk_model_set_state(SpkModel* m, const void* dn_state, const void* conv, const void* kv,
                        int32_t pos, int32_t last_token);
/* fp16 logits [vocab] and final hidden state before the final norm [1024] of
 * the last processed token (either pointer nullable). */
int spk_model_last_output(SpkModel* m, uint16_t* logits, uint16_t* hidden);

/* Writes a seeded synthetic Qwen3.5-0.8B-shaped artifact (layers <= 64,
 * vocab > 0) to <dir>: text_repack_manifest.json + text_weights.bin. */
int spk_artifact_write_synthetic(const char* dir, int32_t layers, int32_t vocab, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif
