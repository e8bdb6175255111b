// deltanet_session.hpp -- the DeltaNet hot path of the reference's
// DecodeSession, on HIP.
//
// Owns the per-layer device buffers that src/runtime/vk_session.hpp:291-401
// and vk_session.cpp:350-378 / :1083-1104 allocate for the DeltaNet layers,
// in the same layouts:
//   dn_state       [layer] x ([H][128][128] fp32 + g[H], beta[H] tail) = 1,048,704 B
//   dn_conv_state  [layer] x [6144][4] fp16 (channel-major)
//   dn_a_log_bias  [layer][H][2] fp32 = (A_log, dt_bias)
//   collect segments per layer: q, k, v fp32 [H][prompt_len][128], g, beta
//   fp32 [H][prompt_len], each 256-byte aligned (align_storage_offset, :63-67;
//   layout :1632-1660), with capacity for max_seq tokens
//   chunk output   [H*total_seq*128 | H*128*128] fp32 (total_seq = prompt_len
//   rounded up to 64)
//   dn_chunk_attn_out [layer][H*128] fp16 (last-token core, :378)
// and runs, on one HIP stream, the operations the session performs on them:
//   collect_prefill_token          deltanet_prefill_collect dispatch, :1632-1670
//   gpu_chunk_prefill_from_gpu_collect(dn_idx, seq_len)          :4466-4828
//   run_chunk_prefill(seq_len)     every layer                   :4830-4952
//   deltanet_decode_step           conv+L2 then g/beta+recurrent+norm-gate,
//                                  :2876-2884 and :3212-3219 (one fused kernel)
//   lm_head_argmax                 :3533-3563
//   reset()                        zero recurrent state          vk_session.hpp:41
// Weights stay caller-owned device memory (the reference's WeightArtifact).
// Like the reference session it is single-threaded, owns its buffers through
// RAII and reports failures as std::runtime_error; unlike it, calls are
// stream-ordered and return without waiting (synchronize() waits).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

#include "hip_buffer.hpp"

namespace spock::hip {

class DeltaNetSession {
 public:
  // Model constants (vk_session.hpp:383-401 for Qwen3.5-0.8B).
  static constexpr std::uint32_t DN_HEADS = 16;
  static constexpr std::uint32_t DN_K_DIM = 128;
  static constexpr std::uint32_t DN_V_DIM = 128;
  static constexpr std::uint32_t DN_CONV_KS = 4;
  static constexpr std::uint32_t DN_KEY_TOTAL = DN_HEADS * DN_K_DIM;
  static constexpr std::uint32_t DN_VAL_TOTAL = DN_HEADS * DN_V_DIM;
  static constexpr std::uint32_t DN_CONV_DIM = DN_KEY_TOTAL * 2 + DN_VAL_TOTAL;
  static constexpr std::uint32_t NUM_DN_LAYERS = 18;
  static constexpr std::uint32_t MAX_SEQ = 2048;
  static constexpr std::size_t kStateFloats = std::size_t(DN_HEADS) * DN_K_DIM * DN_V_DIM + 2 * DN_HEADS;
  static constexpr float kRmsEps = 1e-6f;

  explicit DeltaNetSession(std::uint32_t num_layers = NUM_DN_LAYERS, std::uint32_t max_seq = MAX_SEQ);
  ~DeltaNetSession();
  DeltaNetSession(const DeltaNetSession&) = delete;
  DeltaNetSession& operator=(const DeltaNetSession&) = delete;

  hipStream_t stream() const { return stream_; }
  std::uint32_t num_layers() const { return num_layers_; }
  std::uint32_t max_seq() const { return max_seq_; }

  // Zeroes dn_state (with its g/beta tail), dn_conv_state and the last-token
  // outputs: a fresh prompt.
  void reset();

  // Host uploads of per-layer state (the reference fills these from the
  // artifact and from its own prefill); sizes are checked.
  void upload_a_log_bias(const std::vector<float>& a_log_bias);  // [layers][H][2]
  void upload_state(std::uint32_t dn_idx, const std::vector<float>& state);  // kStateFloats or H*128*128
  void upload_conv_state(std::uint32_t dn_idx, const std::vector<std::uint16_t>& conv);  // [6144][4]
  std::vector<float> download_state(std::uint32_t dn_idx);  // kStateFloats
  std::vector<std::uint16_t> download_conv_state(std::uint32_t dn_idx);
  std::vector<std::uint16_t> download_chunk_attn_out(std::uint32_t dn_idx);  // [H*128] fp16

  // Device addresses of the per-layer buffers (for callers that bind them).
  float* dn_state(std::uint32_t dn_idx) const;
  std::uint16_t* dn_conv_state(std::uint32_t dn_idx) const;
  std::uint16_t* dn_chunk_attn_out(std::uint32_t dn_idx) const;
  const float* dn_a_log_bias() const { return a_log_bias_.get<float>(); }

  // Stores prompt token `token_idx` (of prompt_len) of layer dn_idx in its
  // collect segments. dn_qkv: device fp16 [6144] (conv'd + L2-normed q/k, v).
  // g_beta: device fp32 [g H | beta H]; nullptr reads the layer's dn_state
  // tail, which is what the reference binds (vk_session.cpp:1642).
  void collect_prefill_token(std::uint32_t dn_idx, std::uint32_t token_idx, std::uint32_t prompt_len,
                             const std::uint16_t* dn_qkv, const float* g_beta = nullptr);
  // Chunk rule over the prompt_len collected tokens of layer dn_idx from a
  // zero state: writes the final state into dn_state[dn_idx] (tail untouched)
  // and the fp16 last-token core into dn_chunk_attn_out[dn_idx].
  void gpu_chunk_prefill_from_gpu_collect(std::uint32_t dn_idx, std::uint32_t prompt_len);
  void run_chunk_prefill(std::uint32_t prompt_len);
  // fp32 core_attn_out of the last chunk prefill, [H][prompt_len][128].
  std::vector<float> download_last_core(std::uint32_t prompt_len);

  // One decode token for layer dn_idx. In place: dn_qkv (conv output, then the
  // gated output over V), dn_conv_state[dn_idx], dn_state[dn_idx].
  // a, b fp16 [H]; z fp16 [2048]; conv_weight fp16 [6144][4]; norm_weight fp32 [128].
  void deltanet_decode_step(std::uint32_t dn_idx, std::uint16_t* dn_qkv, const std::uint16_t* a,
                            const std::uint16_t* b, const std::uint16_t* z,
                            const std::uint16_t* conv_weight, const float* norm_weight);

  // Tied lm_head + argmax: the greedy token for hidden x (fp16 [hidden]).
  // Blocks until the index is on the host. logits (nullable) receives fp16 [vocab].
  std::uint32_t lm_head_argmax(const std::uint16_t* embed_tokens, const std::uint16_t* x,
                               std::uint32_t vocab, std::uint32_t hidden, std::uint16_t* logits = nullptr);

  void synchronize();

 private:
  struct Segments {
    float *q, *k, *v, *g, *beta;
  };
  void check_layer(std::uint32_t dn_idx) const;
  void check_prompt_len(std::uint32_t prompt_len) const;
  Segments segments(std::uint32_t dn_idx, std::uint32_t prompt_len) const;

  std::uint32_t num_layers_;
  std::uint32_t max_seq_;
  hipStream_t stream_ = nullptr;
  DeviceBuffer state_;         // num_layers x kStateFloats
  DeviceBuffer conv_state_;    // num_layers x DN_CONV_DIM x 4 fp16
  DeviceBuffer a_log_bias_;    // num_layers x H x 2
  DeviceBuffer collect_q_, collect_k_, collect_v_, collect_g_, collect_beta_;  // dn_persist_*
  DeviceBuffer chunk_out_;     // [H*total_seq*128 | H*128*128]
  std::uint32_t last_total_seq_ = 0;
  DeviceBuffer chunk_ws_;
  DeviceBuffer attn_out_;      // num_layers x H*128 fp16
  DeviceBuffer lm_ws_;
  std::uint32_t lm_ws_vocab_ = 0;
  DeviceBuffer argmax_idx_;    // u32
};

}  // namespace spock::hip
