// qwen35_session.hpp -- the reference's DecodeSession for the full
// Qwen3.5-0.8B-shaped text model, on HIP.
//
// Mirrors src/runtime/vk_session.hpp:22-46 (construct from a repack
// directory, decode(prompt_tokens, max_new_tokens) -> DecodeResult, reset())
// and owns, in the reference's layouts, the per-layer buffers of
// vk_session.cpp:300-378: DeltaNet state [16][128][128] fp32 + g/beta tail
// (1,048,704 B per layer), conv state [6144][4] fp16, KV cache
// [max_seq][K 2x256 | V 2x256] fp16 per attention layer, a_log_bias
// [layers][16][2], the RoPE table, and the decode activations.
//
// Prefill (HF semantics, modeling_qwen3_5.py:519-530): layer-major over the
// prompt; projections either in the matvec's order (spk_matvec_f16_rows) or on
// the matrix cores (spk_gemm_f16); the DeltaNet conv/g/beta of the decode
// shaders over every token; the chunk rule in the reference's order
// (spk_chunk_prefill_ordered) or on MFMA (spk_chunk_prefill); the gated norm;
// full-attention layers attend causally over the prompt.
// Decode: per token one fixed sequence of launches whose token id and
// position live on the device (spk_gemv_fused with the embedding lookup and
// input norms fused, spk_deltanet_decode_step, spk_attention_decode,
// spk_lm_head_argmax, spk_record_token), recorded once as a HIP graph.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "hip_buffer.hpp"
#include "qwen35_artifact.hpp"

namespace spock::hip {

// DecodeResult (src/runtime/vk_decode.hpp:10-24), the fields this backend fills.
struct DecodeResult {
  std::vector<std::uint32_t> prompt_tokens;
  std::vector<std::uint32_t> generated_tokens;
  double elapsed_ms = 0.0;
  double prefill_ms = 0.0;
  double decode_ms = 0.0;
  double gpu_prefill_us = 0.0;
  double gpu_decode_us = 0.0;
  std::uint32_t decode_steps = 0;
  bool used_graph = false;
  // With GPU timestamps on (vk_decode.hpp:16-21): GPU microseconds of each
  // decode step, and per region of the step summed over the steps, in step
  // order: layer_0 .. layer_{n-1} (layer_0 includes the embedding gather,
  // which its input norm reads directly), lm_head (final norm, lm_head and
  // the argmax key in one launch), argmax (the take that records the token).
  std::vector<double> per_token_gpu_us;
  std::vector<std::pair<std::string, double>> gpu_region_us;
  std::string error;
};

// GPU timestamp levels of a session (SPOCK_GPU_TIMESTAMPS and
// SPOCK_GPU_BLOCK_TIMESTAMPS, vk_session.cpp:2188-2218).
enum class GpuTimestamps { off = 0, per_token = 1, per_region = 2 };

class Qwen35Session {
 public:
  static constexpr std::uint32_t MAX_SEQ = 2048;  // qwen35_config.hpp: max_sequence_length_v1
  static constexpr std::size_t kStateFloats = 16u * 128u * 128u + 32u;  // + g/beta tail

  // ordered_prefill: prompt projections and chunk rule in the CPU
  // restatement's operation order (bit-identical prefill, the reference's
  // default CPU chunk path, vk_session.cpp:4840-4868); false: matrix cores.
  // gpu_timestamps: per_token records a HIP event before every decode step;
  // per_region also records one after each layer, lm_head and argmax inside
  // the step, whose kernels are then launched one by one (a recorded graph
  // holds no timing events).
  explicit Qwen35Session(const std::string& repack_dir, bool verbose = false, std::uint32_t max_seq = MAX_SEQ,
                         bool use_graph = true, bool ordered_prefill = true,
                         GpuTimestamps gpu_timestamps = GpuTimestamps::off, bool lm_head_one_launch = true,
                         bool fused_dn_step = true);
  ~Qwen35Session();
  Qwen35Session(const Qwen35Session&) = delete;
  Qwen35Session& operator=(const Qwen35Session&) = delete;

  // reset(), prefill, then max_new_tokens greedy tokens (the first from the
  // prefill logits).  Errors are thrown as std::runtime_error.
  DecodeResult decode(const std::vector<std::uint32_t>& prompt_tokens, std::uint32_t max_new_tokens);
  void reset();

  // Prefill at the current position; returns the greedy token.
  std::uint32_t prefill(const std::vector<std::uint32_t>& tokens);
  // n greedy decode steps from the last token; returns the tokens.
  std::vector<std::uint32_t> decode_steps(std::uint32_t n);

  // State exchange in compact layouts (see include/spock_model.h).
  void get_state(float* dn_state, std::uint16_t* conv, std::uint16_t* kv, std::int32_t* pos,
                 std::int32_t* last_token);
  void set_state(const float* dn_state, const std::uint16_t* conv, const std::uint16_t* kv, std::int32_t pos,
                 std::int32_t last_token);
  void last_output(std::uint16_t* logits, std::uint16_t* hidden);

  const Qwen35Shape& shape() const { return shape_; }
  std::uint32_t max_seq() const { return max_seq_; }
  std::uint32_t num_deltanet_layers() const { return n_dn_; }
  std::uint32_t num_attention_layers() const { return n_attn_; }
  hipStream_t stream() const { return stream_; }
  double last_gpu_prefill_ms() const { return last_gpu_prefill_ms_; }

 private:
  struct LayerW {
    bool attn = false;
    std::uint32_t sub = 0;  // index among layers of its kind
    const std::uint16_t *input_norm = nullptr, *post_norm = nullptr, *mlp_gate = nullptr, *mlp_up = nullptr,
                        *mlp_down = nullptr;
    const std::uint16_t *dn_qkv = nullptr, *dn_z = nullptr, *dn_a = nullptr, *dn_b = nullptr, *dn_conv = nullptr,
                        *dn_out = nullptr;
    const float* dn_norm = nullptr;
    const std::uint16_t *attn_q = nullptr, *attn_k = nullptr, *attn_v = nullptr, *attn_o = nullptr,
                        *attn_q_norm = nullptr, *attn_k_norm = nullptr;
  };

  void ensure_prefill_capacity(std::uint32_t T);
  void enqueue_decode_step();
  void ensure_graph();
  void run_decode_step();
  void ensure_ts_events(std::size_t n);
  void mark(std::size_t k);
  void lm_head_token(const std::uint16_t* h, std::uint32_t* tok, bool marks);
  float* dn_state_layer(std::uint32_t i) const { return dn_state_.get<float>() + std::size_t(i) * kStateFloats; }
  std::uint16_t* conv_layer(std::uint32_t i) const { return conv_state_.get<std::uint16_t>() + std::size_t(i) * 6144 * 4; }
  std::uint16_t* kv_layer(std::uint32_t i) const {
    return kv_cache_.get<std::uint16_t>() + std::size_t(i) * max_seq_ * 1024;
  }

  bool verbose_ = false;
  bool use_graph_ = true;
  bool ordered_prefill_ = true;
  bool lm_one_launch_ = false;  // spk_lm_head_argmax_take, else the key + take pair
  bool fused_dn_step_ = true;  // spk_deltanet_inproj_step, else the projections then the step
  Qwen35Shape shape_;
  std::uint32_t max_seq_ = MAX_SEQ;
  std::uint32_t n_dn_ = 0, n_attn_ = 0;
  hipStream_t stream_ = nullptr;
  hipGraphExec_t graph_exec_ = nullptr;
  hipGraph_t graph_ = nullptr;
  GpuTimestamps gpu_ts_ = GpuTimestamps::off;
  std::vector<hipEvent_t> ts_events_;  // timing events, reused across calls
  hipEvent_t* marks_ = nullptr;        // this step's region events (eager steps only)
  std::int32_t pos_host_ = 0;       // host mirror of the next position
  std::uint32_t history_len_ = 0;   // tokens recorded so far
  double last_gpu_prefill_ms_ = 0.0;

  DeviceBuffer weights_;
  const std::uint16_t* embed_ = nullptr;
  const std::uint16_t* final_norm_ = nullptr;
  std::vector<LayerW> layers_;

  // per-layer state
  DeviceBuffer dn_state_, conv_state_, kv_cache_, a_log_bias_, rope_;
  // decode activations
  DeviceBuffer h_, qkv_, z_, a_, b_, qg_, k_, v_, attn_out_, gate_, up_, logits_;
  DeviceBuffer attn_ws_, argmax_key_, take_slots_, dn_arrive_, tok_, pos_, history_;
  std::uint32_t history_cap_ = 0;   // token history capacity (= max_seq_: one token per position)
  // prefill activations (capacity prefill_cap_ tokens)
  std::uint32_t prefill_cap_ = 0;
  DeviceBuffer p_tokens_, p_h_, p_xn_, p_qkv_, p_z_, p_a_, p_b_, p_qhm_, p_khm_, p_vhm_, p_g_, p_beta_, p_core_,
      p_state_, p_chunk_ws_, p_gated_, p_qg_, p_k_, p_v_, p_ga_, p_up_, p_attn_ws_;
};

// RoPE table [max_seq][64] = (cos, sin) of pos * 1e7^(-2i/64), evaluated in
// double and rounded once (vk_session.cpp:332-346 evaluates it in float).
std::vector<float> rope_table(std::uint32_t max_seq);

}  // namespace spock::hip
