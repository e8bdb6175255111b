// deltanet_chunk_hip.hpp -- the reference's CPU chunk-rule interface, served
// by the MI355X kernels.
//
// Same names, fields, value semantics and errors as
// src/runtime/deltanet_chunk.hpp:8-40 (spock::runtime::run_deltanet_chunk_rule):
// inputs [head][token][dim], g/beta [head][token], optional initial state
// [head][key][value]; outputs core_attn_out [head][token][value] and
// final_state; std::runtime_error for a zero config field or a size mismatch.
// The device kernels work on 128-wide heads and 64-token chunks: narrower
// heads are zero-padded (zero key dims change no dot product or norm, zero
// value dims give zero outputs, the q scale stays 1/sqrt(key_dim)), and the
// chunk size is the kernel's blocking -- the chunk rule's result equals the
// token recurrence for every chunk size, up to fp32 rounding.
#pragma once

#include <cstddef>
#include <vector>

namespace spock::hip {

struct DeltaNetChunkConfig {
  std::size_t num_heads = 0;
  std::size_t sequence_length = 0;
  std::size_t key_dim = 0;
  std::size_t value_dim = 0;
  std::size_t chunk_size = 64;
  bool use_qk_l2norm = true;
};

struct DeltaNetChunkInputs {
  std::vector<float> query;   // [head][token][key_dim]
  std::vector<float> key;     // [head][token][key_dim]
  std::vector<float> value;   // [head][token][value_dim]
  std::vector<float> g;       // [head][token]
  std::vector<float> beta;    // [head][token]
  std::vector<float> initial_state;  // [head][key_dim][value_dim] or empty (zeros)
};

struct DeltaNetChunkOutputs {
  std::vector<float> core_attn_out;  // [head][token][value_dim]
  std::vector<float> final_state;    // [head][key_dim][value_dim]
};

// Runs spk_chunk_prefill on the current device (blocking, default stream).
DeltaNetChunkOutputs run_deltanet_chunk_rule(const DeltaNetChunkConfig& config,
                                             const DeltaNetChunkInputs& inputs);

}  // namespace spock::hip
