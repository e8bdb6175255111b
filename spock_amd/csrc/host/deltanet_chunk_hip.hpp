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
// value dims give zero outputs, the q scale stays 1/sqrt(key_dim)).
//
// chunk_size: validated (non-zero, as the reference requires) and then
// replaced by the kernels' fixed 64-token blocking.  The chunk rule equals the
// token recurrence for every chunk size, so this changes only fp32 rounding:
// a call with chunk_size C returns exactly what the same call with 64 returns,
// which is within 1e-5 of the reference rule at C (checked on the reference's
// own unit case, C = 4).  Callers that need the reference's rounding order
// for another C have no GPU path here.
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
