// deltanet_chunk_hip.cpp -- see deltanet_chunk_hip.hpp.
#include "deltanet_chunk_hip.hpp"

#include <cmath>
#include <stdexcept>
#include <string>

#include "hip_buffer.hpp"

namespace spock::hip {

namespace {

constexpr std::size_t kDim = 128;

void check_size(const std::vector<float>& v, std::size_t expected, const char* name) {
  if (v.size() != expected) {
    throw std::runtime_error(std::string(name) + " size mismatch: expected " +
                             std::to_string(expected) + ", got " + std::to_string(v.size()));
  }
}

// [H][T][w] -> [H][T][128] with zero columns beyond w.
std::vector<float> pad_rows(const std::vector<float>& src, std::size_t rows, std::size_t w) {
  if (w == kDim) return src;
  std::vector<float> out(rows * kDim, 0.0f);
  for (std::size_t r = 0; r < rows; ++r)
    for (std::size_t d = 0; d < w; ++d) out[r * kDim + d] = src[r * w + d];
  return out;
}

}  // namespace

DeltaNetChunkOutputs run_deltanet_chunk_rule(const DeltaNetChunkConfig& config,
                                             const DeltaNetChunkInputs& inputs) {
  if (config.num_heads == 0 || config.sequence_length == 0 || config.key_dim == 0 ||
      config.value_dim == 0 || config.chunk_size == 0) {
    throw std::runtime_error("DeltaNet chunk config fields must be non-zero");
  }
  const std::size_t H = config.num_heads, T = config.sequence_length;
  const std::size_t dk = config.key_dim, dv = config.value_dim;
  check_size(inputs.query, H * T * dk, "query");
  check_size(inputs.key, H * T * dk, "key");
  check_size(inputs.value, H * T * dv, "value");
  check_size(inputs.g, H * T, "g");
  check_size(inputs.beta, H * T, "beta");
  if (!inputs.initial_state.empty()) check_size(inputs.initial_state, H * dk * dv, "initial_state");
  if (dk > kDim || dv > kDim) {
    throw std::runtime_error("key_dim and value_dim must be at most 128 on this device path");
  }

  const std::vector<float> q = pad_rows(inputs.query, H * T, dk);
  const std::vector<float> k = pad_rows(inputs.key, H * T, dk);
  const std::vector<float> v = pad_rows(inputs.value, H * T, dv);
  std::vector<float> init;
  if (!inputs.initial_state.empty()) {
    init.assign(H * kDim * kDim, 0.0f);
    for (std::size_t h = 0; h < H; ++h)
      for (std::size_t i = 0; i < dk; ++i)
        for (std::size_t j = 0; j < dv; ++j)
          init[(h * kDim + i) * kDim + j] = inputs.initial_state[(h * dk + i) * dv + j];
  }

  const std::size_t qkv_bytes = H * T * kDim * sizeof(float);
  DeviceBuffer dq(qkv_bytes), dk_(qkv_bytes), dv_(qkv_bytes);
  DeviceBuffer dg(H * T * sizeof(float)), db(H * T * sizeof(float));
  DeviceBuffer dinit(init.size() * sizeof(float));
  DeviceBuffer dcore(qkv_bytes), dstate(H * kDim * kDim * sizeof(float));
  const std::size_t ws_bytes = spk_chunk_prefill_workspace_size(
      static_cast<int32_t>(H), static_cast<int32_t>(T), 1, 64);
  DeviceBuffer dws(ws_bytes);
  dq.upload(q.data(), qkv_bytes);
  dk_.upload(k.data(), qkv_bytes);
  dv_.upload(v.data(), qkv_bytes);
  dg.upload(inputs.g.data(), H * T * sizeof(float));
  db.upload(inputs.beta.data(), H * T * sizeof(float));
  if (!init.empty()) dinit.upload(init.data(), init.size() * sizeof(float));

  SpkChunkArgs a{};
  a.num_heads = static_cast<int32_t>(H);
  a.total_tokens = static_cast<int32_t>(T);
  a.key_dim = a.value_dim = static_cast<int32_t>(kDim);
  a.chunk_size = 64;  // config.chunk_size only changes rounding (deltanet_chunk_hip.hpp)
  a.use_qk_l2norm = config.use_qk_l2norm ? 1 : 0;
  a.q_scale = 1.0f / std::sqrt(static_cast<float>(dk));  // deltanet_chunk.cpp:87
  a.input_dtype = SPK_F32;
  a.q = dq.get();
  a.k = dk_.get();
  a.v = dv_.get();
  a.g = dg.get<float>();
  a.beta = db.get<float>();
  a.initial_state = init.empty() ? nullptr : dinit.get<float>();
  a.out_core = dcore.get<float>();
  a.out_state = dstate.get<float>();
  a.num_seqs = 1;
  a.workspace = dws.get();
  a.workspace_bytes = ws_bytes;
  spk_check(spk_chunk_prefill(&a, nullptr), "spk_chunk_prefill");
  hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");

  std::vector<float> core(H * T * kDim), state(H * kDim * kDim);
  dcore.download(core.data(), qkv_bytes);
  dstate.download(state.data(), state.size() * sizeof(float));
  DeltaNetChunkOutputs out;
  out.core_attn_out.resize(H * T * dv);
  out.final_state.resize(H * dk * dv);
  for (std::size_t r = 0; r < H * T; ++r)
    for (std::size_t d = 0; d < dv; ++d) out.core_attn_out[r * dv + d] = core[r * kDim + d];
  for (std::size_t h = 0; h < H; ++h)
    for (std::size_t i = 0; i < dk; ++i)
      for (std::size_t j = 0; j < dv; ++j)
        out.final_state[(h * dk + i) * dv + j] = state[(h * kDim + i) * kDim + j];
  return out;
}

}  // namespace spock::hip
