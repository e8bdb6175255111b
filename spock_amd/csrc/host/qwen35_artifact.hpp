// qwen35_artifact.hpp -- the repacked text-weight artifact of the reference
// (text_repack_manifest.json + text_weights.bin) and a seeded synthetic
// writer for Qwen3.5-0.8B-shaped random-init models.
//
// Reader: the reference's WeightArtifact (src/runtime/weight_loader.hpp:22-54,
// weight_loader.cpp:23-98): tensors {role_path, name, offset, nbytes, dtype,
// shape}, lookup by role ("layer.N.delta_in_proj_qkv", "global.token_embedding"),
// by manifest name, or by state-dict key.  Roles follow
// tools/plan_text_artifact.py:16-45; dtypes follow tools/repack_text_weights.py
// (fp16 except delta_a_log and delta_norm, which stay fp32; 256-byte aligned
// offsets).  The file is memory-mapped rather than read per tensor.
//
// Writer: every tensor of the model with values from SplitMix64 -> Box-Muller
// (double) -> fp32 -> fp16 (RNE), one seed per tensor; projections, embedding,
// conv and RMSNorm weights ~ N(0, 0.02) (RMSNorms are applied as 1 + w),
// A_log ~ U(-1, 1), dt_bias ~ N(0, 0.1), the gated-norm weight = 1 (its HF
// initialisation, modeling_qwen3_5.py:171).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace spock::hip {

// Qwen3.5-0.8B text model shape (src/model/qwen35_config.hpp:15-30,
// vk_session.hpp:383-401).  Layers and vocabulary may be reduced for tests;
// every other dimension is fixed by the kernels.
struct Qwen35Shape {
  static constexpr std::uint32_t HIDDEN = 1024;
  static constexpr std::uint32_t INTER = 3584;
  static constexpr std::uint32_t Q_HEADS = 8;
  static constexpr std::uint32_t KV_HEADS = 2;
  static constexpr std::uint32_t HEAD_DIM = 256;
  static constexpr std::uint32_t ROTARY_DIM = 64;
  static constexpr std::uint32_t DN_HEADS = 16;
  static constexpr std::uint32_t DN_DIM = 128;
  static constexpr std::uint32_t DN_CONV_DIM = 6144;
  static constexpr std::uint32_t DN_CONV_KS = 4;
  static constexpr std::uint32_t FULL_VOCAB = 248320;
  static constexpr std::uint32_t FULL_LAYERS = 24;

  std::uint32_t layers = FULL_LAYERS;
  std::uint32_t vocab = FULL_VOCAB;

  // qwen35_config.cpp:7-15: every fourth layer is full attention.
  static bool is_attention(std::uint32_t layer) { return layer % 4 == 3; }
  std::uint32_t num_attention_layers() const;
  std::uint32_t num_deltanet_layers() const { return layers - num_attention_layers(); }
};

struct TensorInfo {
  std::string role_path;  // "layer.0.input_norm", "global.token_embedding"
  std::string name;       // "model.language_model.layers.0.input_layernorm.weight"
  std::uint64_t offset = 0;
  std::uint64_t nbytes = 0;
  std::string dtype;      // "fp16" or "fp32"
  std::vector<std::size_t> shape;
};

class WeightArtifact {
 public:
  // Reads <dir>/text_repack_manifest.json and maps <dir>/text_weights.bin.
  static WeightArtifact load(const std::string& repack_dir);

  WeightArtifact() = default;
  ~WeightArtifact();
  WeightArtifact(WeightArtifact&& o) noexcept;
  WeightArtifact& operator=(WeightArtifact&& o) noexcept;
  WeightArtifact(const WeightArtifact&) = delete;
  WeightArtifact& operator=(const WeightArtifact&) = delete;

  const TensorInfo* find_by_role(const std::string& role_path) const;
  const TensorInfo* find_by_name(const std::string& name) const;
  // "model.layers.X.Y" -> "model.language_model.layers.X.Y" (weight_loader.cpp:64-74)
  const TensorInfo* find_by_state_dict_key(const std::string& key) const;
  const TensorInfo& token_embedding() const;
  const TensorInfo& final_norm() const;
  // Role lookup that throws std::runtime_error naming the role when absent.
  const TensorInfo& require(const std::string& role_path) const;

  const std::string& weights_file_path() const { return bin_path_; }
  const std::vector<TensorInfo>& tensors() const { return entries_; }
  std::size_t total_bytes() const { return extent_; }
  std::size_t tensor_count() const { return entries_.size(); }
  // Mapped bytes of one tensor (valid while the artifact lives).
  const void* data(const TensorInfo& t) const;
  const void* mapped() const { return map_; }
  std::size_t mapped_bytes() const { return map_bytes_; }
  // Model shape recorded in the manifest ("model": {"layers", "vocab"}).
  Qwen35Shape shape() const { return shape_; }

 private:
  std::vector<TensorInfo> entries_;
  std::unordered_map<std::string, std::size_t> by_name_;
  std::unordered_map<std::string, std::size_t> by_role_;
  std::string bin_path_;
  std::size_t extent_ = 0;
  void* map_ = nullptr;
  std::size_t map_bytes_ = 0;
  Qwen35Shape shape_;
};

// The artifact's tensor list for `shape` in file order with 256-byte aligned
// offsets (no data).
std::vector<TensorInfo> qwen35_tensor_plan(const Qwen35Shape& shape);

// Fills `out` (plan total bytes) with the seeded synthetic weights.
void fill_synthetic_weights(const Qwen35Shape& shape, std::uint64_t seed, std::vector<std::uint8_t>& out);

// Writes <dir>/text_repack_manifest.json and <dir>/text_weights.bin.
void write_synthetic_artifact(const std::string& dir, const Qwen35Shape& shape, std::uint64_t seed);

// Per-tensor seed of tensor `index` of an artifact with base seed `seed`.
std::uint64_t tensor_seed(std::uint64_t seed, std::size_t index);

}  // namespace spock::hip
