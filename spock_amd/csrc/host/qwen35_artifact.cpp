// qwen35_artifact.cpp -- repacked text-weight artifact reader and the seeded
// synthetic writer (see qwen35_artifact.hpp).
#include "qwen35_artifact.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <thread>

#include "json_lite.hpp"

namespace spock::hip {

namespace {

constexpr std::uint64_t kAlign = 256;
constexpr double kPi = 3.141592653589793;  // the double nearest pi (numpy's np.pi)
constexpr const char* kLmPrefix = "model.language_model.";

std::uint64_t align_up(std::uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

enum class Dist { Normal002, Normal01, Uniform11, Ones };

struct PlanEntry {
  TensorInfo info;
  Dist dist;
};

void add(std::vector<PlanEntry>& plan, std::uint64_t& off, const std::string& role, const std::string& name,
         std::vector<std::size_t> shape, const char* dtype, Dist dist) {
  std::size_t n = 1;
  for (auto d : shape) n *= d;
  PlanEntry e;
  e.info.role_path = role;
  e.info.name = name;
  e.info.shape = std::move(shape);
  e.info.dtype = dtype;
  e.info.nbytes = n * (std::strcmp(dtype, "fp32") == 0 ? 4 : 2);
  off = align_up(off);
  e.info.offset = off;
  off += e.info.nbytes;
  e.dist = dist;
  plan.push_back(std::move(e));
}

// Tensor list of tools/plan_text_artifact.py:16-45 (roles) with the repack
// dtypes of tools/repack_text_weights.py:63-80, in file order.
std::vector<PlanEntry> build_plan(const Qwen35Shape& s) {
  using S = Qwen35Shape;
  std::vector<PlanEntry> plan;
  std::uint64_t off = 0;
  add(plan, off, "global.token_embedding", std::string(kLmPrefix) + "embed_tokens.weight", {s.vocab, S::HIDDEN},
      "fp16", Dist::Normal002);
  for (std::uint32_t L = 0; L < s.layers; ++L) {
    const std::string role = "layer." + std::to_string(L) + ".";
    const std::string name = std::string(kLmPrefix) + "layers." + std::to_string(L) + ".";
    add(plan, off, role + "input_norm", name + "input_layernorm.weight", {S::HIDDEN}, "fp16", Dist::Normal002);
    add(plan, off, role + "post_norm", name + "post_attention_layernorm.weight", {S::HIDDEN}, "fp16",
        Dist::Normal002);
    if (S::is_attention(L)) {
      add(plan, off, role + "attn_q", name + "self_attn.q_proj.weight", {S::Q_HEADS * S::HEAD_DIM * 2, S::HIDDEN},
          "fp16", Dist::Normal002);
      add(plan, off, role + "attn_k", name + "self_attn.k_proj.weight", {S::KV_HEADS * S::HEAD_DIM, S::HIDDEN},
          "fp16", Dist::Normal002);
      add(plan, off, role + "attn_v", name + "self_attn.v_proj.weight", {S::KV_HEADS * S::HEAD_DIM, S::HIDDEN},
          "fp16", Dist::Normal002);
      add(plan, off, role + "attn_o", name + "self_attn.o_proj.weight", {S::HIDDEN, S::Q_HEADS * S::HEAD_DIM},
          "fp16", Dist::Normal002);
      add(plan, off, role + "attn_q_norm", name + "self_attn.q_norm.weight", {S::HEAD_DIM}, "fp16", Dist::Normal002);
      add(plan, off, role + "attn_k_norm", name + "self_attn.k_norm.weight", {S::HEAD_DIM}, "fp16", Dist::Normal002);
    } else {
      add(plan, off, role + "delta_a_log", name + "linear_attn.A_log", {S::DN_HEADS}, "fp32", Dist::Uniform11);
      add(plan, off, role + "delta_dt_bias", name + "linear_attn.dt_bias", {S::DN_HEADS}, "fp16", Dist::Normal01);
      add(plan, off, role + "delta_conv", name + "linear_attn.conv1d.weight", {S::DN_CONV_DIM, 1, S::DN_CONV_KS},
          "fp16", Dist::Normal002);
      add(plan, off, role + "delta_in_proj_a", name + "linear_attn.in_proj_a.weight", {S::DN_HEADS, S::HIDDEN},
          "fp16", Dist::Normal002);
      add(plan, off, role + "delta_in_proj_b", name + "linear_attn.in_proj_b.weight", {S::DN_HEADS, S::HIDDEN},
          "fp16", Dist::Normal002);
      add(plan, off, role + "delta_in_proj_qkv", name + "linear_attn.in_proj_qkv.weight",
          {S::DN_CONV_DIM, S::HIDDEN}, "fp16", Dist::Normal002);
      add(plan, off, role + "delta_in_proj_z", name + "linear_attn.in_proj_z.weight",
          {S::DN_HEADS * S::DN_DIM, S::HIDDEN}, "fp16", Dist::Normal002);
      add(plan, off, role + "delta_norm", name + "linear_attn.norm.weight", {S::DN_DIM}, "fp32", Dist::Ones);
      add(plan, off, role + "delta_out_proj", name + "linear_attn.out_proj.weight",
          {S::HIDDEN, S::DN_HEADS * S::DN_DIM}, "fp16", Dist::Normal002);
    }
    add(plan, off, role + "mlp_gate", name + "mlp.gate_proj.weight", {S::INTER, S::HIDDEN}, "fp16", Dist::Normal002);
    add(plan, off, role + "mlp_up", name + "mlp.up_proj.weight", {S::INTER, S::HIDDEN}, "fp16", Dist::Normal002);
    add(plan, off, role + "mlp_down", name + "mlp.down_proj.weight", {S::HIDDEN, S::INTER}, "fp16", Dist::Normal002);
  }
  add(plan, off, "global.final_norm", std::string(kLmPrefix) + "norm.weight", {S::HIDDEN}, "fp16", Dist::Normal002);
  return plan;
}

// ---- seeded generator (identical to spock_amd/synth.py) -------------------

inline std::uint64_t splitmix64_at(std::uint64_t seed, std::uint64_t i) {
  std::uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline double unit53(std::uint64_t z) { return static_cast<double>(z >> 11) * (1.0 / 9007199254740992.0); }

inline std::uint16_t f32_to_f16_rne(float f) {
  std::uint32_t x;
  std::memcpy(&x, &f, 4);
  const std::uint32_t sign = (x >> 16) & 0x8000u;
  std::uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return static_cast<std::uint16_t>(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return static_cast<std::uint16_t>(sign | 0x7c00u);  // rounds to >= 65520: inf
  if (ax < 0x38800000u) {  // fp16 subnormal or zero: round |x| * 2^24 to an integer, ties to even
    float a;
    std::memcpy(&a, &ax, 4);
    const float scaled = a * 16777216.0f;  // exact (power of two)
    const float r = std::nearbyint(scaled);
    return static_cast<std::uint16_t>(sign | static_cast<std::uint32_t>(r));
  }
  const std::uint32_t mant = ax & 0x7fffffu;
  const std::uint32_t exp = (ax >> 23) - 127 + 15;
  std::uint32_t h = (exp << 10) | (mant >> 13);
  const std::uint32_t rest = mant & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
  return static_cast<std::uint16_t>(sign | h);
}

// Values [i0, i1) of one tensor; i0 even.
void gen_range(Dist dist, std::uint64_t seed, bool fp32, std::size_t i0, std::size_t i1, std::uint8_t* dst) {
  auto put = [&](std::size_t i, float v) {
    if (fp32)
      std::memcpy(dst + 4 * i, &v, 4);
    else {
      const std::uint16_t h = f32_to_f16_rne(v);
      std::memcpy(dst + 2 * i, &h, 2);
    }
  };
  switch (dist) {
    case Dist::Ones:
      for (std::size_t i = i0; i < i1; ++i) put(i, 1.0f);
      return;
    case Dist::Uniform11:
      for (std::size_t i = i0; i < i1; ++i) put(i, static_cast<float>(-1.0 + unit53(splitmix64_at(seed, i)) * 2.0));
      return;
    case Dist::Normal002:
    case Dist::Normal01: {
      const double stdv = dist == Dist::Normal002 ? 0.02 : 0.1;
      for (std::size_t i = i0; i < i1; i += 2) {
        const double u1 = 1.0 - unit53(splitmix64_at(seed, i));
        const double u2 = unit53(splitmix64_at(seed, i + 1));
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double a = 2.0 * kPi * u2;
        put(i, static_cast<float>(0.0 + stdv * (r * std::cos(a))));
        if (i + 1 < i1) put(i + 1, static_cast<float>(0.0 + stdv * (r * std::sin(a))));
      }
      return;
    }
  }
}

}  // namespace

std::uint32_t Qwen35Shape::num_attention_layers() const {
  std::uint32_t n = 0;
  for (std::uint32_t L = 0; L < layers; ++L) n += is_attention(L) ? 1 : 0;
  return n;
}

std::uint64_t tensor_seed(std::uint64_t seed, std::size_t index) { return seed * 65536ull + index; }

std::vector<TensorInfo> qwen35_tensor_plan(const Qwen35Shape& shape) {
  std::vector<TensorInfo> out;
  for (auto& e : build_plan(shape)) out.push_back(e.info);
  return out;
}

void fill_synthetic_weights(const Qwen35Shape& shape, std::uint64_t seed, std::vector<std::uint8_t>& out) {
  if (shape.layers == 0 || shape.layers > 64 || shape.vocab == 0)
    throw std::runtime_error("synthetic artifact: layers must be in [1, 64] and vocab > 0");
  const auto plan = build_plan(shape);
  const std::uint64_t total = plan.back().info.offset + plan.back().info.nbytes;
  out.assign(total, 0);
  // Work items of at most 1 Mi values, spread over the host threads.
  struct Item { std::size_t t; std::size_t i0, i1; };
  std::vector<Item> items;
  for (std::size_t t = 0; t < plan.size(); ++t) {
    const std::size_t n = plan[t].info.nbytes / (plan[t].info.dtype == "fp32" ? 4 : 2);
    for (std::size_t i0 = 0; i0 < n; i0 += (1u << 20)) items.push_back({t, i0, std::min(n, i0 + (1u << 20))});
  }
  const unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::vector<std::thread> pool;
  std::atomic<std::size_t> next{0};
  for (unsigned w = 0; w < nt; ++w)
    pool.emplace_back([&] {
      for (std::size_t k = next++; k < items.size(); k = next++) {
        const Item& it = items[k];
        const PlanEntry& e = plan[it.t];
        gen_range(e.dist, tensor_seed(seed, it.t), e.info.dtype == "fp32", it.i0, it.i1, out.data() + e.info.offset);
      }
    });
  for (auto& th : pool) th.join();
}

void write_synthetic_artifact(const std::string& dir, const Qwen35Shape& shape, std::uint64_t seed) {
  namespace fs = std::filesystem;
  fs::create_directories(dir);
  std::vector<std::uint8_t> bytes;
  fill_synthetic_weights(shape, seed, bytes);
  const auto plan = qwen35_tensor_plan(shape);
  {
    std::ofstream f(fs::path(dir) / "text_weights.bin", std::ios::binary | std::ios::trunc);
    f.write(reinterpret_cast<const char*>(bytes.data()), static_cast<std::streamsize>(bytes.size()));
    if (!f) throw std::runtime_error("synthetic artifact: cannot write " + dir + "/text_weights.bin");
  }
  std::ostringstream js;
  js << "{\n  \"format\": \"spock-text-repack\",\n  \"artifact_format_version\": 1,\n"
     << "  \"model_id\": \"Qwen/Qwen3.5-0.8B-shaped synthetic\",\n"
     << "  \"synthetic\": {\"seed\": " << seed << ", \"generator\": \"splitmix64-box-muller\"},\n"
     << "  \"model\": {\"layers\": " << shape.layers << ", \"vocab\": " << shape.vocab << "},\n"
     << "  \"alignment\": " << kAlign << ",\n  \"total_bytes\": " << bytes.size() << ",\n  \"tensors\": [\n";
  for (std::size_t i = 0; i < plan.size(); ++i) {
    const TensorInfo& t = plan[i];
    js << "    {\"role_path\": \"" << t.role_path << "\", \"name\": \"" << t.name << "\", \"offset\": " << t.offset
       << ", \"nbytes\": " << t.nbytes << ", \"dtype\": \"" << t.dtype << "\", \"shape\": [";
    for (std::size_t d = 0; d < t.shape.size(); ++d) js << (d ? ", " : "") << t.shape[d];
    js << "]}" << (i + 1 < plan.size() ? "," : "") << "\n";
  }
  js << "  ]\n}\n";
  std::ofstream m(fs::path(dir) / "text_repack_manifest.json", std::ios::trunc);
  m << js.str();
  if (!m) throw std::runtime_error("synthetic artifact: cannot write " + dir + "/text_repack_manifest.json");
}

// ---- reader -----------------------------------------------------------------

WeightArtifact WeightArtifact::load(const std::string& repack_dir) {
  namespace fs = std::filesystem;
  const auto root = json::read_file((fs::path(repack_dir) / "text_repack_manifest.json").string());
  WeightArtifact a;
  a.bin_path_ = (fs::path(repack_dir) / "text_weights.bin").string();
  const json::Value* arr = root.get("tensors");
  if (!arr || !arr->is_array()) throw std::runtime_error("text_repack_manifest.json: no \"tensors\" list");
  for (const auto& e : arr->as_array()) {
    TensorInfo t;
    t.role_path = e.get_string("role_path");
    t.name = e.get_string("name");
    t.offset = static_cast<std::uint64_t>(e.get_int("offset"));
    t.nbytes = static_cast<std::uint64_t>(e.get_int("nbytes"));
    t.dtype = e.get_string("dtype");
    if (const json::Value* sh = e.get("shape"); sh && sh->is_array())
      for (const auto& d : sh->as_array()) t.shape.push_back(static_cast<std::size_t>(d.as_double()));
    const std::size_t idx = a.entries_.size();
    a.by_name_[t.name] = idx;
    a.by_role_[t.role_path] = idx;
    a.extent_ = std::max<std::size_t>(a.extent_, t.offset + t.nbytes);
    a.entries_.push_back(std::move(t));
  }
  if (const json::Value* md = root.get("model"); md && md->is_object()) {
    a.shape_.layers = static_cast<std::uint32_t>(md->get_int("layers"));
    a.shape_.vocab = static_cast<std::uint32_t>(md->get_int("vocab"));
  } else {
    a.shape_.layers = 0;
    while (a.find_by_role("layer." + std::to_string(a.shape_.layers) + ".input_norm")) ++a.shape_.layers;
    a.shape_.vocab = static_cast<std::uint32_t>(a.token_embedding().shape.at(0));
  }
  const int fd = ::open(a.bin_path_.c_str(), O_RDONLY);
  if (fd < 0) throw std::runtime_error("cannot open " + a.bin_path_);
  struct stat sb {};
  if (::fstat(fd, &sb) != 0) {
    ::close(fd);
    throw std::runtime_error("cannot stat " + a.bin_path_);
  }
  if (static_cast<std::size_t>(sb.st_size) < a.extent_) {
    ::close(fd);
    throw std::runtime_error("text_weights.bin is shorter than the manifest's tensor extent");
  }
  a.map_bytes_ = static_cast<std::size_t>(sb.st_size);
  a.map_ = ::mmap(nullptr, a.map_bytes_, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (a.map_ == MAP_FAILED) {
    a.map_ = nullptr;
    throw std::runtime_error("cannot map " + a.bin_path_);
  }
  return a;
}

WeightArtifact::~WeightArtifact() {
  if (map_) ::munmap(map_, map_bytes_);
}

WeightArtifact::WeightArtifact(WeightArtifact&& o) noexcept { *this = std::move(o); }

WeightArtifact& WeightArtifact::operator=(WeightArtifact&& o) noexcept {
  if (this != &o) {
    if (map_) ::munmap(map_, map_bytes_);
    entries_ = std::move(o.entries_);
    by_name_ = std::move(o.by_name_);
    by_role_ = std::move(o.by_role_);
    bin_path_ = std::move(o.bin_path_);
    extent_ = o.extent_;
    map_ = o.map_;
    map_bytes_ = o.map_bytes_;
    shape_ = o.shape_;
    o.map_ = nullptr;
    o.map_bytes_ = 0;
  }
  return *this;
}

const TensorInfo* WeightArtifact::find_by_role(const std::string& role_path) const {
  auto it = by_role_.find(role_path);
  return it == by_role_.end() ? nullptr : &entries_[it->second];
}

const TensorInfo* WeightArtifact::find_by_name(const std::string& name) const {
  auto it = by_name_.find(name);
  return it == by_name_.end() ? nullptr : &entries_[it->second];
}

const TensorInfo* WeightArtifact::find_by_state_dict_key(const std::string& key) const {
  if (key.rfind("model.layers.", 0) == 0) return find_by_name(std::string(kLmPrefix) + key.substr(6));
  return find_by_name(key);
}

const TensorInfo& WeightArtifact::require(const std::string& role_path) const {
  const TensorInfo* t = find_by_role(role_path);
  if (!t) throw std::runtime_error("artifact has no entry for role " + role_path);
  return *t;
}

const TensorInfo& WeightArtifact::token_embedding() const {
  const TensorInfo* t = find_by_role("global.token_embedding");
  if (!t) throw std::runtime_error("artifact has no global.token_embedding entry");
  return *t;
}

const TensorInfo& WeightArtifact::final_norm() const {
  const TensorInfo* t = find_by_role("global.final_norm");
  if (!t) throw std::runtime_error("artifact has no global.final_norm entry");
  return *t;
}

const void* WeightArtifact::data(const TensorInfo& t) const {
  if (!map_ || t.offset + t.nbytes > map_bytes_) throw std::runtime_error("tensor outside the mapped weights");
  return static_cast<const std::uint8_t*>(map_) + t.offset;
}

}  // namespace spock::hip
