// spock-deltanet-chunk (HIP) -- the chunk rule on the GPU behind the command
// line of the reference's CPU driver (apps/spock-deltanet-chunk.cpp:40-112).
//
// Kept from that driver, because callers script against it:
//   `--input FILE` (exit 2 when absent; other arguments are ignored), `--help`
//   (exit 0), a JSON object with num_heads,
//   sequence_length, key_dim, value_dim, chunk_size (default 64),
//   use_qk_l2norm (boolean, default true), query/key/value/g/beta arrays and an
//   optional initial_state (array or null); stdout is a JSON object with
//   core_attn_out and final_state at 9 significant digits; exit 1 on any error
//   with the message on stderr.
//
// Design: the request is described by two tables (integer fields of
// DeltaNetChunkConfig, tensor fields of DeltaNetChunkInputs) that one loader
// walks, so the accepted schema is visible in one place; the response is
// formatted into one buffer and written with a single call.
#include <cmath>
#include <cstdio>
#include <exception>
#include <stdexcept>
#include <string>
#include <vector>

#include "../host/deltanet_chunk_hip.hpp"
#include "../host/json_lite.hpp"

namespace {

namespace json = spock::hip::json;
using Config = spock::hip::DeltaNetChunkConfig;
using Inputs = spock::hip::DeltaNetChunkInputs;

constexpr const char* kTool = "spock-deltanet-chunk";

struct IntegerField {
  const char* key;
  std::size_t Config::*slot;
  bool required;
  std::size_t fallback;
};

constexpr IntegerField kIntegerFields[] = {
    {"num_heads", &Config::num_heads, true, 0},
    {"sequence_length", &Config::sequence_length, true, 0},
    {"key_dim", &Config::key_dim, true, 0},
    {"value_dim", &Config::value_dim, true, 0},
    {"chunk_size", &Config::chunk_size, false, 64},
};

struct TensorField {
  const char* key;
  std::vector<float> Inputs::*slot;
  bool optional;  // absent or null leaves the vector empty
};

constexpr TensorField kTensorFields[] = {
    {"query", &Inputs::query, false},   {"key", &Inputs::key, false},
    {"value", &Inputs::value, false},   {"g", &Inputs::g, false},
    {"beta", &Inputs::beta, false},     {"initial_state", &Inputs::initial_state, true},
};

[[noreturn]] void reject(const char* key, const std::string& what) {
  throw std::runtime_error(std::string("field \"") + key + "\": " + what);
}

std::size_t read_count(const json::Value& root, const IntegerField& f) {
  const json::Value* v = root.get(f.key);
  if (v == nullptr) {
    if (f.required) reject(f.key, "required integer is missing");
    return f.fallback;
  }
  if (!v->is_number()) reject(f.key, "expected an integer");
  const double d = v->as_double();
  if (!(d >= 0.0) || std::floor(d) != d || d > 9.0e15) reject(f.key, "expected a non-negative integer");
  return static_cast<std::size_t>(d);
}

void read_tensor(const json::Value& root, const TensorField& f, std::vector<float>& out) {
  const json::Value* v = root.get(f.key);
  if (v == nullptr || v->is_null()) {
    if (!f.optional) reject(f.key, "required array of numbers is missing");
    return;
  }
  if (!v->is_array()) reject(f.key, "expected an array of numbers");
  const auto& elems = v->as_array();
  out.resize(elems.size());
  for (std::size_t i = 0; i < elems.size(); ++i) {
    if (!elems[i].is_number()) reject(f.key, "element " + std::to_string(i) + " is not a number");
    out[i] = static_cast<float>(elems[i].as_double());
  }
}

void load_request(const json::Value& root, Config& cfg, Inputs& in) {
  if (!root.is_object()) throw std::runtime_error("input: the top-level JSON value is not an object");
  for (const auto& f : kIntegerFields) cfg.*(f.slot) = read_count(root, f);
  if (const json::Value* flag = root.get("use_qk_l2norm")) {
    if (!flag->is_bool()) reject("use_qk_l2norm", "expected true or false");
    cfg.use_qk_l2norm = flag->as_bool();
  }
  for (const auto& f : kTensorFields) read_tensor(root, f, in.*(f.slot));
}

void append_tensor(std::string& buf, const char* key, const std::vector<float>& xs, bool last) {
  buf += "  \"";
  buf += key;
  buf += "\": [";
  char num[32];
  for (std::size_t i = 0; i < xs.size(); ++i) {
    const int n = std::snprintf(num, sizeof num, i ? ", %.9g" : "%.9g", static_cast<double>(xs[i]));
    buf.append(num, static_cast<std::size_t>(n));
  }
  buf += last ? "]\n" : "],\n";
}

int usage_error(const std::string& msg) {
  std::fprintf(stderr, "%s: %s\nusage: %s --input FILE\n", kTool, msg.c_str(), kTool);
  return 2;
}

}  // namespace

int main(int argc, char** argv) {
  std::string path;
  // As the reference driver does, arguments other than --help and
  // "--input FILE" are ignored, and a trailing --input without a FILE counts
  // as no input.
  for (int i = 1; i < argc; ++i) {
    const std::string arg = argv[i];
    if (arg == "--help") {
      std::printf("usage: %s --input FILE\n", kTool);
      return 0;
    }
    if (arg == "--input" && i + 1 < argc) path = argv[++i];
  }
  if (path.empty()) return usage_error("--input is required");

  try {
    Config cfg;
    Inputs in;
    load_request(json::read_file(path), cfg, in);
    const auto out = spock::hip::run_deltanet_chunk_rule(cfg, in);
    std::string buf = "{\n";
    buf.reserve(16 * (out.core_attn_out.size() + out.final_state.size()) + 64);
    append_tensor(buf, "core_attn_out", out.core_attn_out, false);
    append_tensor(buf, "final_state", out.final_state, true);
    buf += "}\n";
    std::fwrite(buf.data(), 1, buf.size(), stdout);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "%s: %s\n", kTool, e.what());
    return 1;
  }
  return 0;
}
