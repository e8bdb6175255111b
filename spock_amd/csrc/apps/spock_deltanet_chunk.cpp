// spock-deltanet-chunk (HIP) -- runs the DeltaNet chunk rule on the GPU.
//
// Same command line, JSON input and JSON output as the reference's CPU
// driver apps/spock-deltanet-chunk.cpp:40-112: `--input FILE` with
// num_heads, sequence_length, key_dim, value_dim, chunk_size (default 64),
// use_qk_l2norm (boolean, default true), query/key/value/g/beta and an
// optional initial_state (array or null); prints core_attn_out and
// final_state with 9 significant digits. Exit 2 for a missing --input,
// 1 for any error (message on stderr).
#include <exception>
#include <iomanip>
#include <iostream>
#include <string>
#include <vector>

#include "../host/deltanet_chunk_hip.hpp"
#include "../host/json_lite.hpp"

namespace {

using spock::hip::json::Value;

std::vector<float> float_array(const Value* v, const char* name) {
  if (v == nullptr || !v->is_array()) throw std::runtime_error(std::string("missing array field: ") + name);
  std::vector<float> out;
  out.reserve(v->as_array().size());
  for (const Value& e : v->as_array()) {
    if (!e.is_number()) throw std::runtime_error(std::string("non-numeric value in field: ") + name);
    out.push_back(static_cast<float>(e.as_double()));
  }
  return out;
}

void write_array(const std::vector<float>& xs) {
  std::cout << '[';
  for (std::size_t i = 0; i < xs.size(); ++i) std::cout << (i ? ", " : "") << xs[i];
  std::cout << ']';
}

}  // namespace

int main(int argc, char** argv) {
  std::string input;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--input" && i + 1 < argc) {
      input = argv[++i];
    } else if (a == "--help") {
      std::cout << "usage: spock-deltanet-chunk --input FILE\n";
      return 0;
    }
  }
  if (input.empty()) {
    std::cerr << "spock-deltanet-chunk: --input is required\n";
    return 2;
  }
  try {
    const Value root = spock::hip::json::read_file(input);
    if (!root.is_object()) throw std::runtime_error("root JSON value must be an object");
    spock::hip::DeltaNetChunkConfig cfg;
    cfg.num_heads = static_cast<std::size_t>(root.get_int("num_heads"));
    cfg.sequence_length = static_cast<std::size_t>(root.get_int("sequence_length"));
    cfg.key_dim = static_cast<std::size_t>(root.get_int("key_dim"));
    cfg.value_dim = static_cast<std::size_t>(root.get_int("value_dim"));
    cfg.chunk_size = static_cast<std::size_t>(root.get_int("chunk_size", 64));
    if (const Value* n = root.get("use_qk_l2norm")) {
      if (!n->is_bool()) throw std::runtime_error("use_qk_l2norm must be a boolean");
      cfg.use_qk_l2norm = n->as_bool();
    }
    spock::hip::DeltaNetChunkInputs in;
    in.query = float_array(root.get("query"), "query");
    in.key = float_array(root.get("key"), "key");
    in.value = float_array(root.get("value"), "value");
    in.g = float_array(root.get("g"), "g");
    in.beta = float_array(root.get("beta"), "beta");
    if (const Value* s = root.get("initial_state"); s != nullptr && !s->is_null())
      in.initial_state = float_array(s, "initial_state");

    const auto out = spock::hip::run_deltanet_chunk_rule(cfg, in);
    std::cout << std::setprecision(9) << "{\n  \"core_attn_out\": ";
    write_array(out.core_attn_out);
    std::cout << ",\n  \"final_state\": ";
    write_array(out.final_state);
    std::cout << "\n}\n";
  } catch (const std::exception& e) {
    std::cerr << "spock-deltanet-chunk: " << e.what() << "\n";
    return 1;
  }
  return 0;
}
