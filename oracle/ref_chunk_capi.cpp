// ref_chunk_capi.cpp -- C entry point around the REFERENCE's own chunk rule.
// TEST INFRASTRUCTURE ONLY.  Compiled by oracle/Makefile together with
// /root/reference/src/runtime/deltanet_chunk.cpp (left where it lies, never
// copied) into oracle/_ref/libref_chunk.so.  It lets tests and bench.py's
// cpu_baseline leg call spock::runtime::run_deltanet_chunk_rule
// (src/runtime/deltanet_chunk.hpp:39-40) through ctypes.
#include "runtime/deltanet_chunk.hpp"

#include <cstring>
#include <exception>
#include <vector>

extern "C" int ref_chunk_rule(std::size_t H, std::size_t T, std::size_t dk, std::size_t dv,
                              std::size_t C, int use_qk_l2norm, const float* q,
                              const float* k, const float* v, const float* g,
                              const float* beta, const float* init, float* out_core,
                              float* out_state) {
  try {
    spock::runtime::DeltaNetChunkConfig cfg;
    cfg.num_heads = H;
    cfg.sequence_length = T;
    cfg.key_dim = dk;
    cfg.value_dim = dv;
    cfg.chunk_size = C;
    cfg.use_qk_l2norm = use_qk_l2norm != 0;
    spock::runtime::DeltaNetChunkInputs in;
    in.query.assign(q, q + H * T * dk);
    in.key.assign(k, k + H * T * dk);
    in.value.assign(v, v + H * T * dv);
    in.g.assign(g, g + H * T);
    in.beta.assign(beta, beta + H * T);
    if (init) in.initial_state.assign(init, init + H * dk * dv);
    const auto out = spock::runtime::run_deltanet_chunk_rule(cfg, in);
    std::memcpy(out_core, out.core_attn_out.data(), out.core_attn_out.size() * sizeof(float));
    std::memcpy(out_state, out.final_state.data(), out.final_state.size() * sizeof(float));
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}
