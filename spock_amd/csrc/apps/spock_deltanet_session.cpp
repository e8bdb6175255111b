// spock-deltanet-session -- drives DeltaNetSession through a prompt prefill,
// decode steps and the lm_head argmax, from binary input files.
//
// The flow is the DeltaNet part of DecodeSession::decode
// (vk_session.cpp:1632-1670 collect per token, :4830-4952 chunk prefill per
// layer, :2876-2884/:3212-3219 decode step per layer and token, :3533-3563
// lm_head + argmax); attention, MLP and the projections are not part of it,
// so the per-token activations come from the input files.
//
// usage: spock-deltanet-session --input DIR --output DIR
// DIR/meta.json {"layers", "prompt_len", "decode_steps", "vocab", "hidden"}
// inputs (raw little-endian):
//   prefill_qkv.u16 [L][T][6144]   prefill_gbeta.f32 [L][T][32]
//   a_log_bias.f32 [L][16][2]      conv_state.u16 [L][6144][4]
//   conv_weight.u16 [L][6144][4]   norm_weight.f32 [128]
//   decode_qkv.u16 [D][L][6144]    decode_a.u16, decode_b.u16 [D][L][16]
//   decode_z.u16 [D][L][2048]      lm_weight.u16 [V][hidden]   lm_x.u16 [hidden]
// outputs:
//   prefill_core.f32 [L][16][T][128]   chunk_attn_out.u16 [L][2048]
//   prefill_state.f32 [L][262176]      decode_out.u16 [D][L][6144]
//   final_state.f32 [L][262176]        final_conv_state.u16 [L][6144][4]
//   token.json {"token": argmax}
#include <cstdint>
#include <cstdio>
#include <exception>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "../host/deltanet_session.hpp"
#include "../host/json_lite.hpp"

namespace {

using spock::hip::DeltaNetSession;
using spock::hip::DeviceBuffer;

template <typename T>
std::vector<T> read_raw(const std::string& path, std::size_t count) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("cannot open " + path);
  std::vector<T> v(count);
  f.read(reinterpret_cast<char*>(v.data()), static_cast<std::streamsize>(count * sizeof(T)));
  if (static_cast<std::size_t>(f.gcount()) != count * sizeof(T) || f.peek() != EOF)
    throw std::runtime_error(path + ": expected " + std::to_string(count * sizeof(T)) + " bytes");
  return v;
}

template <typename T>
void write_raw(const std::string& path, const std::vector<T>& v) {
  std::ofstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("cannot write " + path);
  f.write(reinterpret_cast<const char*>(v.data()), static_cast<std::streamsize>(v.size() * sizeof(T)));
}

template <typename T>
DeviceBuffer to_device(const std::vector<T>& v) {
  DeviceBuffer b(v.size() * sizeof(T));
  b.upload(v.data(), v.size() * sizeof(T));
  return b;
}

template <typename T>
void append(std::vector<T>& dst, const std::vector<T>& src) {
  dst.insert(dst.end(), src.begin(), src.end());
}

int run(const std::string& in, const std::string& out) {
  const auto meta = spock::hip::json::read_file(in + "/meta.json");
  const auto L = static_cast<std::uint32_t>(meta.get_int("layers"));
  const auto T = static_cast<std::uint32_t>(meta.get_int("prompt_len"));
  const auto D = static_cast<std::uint32_t>(meta.get_int("decode_steps"));
  const auto V = static_cast<std::uint32_t>(meta.get_int("vocab"));
  const auto HID = static_cast<std::uint32_t>(meta.get_int("hidden"));
  constexpr std::size_t CD = DeltaNetSession::DN_CONV_DIM;
  constexpr std::size_t NH = DeltaNetSession::DN_HEADS;
  constexpr std::size_t VT = DeltaNetSession::DN_VAL_TOTAL;

  const auto pre_qkv = read_raw<std::uint16_t>(in + "/prefill_qkv.u16", std::size_t(L) * T * CD);
  const auto pre_gb = read_raw<float>(in + "/prefill_gbeta.f32", std::size_t(L) * T * 2 * NH);
  const auto alb = read_raw<float>(in + "/a_log_bias.f32", std::size_t(L) * NH * 2);
  const auto conv0 = read_raw<std::uint16_t>(in + "/conv_state.u16", std::size_t(L) * CD * 4);
  const auto conv_w = read_raw<std::uint16_t>(in + "/conv_weight.u16", std::size_t(L) * CD * 4);
  const auto norm_w = read_raw<float>(in + "/norm_weight.f32", 128);
  const auto dec_qkv = read_raw<std::uint16_t>(in + "/decode_qkv.u16", std::size_t(D) * L * CD);
  const auto dec_a = read_raw<std::uint16_t>(in + "/decode_a.u16", std::size_t(D) * L * NH);
  const auto dec_b = read_raw<std::uint16_t>(in + "/decode_b.u16", std::size_t(D) * L * NH);
  const auto dec_z = read_raw<std::uint16_t>(in + "/decode_z.u16", std::size_t(D) * L * VT);
  const auto lm_w = read_raw<std::uint16_t>(in + "/lm_weight.u16", std::size_t(V) * HID);
  const auto lm_x = read_raw<std::uint16_t>(in + "/lm_x.u16", HID);

  DeltaNetSession s(L, T);
  s.upload_a_log_bias(alb);

  // Prefill: collect every token of every layer, then the chunk rule per layer.
  DeviceBuffer d_pre_qkv = to_device(pre_qkv), d_pre_gb = to_device(pre_gb);
  for (std::uint32_t l = 0; l < L; ++l)
    for (std::uint32_t t = 0; t < T; ++t)
      s.collect_prefill_token(l, t, T, d_pre_qkv.get<std::uint16_t>() + (std::size_t(l) * T + t) * CD,
                              d_pre_gb.get<float>() + (std::size_t(l) * T + t) * 2 * NH);
  std::vector<float> core_all, state_all;
  std::vector<std::uint16_t> attn_all;
  for (std::uint32_t l = 0; l < L; ++l) {
    s.gpu_chunk_prefill_from_gpu_collect(l, T);
    append(core_all, s.download_last_core(T));
  }
  for (std::uint32_t l = 0; l < L; ++l) {
    append(state_all, s.download_state(l));
    append(attn_all, s.download_chunk_attn_out(l));
  }
  write_raw(out + "/prefill_core.f32", core_all);
  write_raw(out + "/chunk_attn_out.u16", attn_all);
  write_raw(out + "/prefill_state.f32", state_all);

  // Decode: one fused step per layer and token, in place on dn_qkv.
  for (std::uint32_t l = 0; l < L; ++l)
    s.upload_conv_state(l, std::vector<std::uint16_t>(conv0.begin() + std::size_t(l) * CD * 4,
                                                      conv0.begin() + std::size_t(l + 1) * CD * 4));
  DeviceBuffer d_qkv = to_device(dec_qkv), d_a = to_device(dec_a), d_b = to_device(dec_b), d_z = to_device(dec_z);
  DeviceBuffer d_cw = to_device(conv_w), d_nw = to_device(norm_w);
  for (std::uint32_t d = 0; d < D; ++d)
    for (std::uint32_t l = 0; l < L; ++l) {
      const std::size_t i = std::size_t(d) * L + l;
      s.deltanet_decode_step(l, d_qkv.get<std::uint16_t>() + i * CD, d_a.get<std::uint16_t>() + i * NH,
                             d_b.get<std::uint16_t>() + i * NH, d_z.get<std::uint16_t>() + i * VT,
                             d_cw.get<std::uint16_t>() + std::size_t(l) * CD * 4, d_nw.get<float>());
    }
  s.synchronize();
  std::vector<std::uint16_t> dec_out(dec_qkv.size());
  d_qkv.download(dec_out.data(), dec_out.size() * sizeof(std::uint16_t));
  write_raw(out + "/decode_out.u16", dec_out);
  std::vector<float> fin_state;
  std::vector<std::uint16_t> fin_conv;
  for (std::uint32_t l = 0; l < L; ++l) {
    append(fin_state, s.download_state(l));
    append(fin_conv, s.download_conv_state(l));
  }
  write_raw(out + "/final_state.f32", fin_state);
  write_raw(out + "/final_conv_state.u16", fin_conv);

  DeviceBuffer d_w = to_device(lm_w), d_x = to_device(lm_x);
  const std::uint32_t tok = s.lm_head_argmax(d_w.get<std::uint16_t>(), d_x.get<std::uint16_t>(), V, HID);
  std::ofstream(out + "/token.json") << "{\"token\": " << tok << "}\n";
  std::cout << "{\"layers\": " << L << ", \"prompt_len\": " << T << ", \"decode_steps\": " << D
            << ", \"token\": " << tok << "}\n";
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  std::string in, out;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if (a == "--input" && i + 1 < argc) in = argv[++i];
    else if (a == "--output" && i + 1 < argc) out = argv[++i];
    else if (a == "--help") {
      std::cout << "usage: spock-deltanet-session --input DIR --output DIR\n";
      return 0;
    }
  }
  if (in.empty() || out.empty()) {
    std::cerr << "spock-deltanet-session: --input and --output are required\n";
    return 2;
  }
  try {
    return run(in, out);
  } catch (const std::exception& e) {
    std::cerr << "spock-deltanet-session: " << e.what() << "\n";
    return 1;
  }
}
