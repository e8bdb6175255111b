// deltanet_session.cpp -- see deltanet_session.hpp.
#include "deltanet_session.hpp"

#include <stdexcept>
#include <string>

namespace spock::hip {

namespace {

// vk_session.cpp:63-67: storage offsets rounded up to 256 bytes.
constexpr std::size_t align256(std::size_t n) { return (n + 255) & ~std::size_t(255); }

}  // namespace

DeltaNetSession::DeltaNetSession(std::uint32_t num_layers, std::uint32_t max_seq)
    : num_layers_(num_layers), max_seq_(max_seq) {
  if (num_layers_ == 0 || max_seq_ == 0) throw std::runtime_error("DeltaNetSession: layers and max_seq must be non-zero");
  hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
  const std::size_t H = DN_HEADS;
  state_ = DeviceBuffer(num_layers_ * kStateFloats * sizeof(float));
  conv_state_ = DeviceBuffer(std::size_t(num_layers_) * DN_CONV_DIM * DN_CONV_KS * sizeof(std::uint16_t));
  a_log_bias_ = DeviceBuffer(std::size_t(num_layers_) * H * 2 * sizeof(float));
  const std::size_t qk = num_layers_ * align256(H * max_seq_ * DN_K_DIM * sizeof(float));
  const std::size_t gb = num_layers_ * align256(H * max_seq_ * sizeof(float));
  collect_q_ = DeviceBuffer(qk);
  collect_k_ = DeviceBuffer(qk);
  collect_v_ = DeviceBuffer(qk);
  collect_g_ = DeviceBuffer(gb);
  collect_beta_ = DeviceBuffer(gb);
  const std::size_t max_total = (std::size_t(max_seq_) + 63) / 64 * 64;
  chunk_out_ = DeviceBuffer((H * max_total * DN_V_DIM + H * DN_K_DIM * DN_V_DIM) * sizeof(float));
  chunk_ws_ = DeviceBuffer(spk_chunk_prefill_workspace_size(DN_HEADS, static_cast<std::int32_t>(max_seq_), 1, 64));
  attn_out_ = DeviceBuffer(std::size_t(num_layers_) * DN_VAL_TOTAL * sizeof(std::uint16_t));
  argmax_idx_ = DeviceBuffer(sizeof(std::uint32_t));
  a_log_bias_.zero(stream_);
  reset();
}

DeltaNetSession::~DeltaNetSession() {
  if (stream_) {
    (void)hipStreamSynchronize(stream_);
    (void)hipStreamDestroy(stream_);
  }
}

void DeltaNetSession::check_prompt_len(std::uint32_t prompt_len) const {
  if (prompt_len == 0 || prompt_len > max_seq_)
    throw std::runtime_error("prompt length " + std::to_string(prompt_len) + " out of range (max_seq " +
                             std::to_string(max_seq_) + ")");
}

// vk_session.cpp:1634-1644 and :4494-4497: layer dn_idx's segment starts at
// dn_idx * align256(segment bytes for this prompt length).
DeltaNetSession::Segments DeltaNetSession::segments(std::uint32_t dn_idx, std::uint32_t prompt_len) const {
  const std::size_t qk = align256(std::size_t(DN_HEADS) * prompt_len * DN_K_DIM * sizeof(float));
  const std::size_t vv = align256(std::size_t(DN_HEADS) * prompt_len * DN_V_DIM * sizeof(float));
  const std::size_t gb = align256(std::size_t(DN_HEADS) * prompt_len * sizeof(float));
  return {reinterpret_cast<float*>(collect_q_.get<char>() + dn_idx * qk),
          reinterpret_cast<float*>(collect_k_.get<char>() + dn_idx * qk),
          reinterpret_cast<float*>(collect_v_.get<char>() + dn_idx * vv),
          reinterpret_cast<float*>(collect_g_.get<char>() + dn_idx * gb),
          reinterpret_cast<float*>(collect_beta_.get<char>() + dn_idx * gb)};
}

void DeltaNetSession::check_layer(std::uint32_t dn_idx) const {
  if (dn_idx >= num_layers_)
    throw std::runtime_error("DeltaNet layer index " + std::to_string(dn_idx) + " out of range (" +
                             std::to_string(num_layers_) + " layers)");
}

float* DeltaNetSession::dn_state(std::uint32_t dn_idx) const {
  check_layer(dn_idx);
  return state_.get<float>() + dn_idx * kStateFloats;
}
std::uint16_t* DeltaNetSession::dn_conv_state(std::uint32_t dn_idx) const {
  check_layer(dn_idx);
  return conv_state_.get<std::uint16_t>() + std::size_t(dn_idx) * DN_CONV_DIM * DN_CONV_KS;
}
std::uint16_t* DeltaNetSession::dn_chunk_attn_out(std::uint32_t dn_idx) const {
  check_layer(dn_idx);
  return attn_out_.get<std::uint16_t>() + std::size_t(dn_idx) * DN_VAL_TOTAL;
}

void DeltaNetSession::reset() {
  state_.zero(stream_);
  conv_state_.zero(stream_);
  attn_out_.zero(stream_);
  synchronize();
}

void DeltaNetSession::synchronize() { hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize"); }

void DeltaNetSession::upload_a_log_bias(const std::vector<float>& v) {
  const std::size_t n = std::size_t(num_layers_) * DN_HEADS * 2;
  if (v.size() != n)
    throw std::runtime_error("a_log_bias size mismatch: expected " + std::to_string(n) + ", got " + std::to_string(v.size()));
  synchronize();
  a_log_bias_.upload(v.data(), n * sizeof(float));
}

void DeltaNetSession::upload_state(std::uint32_t dn_idx, const std::vector<float>& s) {
  check_layer(dn_idx);
  const std::size_t core = std::size_t(DN_HEADS) * DN_K_DIM * DN_V_DIM;
  if (s.size() != core && s.size() != kStateFloats)
    throw std::runtime_error("state size mismatch: expected " + std::to_string(kStateFloats) + ", got " +
                             std::to_string(s.size()));
  synchronize();
  state_.upload(s.data(), s.size() * sizeof(float), dn_idx * kStateFloats * sizeof(float));
}

void DeltaNetSession::upload_conv_state(std::uint32_t dn_idx, const std::vector<std::uint16_t>& c) {
  check_layer(dn_idx);
  const std::size_t n = std::size_t(DN_CONV_DIM) * DN_CONV_KS;
  if (c.size() != n)
    throw std::runtime_error("conv state size mismatch: expected " + std::to_string(n) + ", got " + std::to_string(c.size()));
  synchronize();
  conv_state_.upload(c.data(), n * sizeof(std::uint16_t), dn_idx * n * sizeof(std::uint16_t));
}

std::vector<float> DeltaNetSession::download_state(std::uint32_t dn_idx) {
  check_layer(dn_idx);
  synchronize();
  std::vector<float> s(kStateFloats);
  state_.download(s.data(), kStateFloats * sizeof(float), dn_idx * kStateFloats * sizeof(float));
  return s;
}

std::vector<std::uint16_t> DeltaNetSession::download_conv_state(std::uint32_t dn_idx) {
  check_layer(dn_idx);
  synchronize();
  const std::size_t n = std::size_t(DN_CONV_DIM) * DN_CONV_KS;
  std::vector<std::uint16_t> c(n);
  conv_state_.download(c.data(), n * sizeof(std::uint16_t), dn_idx * n * sizeof(std::uint16_t));
  return c;
}

std::vector<std::uint16_t> DeltaNetSession::download_chunk_attn_out(std::uint32_t dn_idx) {
  check_layer(dn_idx);
  synchronize();
  std::vector<std::uint16_t> o(DN_VAL_TOTAL);
  attn_out_.download(o.data(), DN_VAL_TOTAL * sizeof(std::uint16_t), std::size_t(dn_idx) * DN_VAL_TOTAL * sizeof(std::uint16_t));
  return o;
}

std::vector<float> DeltaNetSession::download_last_core(std::uint32_t prompt_len) {
  check_prompt_len(prompt_len);
  if (last_total_seq_ == 0) throw std::runtime_error("no chunk prefill has run");
  synchronize();
  std::vector<float> out(std::size_t(DN_HEADS) * prompt_len * DN_V_DIM);
  for (std::uint32_t h = 0; h < DN_HEADS; ++h)
    chunk_out_.download(out.data() + std::size_t(h) * prompt_len * DN_V_DIM, std::size_t(prompt_len) * DN_V_DIM * sizeof(float),
                        std::size_t(h) * last_total_seq_ * DN_V_DIM * sizeof(float));
  return out;
}

void DeltaNetSession::collect_prefill_token(std::uint32_t dn_idx, std::uint32_t token_idx, std::uint32_t prompt_len,
                                            const std::uint16_t* dn_qkv, const float* g_beta) {
  check_layer(dn_idx);
  check_prompt_len(prompt_len);
  if (token_idx >= prompt_len) throw std::runtime_error("prefill token index beyond the prompt length");
  if (g_beta == nullptr) g_beta = dn_state(dn_idx) + std::size_t(DN_HEADS) * DN_K_DIM * DN_V_DIM;
  const Segments s = segments(dn_idx, prompt_len);
  spk_check(spk_prefill_collect(dn_qkv, g_beta, s.q, s.k, s.v, s.g, s.beta, DN_HEADS,
                                static_cast<std::int32_t>(prompt_len), static_cast<std::int32_t>(token_idx), DN_K_DIM,
                                DN_V_DIM, stream_),
            "deltanet prefill collect");
}

void DeltaNetSession::gpu_chunk_prefill_from_gpu_collect(std::uint32_t dn_idx, std::uint32_t prompt_len) {
  check_layer(dn_idx);
  check_prompt_len(prompt_len);
  const Segments s = segments(dn_idx, prompt_len);
  const std::uint32_t total_seq = (prompt_len + 63) / 64 * 64;  // vk_session.cpp:4469
  SpkChunkArgs a{};
  a.num_heads = DN_HEADS;
  a.total_tokens = static_cast<std::int32_t>(prompt_len);
  a.key_dim = DN_K_DIM;
  a.value_dim = DN_V_DIM;
  a.chunk_size = 64;
  a.use_qk_l2norm = 0;  // q/k were L2-normed by the conv kernel (vk_session.cpp:4914)
  a.q_scale = 0.0f;     // 1/sqrt(128)
  a.input_dtype = SPK_F32;
  a.q = s.q;
  a.k = s.k;
  a.v = s.v;
  a.g = s.g;
  a.beta = s.beta;
  a.initial_state = nullptr;  // the tiled shader's zero state (:66-71)
  a.out_core = chunk_out_.get<float>();
  a.core_head_stride = total_seq;
  a.out_state = dn_state(dn_idx);  // final_state copy of :4599, tail untouched
  a.num_seqs = 1;
  a.workspace = chunk_ws_.get();
  a.workspace_bytes = chunk_ws_.bytes();
  spk_check(spk_chunk_prefill(&a, stream_), "deltanet chunk prefill");
  spk_check(spk_chunk_last_to_fp16(chunk_out_.get<float>(), dn_chunk_attn_out(dn_idx), DN_HEADS, DN_V_DIM,
                                   static_cast<std::int32_t>(prompt_len), static_cast<std::int32_t>(total_seq), stream_),
            "deltanet chunk last_to_fp16");
  last_total_seq_ = total_seq;
}

void DeltaNetSession::run_chunk_prefill(std::uint32_t prompt_len) {
  for (std::uint32_t l = 0; l < num_layers_; ++l) gpu_chunk_prefill_from_gpu_collect(l, prompt_len);
}

void DeltaNetSession::deltanet_decode_step(std::uint32_t dn_idx, std::uint16_t* dn_qkv, const std::uint16_t* a,
                                           const std::uint16_t* b, const std::uint16_t* z,
                                           const std::uint16_t* conv_weight, const float* norm_weight) {
  check_layer(dn_idx);
  SpkDecodeArgs d{};
  d.batch = 1;
  d.num_heads = DN_HEADS;
  d.layer_idx = static_cast<std::int32_t>(dn_idx);
  d.q_scale = 0.0f;
  d.rms_eps = kRmsEps;
  d.qkv = dn_qkv;
  d.qkv_stride = DN_CONV_DIM;
  d.conv_state = dn_conv_state(dn_idx);
  d.conv_state_stride = std::int64_t(DN_CONV_DIM) * DN_CONV_KS;
  d.conv_weight = conv_weight;
  d.a = a;
  d.b = b;
  d.ab_stride = DN_HEADS;
  d.a_log_bias = a_log_bias_.get<float>();
  d.state = dn_state(dn_idx);
  d.state_stride = static_cast<std::int64_t>(kStateFloats);
  d.z = z;
  d.z_stride = DN_VAL_TOTAL;
  d.norm_weight = norm_weight;
  spk_check(spk_deltanet_decode_step(&d, stream_), "deltanet decode step");
}

std::uint32_t DeltaNetSession::lm_head_argmax(const std::uint16_t* embed_tokens, const std::uint16_t* x,
                                              std::uint32_t vocab, std::uint32_t hidden, std::uint16_t* logits) {
  if (vocab != lm_ws_vocab_) {
    synchronize();
    lm_ws_ = DeviceBuffer(spk_lm_head_workspace_size(static_cast<std::int32_t>(vocab)));
    lm_ws_vocab_ = vocab;
  }
  spk_check(spk_lm_head_argmax(embed_tokens, x, static_cast<std::int32_t>(vocab), static_cast<std::int32_t>(hidden),
                               logits, argmax_idx_.get<std::uint32_t>(), lm_ws_.get(), lm_ws_.bytes(), stream_),
            "lm_head argmax");
  std::uint32_t idx = 0;
  hip_check(hipMemcpyAsync(&idx, argmax_idx_.get(), sizeof(idx), hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync");
  synchronize();
  return idx;
}

}  // namespace spock::hip
