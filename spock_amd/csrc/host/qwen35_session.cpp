// qwen35_session.cpp -- Qwen35Session (see qwen35_session.hpp) and the C ABI
// of include/spock_model.h.
#include "qwen35_session.hpp"

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>

#include "../../../include/spock_model.h"

namespace spock::hip {

namespace {

constexpr std::uint32_t H = 1024, INTER = 3584, CONV = 6144, VAL = 2048;

spk_stream_t S(hipStream_t s) { return reinterpret_cast<spk_stream_t>(s); }

// IEEE half -> float (exact), for host-side reads of fp16 artifact tensors.
float half_to_float(std::uint16_t h) {
  const std::uint32_t sign = std::uint32_t(h >> 15) << 31;
  const std::uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
  std::uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {  // subnormal: m * 2^-24
      const float f = static_cast<float>(m) * 5.9604644775390625e-08f;
      std::memcpy(&bits, &f, 4);
      bits |= sign;
    }
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112) << 23) | (m << 13);
  }
  float out;
  std::memcpy(&out, &bits, 4);
  return out;
}

double ms_since(std::chrono::steady_clock::time_point t0) {
  return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

template <typename T>
const T* tensor_ptr(const DeviceBuffer& w, const WeightArtifact& a, const std::string& role, const char* dtype,
                    std::size_t elems) {
  const TensorInfo& t = a.require(role);
  if (t.dtype != dtype) throw std::runtime_error("artifact tensor " + role + " has dtype " + t.dtype);
  if (t.nbytes != elems * sizeof(T))
    throw std::runtime_error("artifact tensor " + role + " has " + std::to_string(t.nbytes) + " bytes, expected " +
                             std::to_string(elems * sizeof(T)));
  if (t.offset % 256 != 0) throw std::runtime_error("artifact tensor " + role + " is not 256-byte aligned");
  return reinterpret_cast<const T*>(w.get<const std::uint8_t>() + t.offset);
}

// RAII pair of HIP events timing a span of the stream.
struct EventTimer {
  hipEvent_t a = nullptr, b = nullptr;
  EventTimer() {
    hip_check(hipEventCreate(&a), "hipEventCreate");
    hip_check(hipEventCreate(&b), "hipEventCreate");
  }
  ~EventTimer() {
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
  }
  float ms() {
    float v = 0.0f;
    hip_check(hipEventElapsedTime(&v, a, b), "hipEventElapsedTime");
    return v;
  }
};

}  // namespace

std::vector<float> rope_table(std::uint32_t max_seq) {
  std::vector<float> t(std::size_t(max_seq) * 64);
  for (std::uint32_t pos = 0; pos < max_seq; ++pos)
    for (int i = 0; i < 32; ++i) {
      const double inv_freq = std::pow(1.0e7, -(2.0 * i) / 64.0);
      const double ang = static_cast<double>(pos) * inv_freq;
      t[std::size_t(pos) * 64 + 2 * i] = static_cast<float>(std::cos(ang));
      t[std::size_t(pos) * 64 + 2 * i + 1] = static_cast<float>(std::sin(ang));
    }
  return t;
}

Qwen35Session::Qwen35Session(const std::string& repack_dir, bool verbose, std::uint32_t max_seq, bool use_graph,
                             bool ordered_prefill, GpuTimestamps gpu_timestamps, bool lm_head_one_launch,
                             bool fused_dn_step)
    : verbose_(verbose),
      use_graph_(use_graph),
      ordered_prefill_(ordered_prefill),
      lm_one_launch_(lm_head_one_launch),
      fused_dn_step_(fused_dn_step),
      max_seq_(max_seq ? max_seq : MAX_SEQ),
      gpu_ts_(gpu_timestamps) {
  if (max_seq_ > 65536) throw std::runtime_error("max_seq must be <= 65536");
  const auto t0 = std::chrono::steady_clock::now();
  WeightArtifact art = WeightArtifact::load(repack_dir);
  shape_ = art.shape();
  if (shape_.layers == 0 || shape_.layers > 64 || shape_.vocab == 0)
    throw std::runtime_error("artifact model shape unsupported (layers " + std::to_string(shape_.layers) + ")");
  n_attn_ = shape_.num_attention_layers();
  n_dn_ = shape_.num_deltanet_layers();
  hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreateWithFlags");

  // Weights: one device copy of text_weights.bin; tensors addressed by offset.
  weights_ = DeviceBuffer(art.total_bytes());
  hip_check(hipMemcpy(weights_.get(), art.mapped(), art.total_bytes(), hipMemcpyHostToDevice), "upload weights");
  const std::size_t V = shape_.vocab;
  embed_ = tensor_ptr<std::uint16_t>(weights_, art, "global.token_embedding", "fp16", V * H);
  final_norm_ = tensor_ptr<std::uint16_t>(weights_, art, "global.final_norm", "fp16", H);
  std::vector<float> alb(std::size_t(n_dn_) * 16 * 2);
  std::uint32_t dn = 0, at = 0;
  for (std::uint32_t L = 0; L < shape_.layers; ++L) {
    const std::string r = "layer." + std::to_string(L) + ".";
    LayerW w;
    w.attn = Qwen35Shape::is_attention(L);
    w.sub = w.attn ? at++ : dn++;
    w.input_norm = tensor_ptr<std::uint16_t>(weights_, art, r + "input_norm", "fp16", H);
    w.post_norm = tensor_ptr<std::uint16_t>(weights_, art, r + "post_norm", "fp16", H);
    w.mlp_gate = tensor_ptr<std::uint16_t>(weights_, art, r + "mlp_gate", "fp16", std::size_t(INTER) * H);
    w.mlp_up = tensor_ptr<std::uint16_t>(weights_, art, r + "mlp_up", "fp16", std::size_t(INTER) * H);
    w.mlp_down = tensor_ptr<std::uint16_t>(weights_, art, r + "mlp_down", "fp16", std::size_t(H) * INTER);
    if (w.attn) {
      w.attn_q = tensor_ptr<std::uint16_t>(weights_, art, r + "attn_q", "fp16", std::size_t(4096) * H);
      w.attn_k = tensor_ptr<std::uint16_t>(weights_, art, r + "attn_k", "fp16", std::size_t(512) * H);
      w.attn_v = tensor_ptr<std::uint16_t>(weights_, art, r + "attn_v", "fp16", std::size_t(512) * H);
      w.attn_o = tensor_ptr<std::uint16_t>(weights_, art, r + "attn_o", "fp16", std::size_t(H) * 2048);
      w.attn_q_norm = tensor_ptr<std::uint16_t>(weights_, art, r + "attn_q_norm", "fp16", 256);
      w.attn_k_norm = tensor_ptr<std::uint16_t>(weights_, art, r + "attn_k_norm", "fp16", 256);
    } else {
      w.dn_qkv = tensor_ptr<std::uint16_t>(weights_, art, r + "delta_in_proj_qkv", "fp16", std::size_t(CONV) * H);
      w.dn_z = tensor_ptr<std::uint16_t>(weights_, art, r + "delta_in_proj_z", "fp16", std::size_t(VAL) * H);
      w.dn_a = tensor_ptr<std::uint16_t>(weights_, art, r + "delta_in_proj_a", "fp16", std::size_t(16) * H);
      w.dn_b = tensor_ptr<std::uint16_t>(weights_, art, r + "delta_in_proj_b", "fp16", std::size_t(16) * H);
      w.dn_conv = tensor_ptr<std::uint16_t>(weights_, art, r + "delta_conv", "fp16", std::size_t(CONV) * 4);
      w.dn_out = tensor_ptr<std::uint16_t>(weights_, art, r + "delta_out_proj", "fp16", std::size_t(H) * VAL);
      w.dn_norm = tensor_ptr<float>(weights_, art, r + "delta_norm", "fp32", 128);
      (void)tensor_ptr<float>(weights_, art, r + "delta_a_log", "fp32", 16);
      (void)tensor_ptr<std::uint16_t>(weights_, art, r + "delta_dt_bias", "fp16", 16);
      // a_log_bias [layers][16][2] = (A_log, dt_bias) (vk_session.cpp:470-495)
      const float* a_log = static_cast<const float*>(art.data(art.require(r + "delta_a_log")));
      const std::uint16_t* dt = static_cast<const std::uint16_t*>(art.data(art.require(r + "delta_dt_bias")));
      for (int h = 0; h < 16; ++h) {
        alb[(std::size_t(w.sub) * 16 + h) * 2] = a_log[h];
        alb[(std::size_t(w.sub) * 16 + h) * 2 + 1] = half_to_float(dt[h]);
      }
    }
    layers_.push_back(w);
  }

  dn_state_ = DeviceBuffer(std::max<std::size_t>(1, n_dn_) * kStateFloats * 4);
  conv_state_ = DeviceBuffer(std::max<std::size_t>(1, n_dn_) * CONV * 4 * 2);
  kv_cache_ = DeviceBuffer(std::max<std::size_t>(1, n_attn_) * max_seq_ * 1024 * 2);
  a_log_bias_ = DeviceBuffer(std::max<std::size_t>(1, alb.size()) * 4);
  if (!alb.empty()) a_log_bias_.upload(alb.data(), alb.size() * 4);
  const std::vector<float> rope = rope_table(max_seq_);
  rope_ = DeviceBuffer(rope.size() * 4);
  rope_.upload(rope.data(), rope.size() * 4);

  h_ = DeviceBuffer(H * 2);
  qkv_ = DeviceBuffer(CONV * 2);
  z_ = DeviceBuffer(VAL * 2);
  a_ = DeviceBuffer(256);
  b_ = DeviceBuffer(256);
  qg_ = DeviceBuffer(4096 * 2);
  k_ = DeviceBuffer(512 * 2);
  v_ = DeviceBuffer(512 * 2);
  attn_out_ = DeviceBuffer(2048 * 2);
  gate_ = DeviceBuffer(INTER * 2);
  up_ = DeviceBuffer(INTER * 2);
  logits_ = DeviceBuffer(V * 2);
  attn_ws_ = DeviceBuffer(spk_attention_workspace_size(static_cast<int32_t>(max_seq_), 1));
  attn_ws_.zero(stream_);  // spk_attention_decode_oproj's arrival counts start at zero and are left at zero
  argmax_key_ = DeviceBuffer(SPK_ARGMAX_KEY_WORDS * 8);
  argmax_key_.zero(stream_);  // spk_argmax_key_take returns it to zero after every use
  take_slots_ = DeviceBuffer(spk_lm_head_take_slots(static_cast<int32_t>(V)) * 8);
  take_slots_.zero(stream_);  // spk_lm_head_argmax_take returns them to zero after every use
  dn_arrive_ = DeviceBuffer(4096);
  dn_arrive_.zero(stream_);  // spk_deltanet_inproj_step returns its 16 counts to zero after every use
  tok_ = DeviceBuffer(256);
  pos_ = DeviceBuffer(256);
  history_cap_ = max_seq_;
  history_ = DeviceBuffer(std::size_t(history_cap_ + 64) * 4);  // [count | pad | history]
  reset();
  if (verbose_)
    std::fprintf(stderr, "[spock-hip] session: %u layers (%u DeltaNet, %u attention), vocab %u, %.1f MiB weights, %.1f ms\n",
                 shape_.layers, n_dn_, n_attn_, shape_.vocab, art.total_bytes() / 1048576.0, ms_since(t0));
}

Qwen35Session::~Qwen35Session() {
  if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
  if (graph_) (void)hipGraphDestroy(graph_);
  if (stream_) {
    (void)hipStreamSynchronize(stream_);
    (void)hipStreamDestroy(stream_);
  }
  for (hipEvent_t e : ts_events_) (void)hipEventDestroy(e);
}

void Qwen35Session::ensure_ts_events(std::size_t n) {
  while (ts_events_.size() < n) {
    hipEvent_t e = nullptr;
    hip_check(hipEventCreate(&e), "hipEventCreate");
    ts_events_.push_back(e);
  }
}

void Qwen35Session::mark(std::size_t k) {
  if (marks_) hip_check(hipEventRecord(marks_[k], stream_), "hipEventRecord (region)");
}

void Qwen35Session::reset() {
  dn_state_.zero(stream_);
  conv_state_.zero(stream_);
  kv_cache_.zero(stream_);
  tok_.zero(stream_);
  pos_.zero(stream_);
  history_.zero(stream_);
  hip_check(hipStreamSynchronize(stream_), "reset");
  pos_host_ = 0;
  history_len_ = 0;
}

void Qwen35Session::ensure_prefill_capacity(std::uint32_t T) {
  if (T <= prefill_cap_) return;
  const std::size_t n = T;
  p_tokens_ = DeviceBuffer(n * 4);
  p_h_ = DeviceBuffer(n * H * 2);
  p_xn_ = DeviceBuffer(n * H * 2);
  p_qkv_ = DeviceBuffer(n * CONV * 2);
  p_z_ = DeviceBuffer(n * VAL * 2);
  p_a_ = DeviceBuffer(n * 16 * 2);
  p_b_ = DeviceBuffer(n * 16 * 2);
  p_qhm_ = DeviceBuffer(n * VAL * 2);
  p_khm_ = DeviceBuffer(n * VAL * 2);
  p_vhm_ = DeviceBuffer(n * VAL * 2);
  p_g_ = DeviceBuffer(n * 16 * 4);
  p_beta_ = DeviceBuffer(n * 16 * 4);
  p_core_ = DeviceBuffer(n * VAL * 4);
  p_state_ = DeviceBuffer(std::size_t(16) * 128 * 128 * 4);
  p_chunk_ws_ = DeviceBuffer(std::max(spk_chunk_prefill_workspace_size(16, static_cast<int32_t>(T), 1, 64),
                                      spk_chunk_prefill_ordered_workspace_size(16, static_cast<int32_t>(T))));
  p_gated_ = DeviceBuffer(n * VAL * 2);
  p_qg_ = DeviceBuffer(n * 4096 * 2);
  p_k_ = DeviceBuffer(n * 512 * 2);
  p_v_ = DeviceBuffer(n * 512 * 2);
  p_ga_ = DeviceBuffer(n * INTER * 2);
  p_up_ = DeviceBuffer(n * INTER * 2);
  p_attn_ws_ = DeviceBuffer(spk_attention_workspace_size(static_cast<int32_t>(max_seq_), static_cast<int32_t>(T)));
  prefill_cap_ = T;
}

std::uint32_t Qwen35Session::prefill(const std::vector<std::uint32_t>& tokens) {
  const std::uint32_t T = static_cast<std::uint32_t>(tokens.size());
  if (T == 0) throw std::runtime_error("prefill: empty prompt");
  if (std::size_t(pos_host_) + T > max_seq_)
    throw std::runtime_error("prefill: " + std::to_string(T) + " tokens at position " + std::to_string(pos_host_) +
                             " exceed max_seq " + std::to_string(max_seq_));
  for (auto t : tokens)
    if (t >= shape_.vocab) throw std::runtime_error("prefill: token id " + std::to_string(t) + " >= vocab");
  ensure_prefill_capacity(T);
  const std::int32_t p0 = pos_host_;
  const std::int32_t Ti = static_cast<std::int32_t>(T);
  const std::vector<std::int32_t> ids(tokens.begin(), tokens.end());
  EventTimer ev;
  hip_check(hipEventRecord(ev.a, stream_), "hipEventRecord");
  hip_check(hipMemcpyAsync(p_tokens_.get(), ids.data(), T * 4, hipMemcpyHostToDevice, stream_), "upload prompt");
  auto* Hs = p_h_.get<std::uint16_t>();
  auto* XN = p_xn_.get<std::uint16_t>();
  // Prompt projections: the matvec's own order (bit-identical to decode and to
  // the CPU restatement) or the matrix cores.
  auto proj = [&](const std::uint16_t* W, const std::uint16_t* X, std::int64_t ldx, std::uint16_t* Y, std::int64_t ldy,
                  const std::uint16_t* R, std::uint32_t out_dim, std::uint32_t in_dim, const char* what) {
    if (ordered_prefill_)
      spk_check(spk_matvec_f16_rows(W, X, ldx, Y, ldy, R, Ti, static_cast<int32_t>(out_dim),
                                    static_cast<int32_t>(in_dim), S(stream_)),
                what);
    else
      spk_check(spk_gemm_f16(X, ldx, W, in_dim, Y, ldy, R, Ti, static_cast<int32_t>(out_dim),
                             static_cast<int32_t>(in_dim), S(stream_)),
                what);
  };
  spk_check(spk_embedding_f16(embed_, p_tokens_.get<std::int32_t>(), Ti, static_cast<int32_t>(shape_.vocab), Hs, S(stream_)),
            "embedding");
  for (const LayerW& w : layers_) {
    spk_check(spk_rmsnorm_f16(Hs, w.input_norm, XN, Ti, H, S(stream_)), "input norm");
    if (!w.attn) {
      auto* QKV = p_qkv_.get<std::uint16_t>();
      auto* Z = p_z_.get<std::uint16_t>();
      auto* A = p_a_.get<std::uint16_t>();
      auto* B = p_b_.get<std::uint16_t>();
      proj(w.dn_qkv, XN, H, QKV, CONV, nullptr, CONV, H, "in_proj_qkv");
      proj(w.dn_z, XN, H, Z, VAL, nullptr, VAL, H, "in_proj_z");
      proj(w.dn_a, XN, H, A, 16, nullptr, 16, H, "in_proj_a");
      proj(w.dn_b, XN, H, B, 16, nullptr, 16, H, "in_proj_b");
      spk_check(spk_deltanet_prefill_conv(QKV, CONV, conv_layer(w.sub), w.dn_conv, Ti, p_qhm_.get<std::uint16_t>(),
                                          p_khm_.get<std::uint16_t>(), p_vhm_.get<std::uint16_t>(), S(stream_)),
                "prefill conv");
      spk_check(spk_deltanet_prefill_gbeta(A, B, 16, a_log_bias_.get<float>(), static_cast<int32_t>(w.sub), Ti,
                                           p_g_.get<float>(), p_beta_.get<float>(), S(stream_)),
                "prefill g/beta");
      SpkChunkArgs c{};
      c.num_heads = 16;
      c.total_tokens = Ti;
      c.key_dim = 128;
      c.value_dim = 128;
      c.chunk_size = 64;
      c.use_qk_l2norm = 0;
      c.q_scale = 0.0f;
      c.input_dtype = SPK_F16;
      c.q = p_qhm_.get();
      c.k = p_khm_.get();
      c.v = p_vhm_.get();
      c.g = p_g_.get<float>();
      c.beta = p_beta_.get<float>();
      c.initial_state = dn_state_layer(w.sub);
      c.out_core = p_core_.get<float>();
      c.core_head_stride = Ti;
      c.out_state = p_state_.get<float>();
      c.cu_seqlens = nullptr;
      c.cu_seqlens_host = nullptr;
      c.num_seqs = 1;
      c.workspace = p_chunk_ws_.get();
      c.workspace_bytes = p_chunk_ws_.bytes();
      if (ordered_prefill_)
        spk_check(spk_chunk_prefill_ordered(&c, S(stream_)), "chunk prefill (reference order)");
      else
        spk_check(spk_chunk_prefill(&c, S(stream_)), "chunk prefill");
      hip_check(hipMemcpyAsync(dn_state_layer(w.sub), p_state_.get(), std::size_t(16) * 128 * 128 * 4,
                               hipMemcpyDeviceToDevice, stream_),
                "final state");
      spk_check(spk_deltanet_norm_gate(p_core_.get<float>(), Ti, Z, VAL, w.dn_norm, 1e-6f, Ti,
                                       p_gated_.get<std::uint16_t>(), VAL, S(stream_)),
                "norm gate");
      proj(w.dn_out, p_gated_.get<std::uint16_t>(), VAL, Hs, H, Hs, H, VAL, "out_proj");
    } else {
      proj(w.attn_q, XN, H, p_qg_.get<std::uint16_t>(), 4096, nullptr, 4096, H, "q_proj");
      proj(w.attn_k, XN, H, p_k_.get<std::uint16_t>(), 512, nullptr, 512, H, "k_proj");
      proj(w.attn_v, XN, H, p_v_.get<std::uint16_t>(), 512, nullptr, 512, H, "v_proj");
      SpkAttnArgs aa{};
      aa.qg = p_qg_.get<std::uint16_t>();
      aa.k = p_k_.get<std::uint16_t>();
      aa.v = p_v_.get<std::uint16_t>();
      aa.q_norm_w = w.attn_q_norm;
      aa.k_norm_w = w.attn_k_norm;
      aa.rope = rope_.get<float>();
      aa.kv_cache = kv_layer(w.sub);
      aa.max_seq = static_cast<int32_t>(max_seq_);
      aa.pos_dev = nullptr;
      aa.out = p_gated_.get<std::uint16_t>();
      aa.workspace = p_attn_ws_.get();
      aa.workspace_bytes = p_attn_ws_.bytes();
      spk_check(spk_attention_prefill(&aa, p0, Ti, S(stream_)), "attention prefill");
      proj(w.attn_o, p_gated_.get<std::uint16_t>(), 2048, Hs, H, Hs, H, 2048, "o_proj");
    }
    spk_check(spk_rmsnorm_f16(Hs, w.post_norm, XN, Ti, H, S(stream_)), "post norm");
    proj(w.mlp_gate, XN, H, p_ga_.get<std::uint16_t>(), INTER, nullptr, INTER, H, "gate_proj");
    proj(w.mlp_up, XN, H, p_up_.get<std::uint16_t>(), INTER, nullptr, INTER, H, "up_proj");
    spk_check(spk_silu_gate_f16(p_ga_.get<std::uint16_t>(), p_up_.get<std::uint16_t>(), p_ga_.get<std::uint16_t>(),
                                std::int64_t(T) * INTER, S(stream_)),
              "silu gate");
    proj(w.mlp_down, p_ga_.get<std::uint16_t>(), INTER, Hs, H, Hs, H, INTER, "down_proj");
  }
  // Last token: final norm, lm_head + argmax, token bookkeeping on the device.
  const std::uint16_t* last = Hs + std::size_t(T - 1) * H;
  hip_check(hipMemcpyAsync(h_.get(), last, H * 2, hipMemcpyDeviceToDevice, stream_), "last hidden");
  const std::int32_t pos_count[2] = {p0 + Ti - 1, 0};
  hip_check(hipMemcpyAsync(pos_.get(), &pos_count[0], 4, hipMemcpyHostToDevice, stream_), "position");
  hip_check(hipMemcpyAsync(history_.get(), &pos_count[1], 4, hipMemcpyHostToDevice, stream_), "history count");
  lm_head_token(last, tok_.get<std::uint32_t>(), false);
  hip_check(hipEventRecord(ev.b, stream_), "hipEventRecord");
  std::int32_t first = 0;
  hip_check(hipMemcpyAsync(&first, history_.get<std::int32_t>() + 64, 4, hipMemcpyDeviceToHost, stream_),
            "first token");
  hip_check(hipStreamSynchronize(stream_), "prefill");
  last_gpu_prefill_ms_ = ev.ms();
  pos_host_ = p0 + Ti;
  history_len_ = 1;
  return static_cast<std::uint32_t>(first);
}

void Qwen35Session::enqueue_decode_step() {
  std::int32_t* tok = tok_.get<std::int32_t>();
  std::uint16_t* h = h_.get<std::uint16_t>();
  const std::size_t NL = layers_.size();
  mark(0);
  for (std::size_t L = 0; L < NL; ++L) {
    const LayerW& w = layers_[L];
    SpkGemvInput in{};
    in.kind = SPK_GEMV_IN_RMSNORM;
    in.in_dim = H;
    in.x = L == 0 ? embed_ : h;
    in.x2 = w.input_norm;
    in.token = L == 0 ? tok : nullptr;
    in.token_rows = static_cast<int32_t>(shape_.vocab);
    in.h_out = L == 0 ? h : nullptr;
    if (!w.attn) {
      const SpkGemvOutput outs[4] = {
          {w.dn_qkv, qkv_.get<std::uint16_t>(), nullptr, static_cast<int32_t>(CONV), nullptr},
          {w.dn_z, z_.get<std::uint16_t>(), nullptr, static_cast<int32_t>(VAL), nullptr},
          {w.dn_a, a_.get<std::uint16_t>(), nullptr, 16, nullptr},
          {w.dn_b, b_.get<std::uint16_t>(), nullptr, 16, nullptr}};
      SpkDecodeArgs d{};
      d.batch = 1;
      d.num_heads = 16;
      d.layer_idx = static_cast<int32_t>(w.sub);
      d.qkv = qkv_.get<std::uint16_t>();
      d.qkv_stride = CONV;
      d.conv_state = conv_layer(w.sub);
      d.conv_state_stride = CONV * 4;
      d.conv_weight = w.dn_conv;
      d.a = a_.get<std::uint16_t>();
      d.b = b_.get<std::uint16_t>();
      d.ab_stride = 16;
      d.a_log_bias = a_log_bias_.get<float>();
      d.state = dn_state_layer(w.sub);
      d.state_stride = static_cast<int64_t>(kStateFloats);
      d.z = z_.get<std::uint16_t>();
      d.z_stride = VAL;
      d.norm_weight = w.dn_norm;
      if (fused_dn_step_) {
        spk_check(spk_deltanet_inproj_step(&in, outs, &d, dn_arrive_.get<std::int32_t>(), S(stream_)),
                  "deltanet projections + decode step");
      } else {
        spk_check(spk_gemv_fused(&in, outs, 4, S(stream_)), "deltanet projections");
        spk_check(spk_deltanet_decode_step(&d, S(stream_)), "deltanet decode step");
      }
      SpkGemvInput oi{};
      oi.kind = SPK_GEMV_IN_PLAIN;
      oi.in_dim = VAL;
      oi.x = qkv_.get<std::uint16_t>() + 4096;
      const SpkGemvOutput oo{w.dn_out, h, h, static_cast<int32_t>(H), nullptr};
      spk_check(spk_gemv_fused(&oi, &oo, 1, S(stream_)), "out_proj");
    } else {
      const SpkGemvOutput outs[3] = {{w.attn_q, qg_.get<std::uint16_t>(), nullptr, 4096, nullptr},
                                     {w.attn_k, k_.get<std::uint16_t>(), nullptr, 512, nullptr},
                                     {w.attn_v, v_.get<std::uint16_t>(), nullptr, 512, nullptr}};
      SpkAttnArgs aa{};
      aa.qg = qg_.get<std::uint16_t>();
      aa.k = k_.get<std::uint16_t>();
      aa.v = v_.get<std::uint16_t>();
      aa.q_norm_w = w.attn_q_norm;
      aa.k_norm_w = w.attn_k_norm;
      aa.rope = rope_.get<float>();
      aa.kv_cache = kv_layer(w.sub);
      aa.max_seq = static_cast<int32_t>(max_seq_);
      aa.pos_dev = pos_.get<std::int32_t>();
      aa.out = attn_out_.get<std::uint16_t>();
      aa.workspace = attn_ws_.get();
      aa.workspace_bytes = attn_ws_.bytes();
      // the projections, reading the layer's cached K/V rows into the caches
      // for the attention launch (about 0.5 us off its K/V staging)
      spk_check(spk_attention_inproj(&in, outs, &aa, S(stream_)), "attention projections");
      // attention blocks (the last block workgroup of each KV head combines
      // the blocks and applies the sigmoid gate), then o_proj + residual
      const SpkGemvOutput oo{w.attn_o, h, h, static_cast<int32_t>(H), nullptr};
      spk_check(spk_attention_decode_oproj(&aa, &oo, S(stream_)), "attention decode + o_proj");
    }
    SpkGemvInput mi{};
    mi.kind = SPK_GEMV_IN_RMSNORM;
    mi.in_dim = H;
    mi.x = h;
    mi.x2 = w.post_norm;
    // gate/up matvecs with silu_gate.comp fused: m = fp16(silu(gate) * up)
    const SpkGemvOutput mo{w.mlp_gate, gate_.get<std::uint16_t>(), nullptr, static_cast<int32_t>(INTER), w.mlp_up};
    spk_check(spk_gemv_fused(&mi, &mo, 1, S(stream_)), "gate/up");
    SpkGemvInput di{};
    di.kind = SPK_GEMV_IN_PLAIN;
    di.in_dim = INTER;
    di.x = gate_.get<std::uint16_t>();
    const SpkGemvOutput dout{w.mlp_down, h, h, static_cast<int32_t>(H), nullptr};
    spk_check(spk_gemv_fused(&di, &dout, 1, S(stream_)), "down_proj");
    mark(L + 1);
  }
  // final norm + lm_head + argmax + the token's bookkeeping
  lm_head_token(h, reinterpret_cast<std::uint32_t*>(tok), true);
}

// Final norm, lm_head and argmax of hidden row h; the token goes to *tok and
// is recorded in the history (count, position).  One launch by default
// (spk_lm_head_argmax_take: per-workgroup key slots, taken by an extra last
// workgroup; config 4 measured 651 vs 660 us per token for the key launch then
// the take, same build and box), else the pair; with region marks, "lm_head"
// ends after the first launch and "argmax" after the take (in the one-launch
// form the two marks are back to back, so "argmax" is the marks' own gap).
void Qwen35Session::lm_head_token(const std::uint16_t* h, std::uint32_t* tok, bool marks) {
  const int32_t vocab = static_cast<int32_t>(shape_.vocab);
  std::int32_t* hist = history_.get<std::int32_t>();
  const std::size_t NL = layers_.size();
  if (lm_one_launch_) {
    spk_check(spk_lm_head_argmax_take(embed_, h, final_norm_, vocab, H, logits_.get<std::uint16_t>(),
                                      take_slots_.get<std::uint64_t>(), take_slots_.bytes() / 8, tok,
                                      pos_.get<std::int32_t>(), hist, hist + 64,
                                      static_cast<int32_t>(history_cap_), S(stream_)),
              "lm_head + argmax");
    if (marks) {
      mark(NL + 1);
      mark(NL + 2);
    }
    return;
  }
  spk_check(spk_lm_head_argmax_key(embed_, h, final_norm_, vocab, H, logits_.get<std::uint16_t>(),
                                   argmax_key_.get<std::uint64_t>(), S(stream_)),
            "lm_head");
  if (marks) mark(NL + 1);
  spk_check(spk_argmax_key_take(argmax_key_.get<std::uint64_t>(), vocab, tok, pos_.get<std::int32_t>(), hist,
                                hist + 64, static_cast<int32_t>(history_cap_), S(stream_)),
            "argmax take");
  if (marks) mark(NL + 2);
}

void Qwen35Session::ensure_graph() {
  if (!use_graph_ || graph_exec_) return;
  // Every argument of the step is a fixed device address (token id and
  // position are read on the device), so one recording serves every token.
  hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  try {
    enqueue_decode_step();
  } catch (...) {
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(stream_, &g);
    if (g) (void)hipGraphDestroy(g);
    throw;
  }
  hip_check(hipStreamEndCapture(stream_, &graph_), "hipStreamEndCapture");
  hip_check(hipGraphInstantiate(&graph_exec_, graph_, nullptr, nullptr, 0), "hipGraphInstantiate");
}

void Qwen35Session::run_decode_step() {
  if (!use_graph_) {
    enqueue_decode_step();
    return;
  }
  ensure_graph();
  hip_check(hipGraphLaunch(graph_exec_, stream_), "hipGraphLaunch");
}

std::vector<std::uint32_t> Qwen35Session::decode_steps(std::uint32_t n) {
  if (n == 0) return {};
  if (std::size_t(pos_host_) + n > max_seq_)
    throw std::runtime_error("decode: position " + std::to_string(pos_host_ + n) + " exceeds max_seq " +
                             std::to_string(max_seq_));
  if (std::size_t(history_len_) + n > history_cap_) throw std::runtime_error("decode: token history full");
  for (std::uint32_t i = 0; i < n; ++i) run_decode_step();
  std::vector<std::int32_t> out(n);
  hip_check(hipMemcpyAsync(out.data(), history_.get<std::int32_t>() + 64 + history_len_, n * 4, hipMemcpyDeviceToHost,
                           stream_),
            "download tokens");
  hip_check(hipStreamSynchronize(stream_), "decode");
  pos_host_ += static_cast<std::int32_t>(n);
  history_len_ += n;
  return std::vector<std::uint32_t>(out.begin(), out.end());
}

DecodeResult Qwen35Session::decode(const std::vector<std::uint32_t>& prompt_tokens, std::uint32_t max_new_tokens) {
  DecodeResult r;
  r.prompt_tokens = prompt_tokens;
  const auto t0 = std::chrono::steady_clock::now();
  reset();
  if (max_new_tokens == 0) return r;
  const std::uint32_t first = prefill(prompt_tokens);
  r.prefill_ms = ms_since(t0);
  r.gpu_prefill_us = last_gpu_prefill_ms_ * 1000.0;
  r.generated_tokens.push_back(first);
  if (max_new_tokens > 1) {
    const std::uint32_t n = max_new_tokens - 1;
    if (std::size_t(pos_host_) + n > max_seq_)
      throw std::runtime_error("decode: position " + std::to_string(pos_host_ + n) + " exceeds max_seq " +
                               std::to_string(max_seq_));
    if (std::size_t(history_len_) + n > history_cap_) throw std::runtime_error("decode: token history full");
    const bool regions = gpu_ts_ == GpuTimestamps::per_region;
    const bool timed = gpu_ts_ != GpuTimestamps::off;
    // Events of one step: per region, start + one after each layer, lm_head
    // and argmax; per token, start and end.  Steps are timed in batches of
    // kTsBatch over two alternating event sets: the host reads batch k (its
    // last event completed) while the GPU runs batch k+1, so the pool stays
    // at 2 x kTsBatch steps' events however many tokens are generated.
    const std::size_t NL = layers_.size();
    const std::size_t per_step = regions ? NL + 3 : 2;
    constexpr std::uint32_t kTsBatch = 64;
    if (timed) ensure_ts_events(2 * kTsBatch * per_step);
    if (regions) {
      for (std::size_t L = 0; L < NL; ++L) r.gpu_region_us.emplace_back("layer_" + std::to_string(L), 0.0);
      r.gpu_region_us.emplace_back("lm_head", 0.0);
      r.gpu_region_us.emplace_back("argmax", 0.0);
    }
    auto step_events = [&](std::uint32_t i) { return &ts_events_[(((i / kTsBatch) & 1u) * kTsBatch + i % kTsBatch) * per_step]; };
    auto us = [&](hipEvent_t a, hipEvent_t b) {
      float v = 0.0f;
      hip_check(hipEventElapsedTime(&v, a, b), "hipEventElapsedTime");
      return double(v) * 1000.0;
    };
    std::uint32_t collected = 0;  // steps whose times have been read
    auto collect = [&](std::uint32_t upto) {  // reads steps [collected, upto), in order
      if (collected >= upto) return;
      hip_check(hipEventSynchronize(step_events(upto - 1)[per_step - 1]), "hipEventSynchronize");
      for (; collected < upto; ++collected) {
        hipEvent_t* e = step_events(collected);
        r.per_token_gpu_us.push_back(us(e[0], e[per_step - 1]));
        if (regions)
          for (std::size_t k = 0; k < NL + 2; ++k) r.gpu_region_us[k].second += us(e[k], e[k + 1]);
      }
    };
    if (!regions) ensure_graph();  // recorded outside the timed region
    EventTimer ev;
    const auto t1 = std::chrono::steady_clock::now();
    hip_check(hipEventRecord(ev.a, stream_), "hipEventRecord");
    for (std::uint32_t i = 0; i < n; ++i) {
      // this step reuses the event set of step i - 2 kTsBatch: read that batch first
      if (timed && i % kTsBatch == 0 && i >= 2 * kTsBatch) collect(i - kTsBatch);
      if (regions) {
        // cleared on every exit, so a later graph capture never records events
        struct MarksGuard {
          hipEvent_t*& m;
          ~MarksGuard() { m = nullptr; }
        } guard{marks_};
        marks_ = step_events(i);
        enqueue_decode_step();
      } else {
        if (timed) hip_check(hipEventRecord(step_events(i)[0], stream_), "hipEventRecord");
        run_decode_step();
        if (timed) hip_check(hipEventRecord(step_events(i)[1], stream_), "hipEventRecord");
      }
    }
    hip_check(hipEventRecord(ev.b, stream_), "hipEventRecord");
    std::vector<std::int32_t> out(n);
    hip_check(hipMemcpyAsync(out.data(), history_.get<std::int32_t>() + 64 + history_len_, n * 4,
                             hipMemcpyDeviceToHost, stream_),
              "download tokens");
    hip_check(hipStreamSynchronize(stream_), "decode");
    r.decode_ms = ms_since(t1);
    r.gpu_decode_us = ev.ms() * 1000.0;
    if (timed) collect(n);
    pos_host_ += static_cast<std::int32_t>(n);
    history_len_ += n;
    for (auto t : out) r.generated_tokens.push_back(static_cast<std::uint32_t>(t));
    r.decode_steps = n;
  }
  r.used_graph = use_graph_ && gpu_ts_ != GpuTimestamps::per_region;
  r.elapsed_ms = ms_since(t0);
  return r;
}

void Qwen35Session::get_state(float* dn_state, std::uint16_t* conv, std::uint16_t* kv, std::int32_t* pos,
                              std::int32_t* last_token) {
  hip_check(hipStreamSynchronize(stream_), "get_state");
  for (std::uint32_t i = 0; i < n_dn_ && dn_state; ++i)
    hip_check(hipMemcpy(dn_state + std::size_t(i) * 16 * 128 * 128, dn_state_layer(i), std::size_t(16) * 128 * 128 * 4,
                        hipMemcpyDeviceToHost),
              "download state");
  if (conv && n_dn_) conv_state_.download(conv, std::size_t(n_dn_) * CONV * 4 * 2);
  if (kv && n_attn_) kv_cache_.download(kv, std::size_t(n_attn_) * max_seq_ * 1024 * 2);
  if (pos) *pos = pos_host_;
  if (last_token) tok_.download(last_token, 4);
}

void Qwen35Session::set_state(const float* dn_state, const std::uint16_t* conv, const std::uint16_t* kv,
                              std::int32_t pos, std::int32_t last_token) {
  if (pos < 0 || static_cast<std::uint32_t>(pos) >= max_seq_) throw std::runtime_error("set_state: position out of range");
  if (last_token < 0 || static_cast<std::uint32_t>(last_token) >= shape_.vocab)
    throw std::runtime_error("set_state: token out of range");
  hip_check(hipStreamSynchronize(stream_), "set_state");
  for (std::uint32_t i = 0; i < n_dn_ && dn_state; ++i)
    hip_check(hipMemcpy(dn_state_layer(i), dn_state + std::size_t(i) * 16 * 128 * 128, std::size_t(16) * 128 * 128 * 4,
                        hipMemcpyHostToDevice),
              "upload state");
  if (conv && n_dn_) conv_state_.upload(conv, std::size_t(n_dn_) * CONV * 4 * 2);
  if (kv && n_attn_) kv_cache_.upload(kv, std::size_t(n_attn_) * max_seq_ * 1024 * 2);
  pos_.upload(&pos, 4);
  tok_.upload(&last_token, 4);
  const std::int32_t zero = 0;
  history_.upload(&zero, 4);
  pos_host_ = pos;
  history_len_ = 0;
}

void Qwen35Session::last_output(std::uint16_t* logits, std::uint16_t* hidden) {
  hip_check(hipStreamSynchronize(stream_), "last_output");
  if (logits) logits_.download(logits, std::size_t(shape_.vocab) * 2);
  if (hidden) h_.download(hidden, H * 2);
}

}  // namespace spock::hip

// ---------------------------------------------------------------------------
// C ABI (include/spock_model.h)
// ---------------------------------------------------------------------------

struct SpkModel {
  std::unique_ptr<spock::hip::Qwen35Session> s;
  spock::hip::DecodeResult last;  // timings of the last spk_model_generate call
};

namespace {
thread_local std::string g_model_error;

template <typename F>
int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_model_error = e.what();
    return -1;
  }
}
}  // namespace

extern "C" const char* spk_model_last_error(void) { return g_model_error.c_str(); }

extern "C" SpkModel* spk_model_open(const char* repack_dir, int32_t max_seq, int32_t flags) {
  SpkModel* m = nullptr;
  const int rc = guarded([&] {
    if (!repack_dir) throw std::runtime_error("spk_model_open: NULL directory");
    if (flags & ~(SPK_MODEL_NO_GRAPH | SPK_MODEL_MATRIX_PREFILL | SPK_MODEL_GPU_TIMESTAMPS | SPK_MODEL_GPU_REGIONS |
                  SPK_MODEL_LMHEAD_ONE_LAUNCH | SPK_MODEL_SPLIT_DN_STEP | SPK_MODEL_LMHEAD_KEY_TAKE))
      throw std::runtime_error("spk_model_open: unknown flags");
    using spock::hip::GpuTimestamps;
    const GpuTimestamps ts = (flags & SPK_MODEL_GPU_REGIONS)      ? GpuTimestamps::per_region
                             : (flags & SPK_MODEL_GPU_TIMESTAMPS) ? GpuTimestamps::per_token
                                                                  : GpuTimestamps::off;
    auto s = std::make_unique<spock::hip::Qwen35Session>(repack_dir, false,
                                                         max_seq > 0 ? static_cast<std::uint32_t>(max_seq) : 0u,
                                                         (flags & SPK_MODEL_NO_GRAPH) == 0,
                                                         (flags & SPK_MODEL_MATRIX_PREFILL) == 0, ts,
                                                         (flags & SPK_MODEL_LMHEAD_KEY_TAKE) == 0,
                                                         (flags & SPK_MODEL_SPLIT_DN_STEP) == 0);
    m = new SpkModel{std::move(s), {}};
  });
  return rc == 0 ? m : nullptr;
}

extern "C" void spk_model_close(SpkModel* m) { delete m; }

extern "C" int spk_model_info(const SpkModel* m, int32_t* layers, int32_t* vocab, int32_t* max_seq) {
  return guarded([&] {
    if (!m) throw std::runtime_error("spk_model_info: NULL session");
    if (layers) *layers = static_cast<int32_t>(m->s->shape().layers);
    if (vocab) *vocab = static_cast<int32_t>(m->s->shape().vocab);
    if (max_seq) *max_seq = static_cast<int32_t>(m->s->max_seq());
  });
}

extern "C" int spk_model_reset(SpkModel* m) {
  return guarded([&] {
    if (!m) throw std::runtime_error("spk_model_reset: NULL session");
    m->s->reset();
  });
}

extern "C" int spk_model_generate(SpkModel* m, const int32_t* prompt, int32_t prompt_len, int32_t max_new,
                                  int32_t* out_tokens, SpkGenerateStats* stats) {
  return guarded([&] {
    if (!m || !prompt || (max_new > 0 && !out_tokens)) throw std::runtime_error("spk_model_generate: NULL argument");
    if (prompt_len <= 0 || max_new < 0) throw std::runtime_error("spk_model_generate: bad lengths");
    std::vector<std::uint32_t> p;
    for (int32_t i = 0; i < prompt_len; ++i) {
      if (prompt[i] < 0) throw std::runtime_error("spk_model_generate: negative token id");
      p.push_back(static_cast<std::uint32_t>(prompt[i]));
    }
    m->last = m->s->decode(p, static_cast<std::uint32_t>(max_new));
    const spock::hip::DecodeResult& r = m->last;
    for (std::size_t i = 0; i < r.generated_tokens.size(); ++i) out_tokens[i] = static_cast<int32_t>(r.generated_tokens[i]);
    if (stats) {
      stats->prefill_ms = r.prefill_ms;
      stats->decode_ms = r.decode_ms;
      stats->gpu_prefill_ms = r.gpu_prefill_us / 1000.0;
      stats->gpu_decode_ms = r.gpu_decode_us / 1000.0;
      stats->decode_steps = static_cast<int32_t>(r.decode_steps);
      stats->used_graph = r.used_graph ? 1 : 0;
    }
  });
}

extern "C" int spk_model_gpu_token_us(const SpkModel* m, double* us, int32_t capacity, int32_t* count) {
  return guarded([&] {
    if (!m || !count || (capacity > 0 && !us)) throw std::runtime_error("spk_model_gpu_token_us: NULL argument");
    const auto& v = m->last.per_token_gpu_us;
    *count = static_cast<int32_t>(v.size());
    for (std::size_t i = 0; i < v.size() && i < std::size_t(capacity > 0 ? capacity : 0); ++i) us[i] = v[i];
  });
}

extern "C" int spk_model_gpu_region_count(const SpkModel* m, int32_t* count) {
  return guarded([&] {
    if (!m || !count) throw std::runtime_error("spk_model_gpu_region_count: NULL argument");
    *count = static_cast<int32_t>(m->last.gpu_region_us.size());
  });
}

extern "C" int spk_model_gpu_region(const SpkModel* m, int32_t index, const char** name, double* us) {
  return guarded([&] {
    if (!m || !name || !us) throw std::runtime_error("spk_model_gpu_region: NULL argument");
    const auto& v = m->last.gpu_region_us;
    if (index < 0 || std::size_t(index) >= v.size())
      throw std::runtime_error("spk_model_gpu_region: index " + std::to_string(index) + " of " +
                               std::to_string(v.size()) + " regions");
    *name = v[index].first.c_str();
    *us = v[index].second;
  });
}

extern "C" int spk_model_prefill(SpkModel* m, const int32_t* prompt, int32_t prompt_len, int32_t* out_token) {
  return guarded([&] {
    if (!m || !prompt) throw std::runtime_error("spk_model_prefill: NULL argument");
    if (prompt_len <= 0) throw std::runtime_error("spk_model_prefill: empty prompt");
    std::vector<std::uint32_t> p;
    for (int32_t i = 0; i < prompt_len; ++i) {
      if (prompt[i] < 0) throw std::runtime_error("spk_model_prefill: negative token id");
      p.push_back(static_cast<std::uint32_t>(prompt[i]));
    }
    const std::uint32_t t = m->s->prefill(p);
    if (out_token) *out_token = static_cast<int32_t>(t);
  });
}

extern "C" int spk_model_decode(SpkModel* m, int32_t n_steps, int32_t* out_tokens) {
  return guarded([&] {
    if (!m || (n_steps > 0 && !out_tokens)) throw std::runtime_error("spk_model_decode: NULL argument");
    if (n_steps < 0) throw std::runtime_error("spk_model_decode: negative step count");
    const auto t = m->s->decode_steps(static_cast<std::uint32_t>(n_steps));
    for (std::size_t i = 0; i < t.size(); ++i) out_tokens[i] = static_cast<int32_t>(t[i]);
  });
}

extern "C" int spk_model_state_sizes(const SpkModel* m, size_t* dn_state_bytes, size_t* conv_bytes, size_t* kv_bytes) {
  return guarded([&] {
    if (!m) throw std::runtime_error("spk_model_state_sizes: NULL session");
    if (dn_state_bytes) *dn_state_bytes = std::size_t(m->s->num_deltanet_layers()) * 16 * 128 * 128 * 4;
    if (conv_bytes) *conv_bytes = std::size_t(m->s->num_deltanet_layers()) * 6144 * 4 * 2;
    if (kv_bytes) *kv_bytes = std::size_t(m->s->num_attention_layers()) * m->s->max_seq() * 1024 * 2;
  });
}

extern "C" int spk_model_get_state(SpkModel* m, void* dn_state, void* conv, void* kv, int32_t* pos,
                                   int32_t* last_token) {
  return guarded([&] {
    if (!m) throw std::runtime_error("spk_model_get_state: NULL session");
    m->s->get_state(static_cast<float*>(dn_state), static_cast<std::uint16_t*>(conv), static_cast<std::uint16_t*>(kv),
                    pos, last_token);
  });
}

extern "C" int spk_model_set_state(SpkModel* m, const void* dn_state, const void* conv, const void* kv, int32_t pos,
                                   int32_t last_token) {
  return guarded([&] {
    if (!m) throw std::runtime_error("spk_model_set_state: NULL session");
    m->s->set_state(static_cast<const float*>(dn_state), static_cast<const std::uint16_t*>(conv),
                    static_cast<const std::uint16_t*>(kv), pos, last_token);
  });
}

extern "C" int spk_model_last_output(SpkModel* m, uint16_t* logits, uint16_t* hidden) {
  return guarded([&] {
    if (!m) throw std::runtime_error("spk_model_last_output: NULL session");
    m->s->last_output(logits, hidden);
  });
}

extern "C" int spk_artifact_write_synthetic(const char* dir, int32_t layers, int32_t vocab, uint64_t seed) {
  return guarded([&] {
    if (!dir) throw std::runtime_error("spk_artifact_write_synthetic: NULL directory");
    if (layers <= 0 || vocab <= 0) throw std::runtime_error("spk_artifact_write_synthetic: bad shape");
    spock::hip::Qwen35Shape s;
    s.layers = static_cast<std::uint32_t>(layers);
    s.vocab = static_cast<std::uint32_t>(vocab);
    spock::hip::write_synthetic_artifact(dir, s, seed);
  });
}
