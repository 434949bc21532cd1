// qwen_decode.hpp -- header-only C++ wrappers over the C ABI in qwen_decode.h.
//
// They keep the method shapes and semantics of the reference's host classes
// so the reference's decode driver (benchmarks/triton_mini_decoder_layer.cpp:
// 1051-1068) ports call for call:
//   qd::DecoderLayer  ~ examples/triton/mini_decoder_layer.hpp:179-768
//                       (copy_hidden_state, decode_to_hidden_state,
//                       decode_to_buffer, copy_inputs' KV half)
//   qd::ModelTail     ~ examples/triton/mini_decoder_layer.hpp:770-894
//                       (hidden_buffer, run, copy_logits, copy_hidden) + the
//                       host top-1 of benchmarks/triton_mini_decoder_layer.cpp:394-422
//   qd::ResidentExecutor ~ include/lrrt/persistent_graph/resident_executor.hpp:268-475
//                       (initialize, launch, read_state)
// One difference: the layers of a sequence slot share one device hidden
// vector, so a hand-off's destination position is the query's own.
// Errors surface as qd::Error (a std::runtime_error carrying the status), the
// way the reference's C++ layer throws lrrt::Error (include/lrrt/error.hpp:10-27).
#pragma once

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "qwen_decode.h"

namespace qd {

class Error : public std::runtime_error {
 public:
  Error(qd_status status, const std::string &what)
      : std::runtime_error(what), status_(status) {}
  qd_status status() const noexcept { return status_; }

 private:
  qd_status status_;
};

inline void check(qd_status status) {
  if (status != QD_SUCCESS) {
    const char *detail = qd_last_error();
    throw Error(status, std::string(qd_status_string(status)) + ": " +
                            (detail && *detail ? detail : "no detail"));
  }
}

// Default configuration: the Qwen2.5-0.5B shape.
inline qd_config qwen25_05b_config(uint32_t capacity = 4096,
                                   uint32_t max_batch = 1) {
  qd_config c{};
  c.hidden = 896;
  c.heads = 14;
  c.kv_heads = 2;
  c.head_dim = 64;
  c.intermediate = 4864;
  c.vocab = 151936;
  c.layers = 24;
  c.capacity = capacity;
  c.max_batch = max_batch;
  c.tied_lm_head = 1;
  c.rms_eps = 1e-6f;
  c.rope_theta = 1e6f;
  c.device = 0;
  return c;
}

// Owns one engine: resident weights, KV cache and decode state on one GPU.
class Engine {
 public:
  explicit Engine(const qd_config &config) {
    qd_engine *e = nullptr;
    check(qd_engine_create(&config, &e));
    engine_.reset(e);
  }
  Engine(const Engine &) = delete;
  Engine &operator=(const Engine &) = delete;
  Engine(Engine &&) = default;
  Engine &operator=(Engine &&) = default;

  qd_engine *get() const noexcept { return engine_.get(); }

  qd_config config() const {
    qd_config c{};
    check(qd_engine_config(get(), &c));
    return c;
  }
  uint64_t device_bytes() const {
    uint64_t b = 0;
    check(qd_engine_device_bytes(get(), &b));
    return b;
  }
  uint32_t resident_grid() const {
    uint32_t g = 0;
    check(qd_engine_resident_grid(get(), &g));
    return g;
  }

  void load_bundle(const std::string &directory) {
    check(qd_load_bundle(get(), directory.c_str()));
  }
  void load_synthetic(uint64_t seed, float weight_std = 0.02f,
                      float bias_std = 0.01f, float norm_gain = 1.0f) {
    const qd_synthetic_init init{weight_std, bias_std, norm_gain, 0.f};
    check(qd_load_synthetic(get(), seed, &init));
  }

  void kv_reset(uint32_t seq, uint32_t position) {
    check(qd_kv_reset(get(), seq, position));
  }

  // One full decode step; returns the greedy token. logits may be null.
  uint32_t step(uint32_t seq, uint32_t token, std::vector<float> *logits = nullptr,
                float *top_logit = nullptr) {
    if (logits) logits->resize(config().vocab);
    uint32_t greedy = 0;
    check(qd_step(get(), seq, token, logits ? logits->data() : nullptr, &greedy,
                  top_logit));
    return greedy;
  }
  // The same step replayed from the slot's captured HIP graph (qd_step_graph).
  uint32_t step_graph(uint32_t seq, uint32_t token, std::vector<float> *logits = nullptr,
                      float *top_logit = nullptr) {
    if (logits) logits->resize(config().vocab);
    uint32_t greedy = 0;
    check(qd_step_graph(get(), seq, token, logits ? logits->data() : nullptr, &greedy,
                        top_logit));
    return greedy;
  }

  uint32_t prefill(uint32_t seq, const std::vector<uint32_t> &tokens,
                   std::vector<float> *last_logits = nullptr,
                   float *top_logit = nullptr) {
    if (last_logits) last_logits->resize(config().vocab);
    uint32_t greedy = 0;
    check(qd_prefill(get(), seq, tokens.data(), static_cast<uint32_t>(tokens.size()),
                     last_logits ? last_logits->data() : nullptr, &greedy,
                     top_logit));
    return greedy;
  }

  void sync() { check(qd_sync(get())); }

 private:
  struct Destroy {
    void operator()(qd_engine *e) const noexcept { (void)qd_engine_destroy(e); }
  };
  std::unique_ptr<qd_engine, Destroy> engine_;
};

class ModelTail;

// The hidden vector a ModelTail reads (the reference's
// ModelTail::hidden_buffer()): the slot's device hidden vector, which the
// last layer's decode_to_buffer writes.
struct HiddenBuffer {
  Engine *engine;
  uint32_t seq;
};

// One decoder layer of one sequence slot, with the reference DecoderLayer's
// decode methods (examples/triton/mini_decoder_layer.hpp:286-372). The
// engine keeps one hidden vector per slot on the device: each layer reads
// it and leaves its output there for the next, so a hand-off never
// touches the host, and `dst_position` must be the query position
// valid_keys - 1 (the one row the slot holds).
class DecoderLayer {
 public:
  DecoderLayer(Engine &engine, uint32_t layer, uint32_t seq = 0)
      : engine_(&engine), layer_(layer), seq_(seq) {}

  uint32_t layer() const noexcept { return layer_; }
  uint32_t seq() const noexcept { return seq_; }

  // KV half of DecoderLayer::copy_inputs: token-major [count][kv_heads*64].
  void copy_kv(uint32_t start, uint32_t count, const std::vector<float> &k,
               const std::vector<float> &v) {
    check(qd_write_kv(engine_->get(), seq_, layer_, start, count, k.data(), v.data()));
  }
  // DecoderLayer::copy_hidden_state: the input row of the token at
  // `position` (the slot's one hidden row).
  void copy_hidden_state(uint32_t position, const std::vector<float> &hidden_state) {
    if (position >= engine_->config().capacity)
      throw Error(QD_ERROR_INVALID_ARGUMENT, "hidden state position is out of range");
    if (hidden_state.size() != engine_->config().hidden)
      throw Error(QD_ERROR_INVALID_ARGUMENT, "hidden state row shape mismatch");
    check(qd_load_hidden(engine_->get(), seq_, hidden_state.data()));
  }
  // The same row from the engine's embedding table, looked up on the device.
  void embed_token(uint32_t position, uint32_t token) {
    if (position >= engine_->config().capacity)
      throw Error(QD_ERROR_INVALID_ARGUMENT, "hidden state position is out of range");
    check(qd_embed_hidden(engine_->get(), seq_, token));
  }
  // Decodes the query at valid_keys - 1 (K/V row written there, attention
  // over 0..valid_keys - 1) into dst's input on the device.
  void decode_to_hidden_state(uint32_t valid_keys, DecoderLayer &dst, uint32_t dst_position) {
    if (dst.engine_ != engine_ || dst.seq_ != seq_)
      throw Error(QD_ERROR_INVALID_ARGUMENT,
                  "direct handoff requires a layer of the same engine and sequence slot");
    if (valid_keys == 0 || dst_position != valid_keys - 1)
      throw Error(QD_ERROR_INVALID_ARGUMENT,
                  "direct handoff position must be the query position valid_keys - 1");
    check(qd_layer_decode(engine_->get(), seq_, layer_, 1, valid_keys));
  }
  // The same into the model tail's input (the last layer of a stack).
  void decode_to_buffer(uint32_t valid_keys, const HiddenBuffer &dst) {
    if (dst.engine != engine_ || dst.seq != seq_)
      throw Error(QD_ERROR_INVALID_ARGUMENT,
                  "direct output buffer must be the same engine and sequence slot's tail");
    check(qd_layer_decode(engine_->get(), seq_, layer_, 1, valid_keys));
  }
  // The layer's output row (the slot's hidden vector) on the host.
  void copy_output(std::vector<float> &hidden) const {
    hidden.resize(engine_->config().hidden);
    check(qd_read_activation(engine_->get(), seq_, 0, hidden.data(), hidden.size()));
  }
  void synchronize() { engine_->sync(); }

 private:
  Engine *engine_;
  uint32_t layer_;
  uint32_t seq_;
};

// Final RMSNorm + LM head + greedy top-1 of one sequence slot, with the
// reference ModelTail's methods (examples/triton/mini_decoder_layer.hpp:
// 770-894); run() takes no token: it reads the hidden vector the last
// decoder layer left, and completes that token (the slot's position
// advances by one).
class ModelTail {
 public:
  explicit ModelTail(Engine &engine, uint32_t seq = 0) : engine_(&engine), seq_(seq) {}

  HiddenBuffer hidden_buffer() const { return HiddenBuffer{engine_, seq_}; }
  void run() { check(qd_tail(engine_->get(), seq_, nullptr, &top_token_, &top_logit_)); }
  void synchronize() { engine_->sync(); }
  void copy_logits(std::vector<float> &out) const {
    if (out.size() != engine_->config().vocab)
      throw Error(QD_ERROR_INVALID_ARGUMENT, "model tail logits shape mismatch");
    check(qd_read_logits(engine_->get(), seq_, out.data(), out.size()));
  }
  void copy_hidden(std::vector<float> &out) const {
    if (out.size() != engine_->config().hidden)
      throw Error(QD_ERROR_INVALID_ARGUMENT, "model tail hidden shape mismatch");
    check(qd_read_activation(engine_->get(), seq_, 0, out.data(), out.size()));
  }
  // Greedy token and its logit of the last run() (the device argmax: the
  // largest logit, the lowest index on ties).
  uint32_t top_token() const noexcept { return top_token_; }
  float top_logit() const noexcept { return top_logit_; }

 private:
  Engine *engine_;
  uint32_t seq_;
  uint32_t top_token_ = 0;
  float top_logit_ = 0.f;
};

// Device-resident greedy generation (the persistent executor's role).
class ResidentExecutor {
 public:
  explicit ResidentExecutor(Engine &engine, uint32_t seq = 0)
      : engine_(&engine), seq_(seq) {}

  // Sets the slot's position (KV length) and clears its decode state.
  void initialize(uint32_t position) { engine_->kv_reset(seq_, position); }

  struct Result {
    std::vector<uint32_t> tokens;
    qd_stop_reason stop_reason = QD_STOP_NONE;
  };
  // Consumes first_token, feeds every argmax back on the device.
  Result launch(uint32_t first_token, uint32_t max_tokens,
                uint32_t eos = UINT32_MAX, std::vector<float> *all_logits = nullptr) {
    Result r;
    r.tokens.resize(max_tokens);
    if (all_logits)
      all_logits->resize(static_cast<size_t>(max_tokens) * engine_->config().vocab);
    uint32_t generated = 0, stop = 0;
    check(qd_generate_resident(engine_->get(), seq_, first_token, max_tokens, eos,
                               r.tokens.data(), &generated, &stop,
                               all_logits ? all_logits->data() : nullptr));
    r.tokens.resize(generated);
    r.stop_reason = static_cast<qd_stop_reason>(stop);
    return r;
  }
  qd_decode_state read_state() const {
    qd_decode_state s{};
    check(qd_read_decode_state(engine_->get(), seq_, &s));
    return s;
  }
  qd_timing last_timing() const {
    qd_timing t{};
    check(qd_last_timing(engine_->get(), &t));
    return t;
  }

 private:
  Engine *engine_;
  uint32_t seq_;
};

}  // namespace qd
