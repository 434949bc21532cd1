// qwen_decode.hpp -- header-only C++ wrappers over the C ABI in qwen_decode.h.
//
// They keep the method shapes of the reference's host classes so a driver
// written against them ports call for call:
//   qd::DecoderLayer  ~ examples/triton/mini_decoder_layer.hpp:179-768
//                       (decode_to_hidden_state, copy_inputs' KV half)
//   qd::ModelTail     ~ examples/triton/mini_decoder_layer.hpp:770-894
//                       (run, copy_logits) + host top-1 of
//                       benchmarks/triton_mini_decoder_layer.cpp:394-422
//   qd::ResidentExecutor ~ include/lrrt/persistent_graph/resident_executor.hpp:268-475
//                       (initialize, launch, read_state)
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

// One decoder layer of an engine, driven on a host hidden vector
// (the reference's DecoderLayer::decode_to_hidden_state).
class DecoderLayer {
 public:
  DecoderLayer(Engine &engine, uint32_t layer, uint32_t seq = 0)
      : engine_(&engine), layer_(layer), seq_(seq) {}

  // KV half of DecoderLayer::copy_inputs: token-major [count][kv_heads*64].
  void copy_kv(uint32_t start, uint32_t count, const std::vector<float> &k,
               const std::vector<float> &v) {
    check(qd_write_kv(engine_->get(), seq_, layer_, start, count, k.data(), v.data()));
  }
  // Runs the layer at the slot's position; hidden is updated in place.
  void decode_to_hidden_state(std::vector<float> &hidden) {
    check(qd_layer_step(engine_->get(), seq_, layer_, hidden.data()));
  }
  void synchronize() { engine_->sync(); }

 private:
  Engine *engine_;
  uint32_t layer_;
  uint32_t seq_;
};

// Final norm + LM head + top-1 for one sequence slot (ModelTail::run,
// copy_logits and the host top-1 in one call per token).
class ModelTail {
 public:
  explicit ModelTail(Engine &engine, uint32_t seq = 0) : engine_(&engine), seq_(seq) {}

  // Consumes `token` through the whole model; keeps the logits.
  uint32_t run(uint32_t token) {
    return top_token_ = engine_->step(seq_, token, &logits_, &top_logit_);
  }
  const std::vector<float> &copy_logits() const { return logits_; }
  uint32_t top_token() const noexcept { return top_token_; }
  float top_logit() const noexcept { return top_logit_; }

 private:
  Engine *engine_;
  uint32_t seq_;
  std::vector<float> logits_;
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
