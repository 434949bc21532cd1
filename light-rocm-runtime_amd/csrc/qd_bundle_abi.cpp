// C-ABI wrappers of the weight-bundle reader/writer (qd_bundle.cpp). Host
// only: usable without a GPU.
#include <cstring>
#include <stdexcept>
#include <string>

#include "qd/qwen_decode.h"
#include "qd_bundle.hpp"

namespace qd {
// Defined in qd_engine.cpp: runs fn, maps exceptions to qd_status and keeps
// the message for qd_last_error().
qd_status guard_call(void (*fn)(void *), void *ctx);
}  // namespace qd

namespace {

template <typename F>
qd_status run(F &&f) {
  return qd::guard_call([](void *p) { (*static_cast<F *>(p))(); }, &f);
}

qd::bundle::LayerShape shape_of(const uint32_t *s) {
  qd::bundle::LayerShape shape;
  shape.keys = s[0];
  shape.hidden = s[1];
  shape.heads = s[2];
  shape.kv_heads = s[3];
  shape.head_dim = s[4];
  shape.intermediate = s[5];
  return shape;
}

}  // namespace

extern "C" {

qd_status qd_bundle_write_layer(const char *manifest, const char *data_name, const uint32_t *shape6,
                                float rope_theta, const float *tensors) {
  return run([&] {
    if (!manifest || !data_name || !shape6 || !tensors) throw std::invalid_argument("null argument");
    qd::bundle::LayerWeights w;
    w.shape = shape_of(shape6);
    w.rope_theta = rope_theta;
    size_t at = 0;
    for (int t = 0; t < qd::bundle::kLayerTensorCount; ++t) {
      const size_t n = qd::bundle::layer_tensor_count(w.shape, t);
      w.tensors[t].assign(tensors + at, tensors + at + n);
      at += n;
    }
    qd::bundle::write_layer(manifest, data_name, w);
  });
}

qd_status qd_bundle_read_layer(const char *manifest, uint32_t *shape6, float *rope_theta, float *tensors,
                               size_t capacity, size_t *count) {
  return run([&] {
    if (!manifest || !shape6 || !rope_theta || !count) throw std::invalid_argument("null argument");
    const qd::bundle::LayerWeights w = qd::bundle::load_layer(manifest);
    const uint32_t s[6] = {w.shape.keys, w.shape.hidden, w.shape.heads,
                           w.shape.kv_heads, w.shape.head_dim, w.shape.intermediate};
    std::memcpy(shape6, s, sizeof(s));
    *rope_theta = w.rope_theta;
    size_t total = 0;
    for (const auto &t : w.tensors) total += t.size();
    *count = total;
    if (total > capacity || (!tensors && total)) throw std::invalid_argument("tensor buffer too small");
    size_t at = 0;
    for (const auto &t : w.tensors) {
      std::memcpy(tensors + at, t.data(), t.size() * sizeof(float));
      at += t.size();
    }
  });
}

qd_status qd_bundle_write_tail(const char *manifest, const char *data_name, uint32_t hidden, uint32_t vocab,
                               const uint32_t *token_ids, size_t token_count, const float *embeddings,
                               const float *final_norm, const float *lm_head) {
  return run([&] {
    if (!manifest || !data_name || !token_ids || !embeddings || !final_norm || !lm_head)
      throw std::invalid_argument("null argument");
    qd::bundle::TailWeights w;
    w.hidden = hidden;
    w.vocab = vocab;
    w.token_ids.assign(token_ids, token_ids + token_count);
    w.token_embeddings.assign(embeddings, embeddings + token_count * hidden);
    w.final_norm_weight.assign(final_norm, final_norm + hidden);
    w.lm_head_weight.assign(lm_head, lm_head + size_t(vocab) * hidden);
    qd::bundle::write_tail(manifest, data_name, w);
  });
}

qd_status qd_bundle_read_tail(const char *manifest, uint32_t *hidden, uint32_t *vocab, uint32_t *token_ids,
                              size_t ids_capacity, size_t *token_count, float *tensors, size_t capacity,
                              size_t *count) {
  return run([&] {
    if (!manifest || !hidden || !vocab || !token_count || !count) throw std::invalid_argument("null argument");
    const qd::bundle::TailWeights w = qd::bundle::load_tail(manifest);
    *hidden = w.hidden;
    *vocab = w.vocab;
    *token_count = w.token_ids.size();
    *count = w.token_embeddings.size() + w.final_norm_weight.size() + w.lm_head_weight.size();
    if (w.token_ids.size() > ids_capacity || *count > capacity || (!token_ids && !w.token_ids.empty()) ||
        (!tensors && *count))
      throw std::invalid_argument("output buffer too small");
    std::memcpy(token_ids, w.token_ids.data(), w.token_ids.size() * 4);
    size_t at = 0;
    for (const auto *v : {&w.token_embeddings, &w.final_norm_weight, &w.lm_head_weight}) {
      std::memcpy(tensors + at, v->data(), v->size() * 4);
      at += v->size();
    }
  });
}

}  // extern "C"
