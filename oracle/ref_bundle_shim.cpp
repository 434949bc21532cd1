// C-ABI shim over the reference's header-only weight-bundle reader/writer
// (/root/reference/executor/qwen/weight_bundle.hpp:460-757). Test
// infrastructure only: oracle/Makefile compiles it, with the reference header
// where it lies, into oracle/_ref/libref_bundle.so, and the CPU tests use it to
// cross-check this build's bundle I/O in both directions.
#include "executor/qwen/weight_bundle.hpp"

#include <cstring>
#include <exception>
#include <string>

namespace {

namespace q = lrrt::executor::qwen;

thread_local std::string g_error;

// Canonical tensor order, matching tensor_specs (weight_bundle.hpp:358-386).
std::vector<float> q::DecoderLayerWeights::*const kLayerFields[] = {
    &q::DecoderLayerWeights::attention_norm_weight,
    &q::DecoderLayerWeights::mlp_norm_weight,
    &q::DecoderLayerWeights::q_weight,
    &q::DecoderLayerWeights::k_weight,
    &q::DecoderLayerWeights::v_weight,
    &q::DecoderLayerWeights::q_bias,
    &q::DecoderLayerWeights::k_bias,
    &q::DecoderLayerWeights::v_bias,
    &q::DecoderLayerWeights::out_weight,
    &q::DecoderLayerWeights::gate_weight,
    &q::DecoderLayerWeights::up_weight,
    &q::DecoderLayerWeights::down_weight,
};

size_t layer_count(const q::DecoderLayerShape &s, int field) {
  const size_t h = s.hidden, qd = size_t(s.heads) * s.head_dim,
               kv = size_t(s.kv_heads) * s.head_dim, i = s.intermediate;
  const size_t counts[] = {h,  h,  qd * h, kv * h, kv * h, qd,
                           kv, kv, h * qd, i * h,  i * h,  h * i};
  return counts[field];
}

} // namespace

extern "C" {

const char *ref_last_error(void) { return g_error.c_str(); }

// shape6 = {keys, hidden, heads, kv_heads, head_dim, intermediate}. Writes
// the 12 tensors concatenated in canonical order. Returns the float count, or
// -1 on a loader error, or -2 if `capacity` is too small.
long long ref_load_layer(const char *manifest, uint32_t *shape6,
                         float *rope_theta, float *out, size_t capacity) {
  try {
    q::DecoderLayerWeights w = q::load_decoder_layer_weights(manifest);
    const uint32_t s[6] = {w.shape.keys,     w.shape.hidden,
                           w.shape.heads,    w.shape.kv_heads,
                           w.shape.head_dim, w.shape.intermediate};
    std::memcpy(shape6, s, sizeof(s));
    *rope_theta = w.rope_theta;
    size_t total = 0;
    for (auto field : kLayerFields) {
      total += (w.*field).size();
    }
    if (total > capacity) {
      return -2;
    }
    size_t at = 0;
    for (auto field : kLayerFields) {
      std::memcpy(out + at, (w.*field).data(), (w.*field).size() * 4);
      at += (w.*field).size();
    }
    return static_cast<long long>(total);
  } catch (const std::exception &e) {
    g_error = e.what();
    return -1;
  }
}

int ref_write_layer(const char *manifest, const char *data_name,
                    const uint32_t *shape6, float rope_theta,
                    const float *tensors) {
  try {
    q::DecoderLayerWeights w{};
    w.shape = {shape6[0], shape6[1], shape6[2],
               shape6[3], shape6[4], shape6[5]};
    w.rope_theta = rope_theta;
    size_t at = 0;
    for (int f = 0; f < 12; ++f) {
      const size_t n = layer_count(w.shape, f);
      (w.*kLayerFields[f]).assign(tensors + at, tensors + at + n);
      at += n;
    }
    q::write_decoder_layer_weights(manifest, data_name, w);
    return 0;
  } catch (const std::exception &e) {
    g_error = e.what();
    return -1;
  }
}

// Tail: writes token_ids into ids (capacity ids_capacity) and the tensors
// embeddings | final_norm | lm_head concatenated into out.
long long ref_load_tail(const char *manifest, uint32_t *hidden,
                        uint32_t *vocab, uint32_t *ids, size_t ids_capacity,
                        size_t *id_count, float *out, size_t capacity) {
  try {
    q::ModelTailWeights w = q::load_model_tail_weights(manifest);
    *hidden = w.hidden;
    *vocab = w.vocab;
    *id_count = w.token_ids.size();
    const size_t total = w.token_embeddings.size() +
                         w.final_norm_weight.size() + w.lm_head_weight.size();
    if (w.token_ids.size() > ids_capacity || total > capacity) {
      return -2;
    }
    std::memcpy(ids, w.token_ids.data(), w.token_ids.size() * 4);
    size_t at = 0;
    for (const std::vector<float> *v :
         {&w.token_embeddings, &w.final_norm_weight, &w.lm_head_weight}) {
      std::memcpy(out + at, v->data(), v->size() * 4);
      at += v->size();
    }
    return static_cast<long long>(total);
  } catch (const std::exception &e) {
    g_error = e.what();
    return -1;
  }
}

int ref_write_tail(const char *manifest, const char *data_name,
                   uint32_t hidden, uint32_t vocab, const uint32_t *ids,
                   size_t id_count, const float *embeddings,
                   const float *final_norm, const float *lm_head) {
  try {
    q::ModelTailWeights w{};
    w.hidden = hidden;
    w.vocab = vocab;
    w.token_ids.assign(ids, ids + id_count);
    w.token_embeddings.assign(embeddings, embeddings + id_count * hidden);
    w.final_norm_weight.assign(final_norm, final_norm + hidden);
    w.lm_head_weight.assign(lm_head, lm_head + size_t(vocab) * hidden);
    q::write_model_tail_weights(manifest, data_name, w);
    return 0;
  } catch (const std::exception &e) {
    g_error = e.what();
    return -1;
  }
}

} // extern "C"
