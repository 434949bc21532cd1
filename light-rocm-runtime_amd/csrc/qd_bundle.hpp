// Reader and writer of the reference's FP32 weight bundles:
//   layer_<i>/weights.json  "lrrt.mini_decoder_weights" version 2
//   model_tail/weights.json "lrrt.mini_model_tail_weights" version 1
// Same files, same validation and the same diagnostics as
// executor/qwen/weight_bundle.hpp:460-757, so either side can read what the
// other wrote. The manifest is parsed as JSON (not substring-scanned).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace qd::bundle {

// Tensor order of the layer bundle (weight_bundle.hpp:358-386).
enum LayerTensor : int {
  kAttnNorm = 0,
  kMlpNorm,
  kQW,
  kKW,
  kVW,
  kQB,
  kKB,
  kVB,
  kOW,
  kGateW,
  kUpW,
  kDownW,
  kLayerTensorCount
};

extern const char *const kLayerTensorNames[kLayerTensorCount];

struct LayerShape {
  uint32_t keys = 0;
  uint32_t hidden = 0;
  uint32_t heads = 0;
  uint32_t kv_heads = 0;
  uint32_t head_dim = 0;
  uint32_t intermediate = 0;
};

struct LayerWeights {
  LayerShape shape;
  float rope_theta = 10000.0f;
  std::vector<float> tensors[kLayerTensorCount];
};

struct TailWeights {
  uint32_t hidden = 0;
  uint32_t vocab = 0;
  std::vector<uint32_t> token_ids;
  std::vector<float> token_embeddings;
  std::vector<float> final_norm_weight;
  std::vector<float> lm_head_weight;
};

size_t layer_tensor_count(const LayerShape &shape, int tensor);

// Throw std::runtime_error (or std::invalid_argument / std::overflow_error)
// with the reference's messages.
LayerWeights load_layer(const std::string &manifest_path);
TailWeights load_tail(const std::string &manifest_path);
void write_layer(const std::string &manifest_path, const std::string &data_name,
                 const LayerWeights &weights);
void write_tail(const std::string &manifest_path, const std::string &data_name,
                const TailWeights &weights);

}  // namespace qd::bundle
