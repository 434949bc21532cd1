// Device-side types shared by the decode kernels and the host engine.
#pragma once

#include <cstddef>
#include <cstdint>

namespace qd {

constexpr int kHeadDim = 64;           // the only head size the kernels take
constexpr int kRotary = kHeadDim / 2;  // rotate-half frequencies per head
constexpr int kWave = 64;              // CDNA wavefront
constexpr int kBlock = 256;            // threads per workgroup
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr int kMaxGroup = 16;          // query heads per KV head

// Split-KV attention geometry (qd_attention.hpp): chunks are whole grains
// of positions, at most kAttnMaxChunks per head; a partial record is (m, l,
// acc[64]). The batch-1 decode paths cut chunks in grains of one attention
// tile (kAttnGrain, 16 positions); the batched kernel in passes of 64 (16
// positions per wave of its four-wave unit).
constexpr int kAttnPass = 64;
constexpr int kAttnGrain = 16;
constexpr int kAttnMaxChunks = 16;
constexpr int kPartStride = kHeadDim + 2;

// Chunks of a context of `length` positions split `parts` ways (parts <=
// kAttnMaxChunks; the decode engine uses its resident plan's attention CUs
// per KV group, so that each takes one chunk): whole grains per chunk.
__host__ __device__ inline int attn_chunk_len(int length, int parts = kAttnMaxChunks, int grain = kAttnPass) {
  const int grains = (length + grain - 1) / grain;
  const int per_chunk = (grains + parts - 1) / parts;
  return per_chunk * grain;
}

__host__ __device__ inline int attn_chunks(int length, int parts = kAttnMaxChunks, int grain = kAttnPass) {
  const int cl = attn_chunk_len(length, parts, grain);
  return (length + cl - 1) / cl;
}

enum Mode : uint32_t { kModeStep = 0, kModeGenerate = 1 };

// Storage of the decoder layers' matrices (the values of qd_dtype).
enum WeightStorage : int { kWeightsF32 = 0, kWeightsBf16 = 1, kWeightsF16 = 2 };

// Device-resident state of one sequence slot. The step kernels read
// `position` and `token`; the argmax finaliser writes the sampled token and
// advances the position (the reference's embedding_feedback,
// benchmarks/qwen_stateful_graph_kernel.cpp:358-390).
struct alignas(64) SeqState {
  uint32_t position;   // next free KV slot = tokens already in the cache
  uint32_t token;      // token consumed by the next step
  uint32_t generated;  // tokens produced in generate mode
  uint32_t eos;        // UINT32_MAX: no EOS test
  uint32_t max_tokens;
  uint32_t stop_reason;
  uint32_t stopped;    // nonzero: generate mode ended; step kernels exit
  float top_logit;
  uint32_t mode;
  uint32_t reserved[7];
};
static_assert(sizeof(SeqState) == 64, "SeqState layout");

// Resident weights of one decoder layer. wqkv packs the q, k and v rows
// ([heads*64 + 2*kv_heads*64, hidden], row-major) and bqkv their biases.
struct LayerPtrs {
  const float *wqkv;
  const float *bqkv;
  const float *wo;    // [hidden, heads*64]
  const float *wg;    // [intermediate, hidden]
  const float *wu;    // [intermediate, hidden]
  const float *wd;    // [hidden, intermediate]
  const float *attn_norm;
  const float *mlp_norm;
};

}  // namespace qd
