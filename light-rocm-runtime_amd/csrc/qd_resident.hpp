// Host-side launcher of the resident decode megakernel (qd_resident.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qd_device.hpp"

namespace qd {

constexpr int kResidentMaxChunks = 80;  // split-KV chunks the merge holds in LDS
// Profiled stages: QKV, attention, O-proj, gate/up, down, LM head, argmax.
constexpr int kResidentStages = 7;

// Arguments of one resident generation on one sequence slot.
struct ResidentArgs {
  const LayerPtrs *layer_ptrs;  // device array [layers]
  const float *embed;           // [vocab, hidden]
  const float *head;            // [vocab, hidden]
  const float *final_norm;      // [hidden]
  const float *rope_cos;        // [capacity, 32]
  const float *rope_sin;
  float *k_cache;               // slot base [layers][capacity][kv_heads*64]
  float *v_cache;
  float *hidden;                // [hidden] residual after each layer
  float *h1;                    // [hidden] residual after the attention block
  float *q;                     // [heads*64]
  float *attn;                  // [heads*64]
  float *act;                   // [intermediate]
  float *part_m;                // [max_chunks, heads]
  float *part_l;
  float *part_acc;              // [max_chunks, heads, 64]
  uint32_t *group_count;        // [kv_heads * 64], zero at launch
  float *logits;                // [vocab] or [max_tokens][vocab]
  float *top_val;               // [grid]
  uint32_t *top_idx;            // [grid]
  uint32_t *flags;              // [grid], zero at launch
  uint32_t *out_tokens;         // [max_tokens]
  SeqState *st;
  uint32_t *error;              // zero at launch; nonzero: a barrier gave up
  uint64_t *stage_ticks;        // nullptr, or [kResidentStages] 100 MHz ticks
  int history;
  int capacity;
  int vocab;
  int layers;
  int nq;
  int nkv;
  int max_chunks;
  float eps;
  uint32_t first_token;
  uint32_t start_position;
  uint32_t max_tokens;
  uint32_t eos;
};

hipError_t launch_resident(hipStream_t s, const ResidentArgs &args, int grid);
// Largest co-resident grid on `device` (0 if the query fails).
int resident_max_grid(int device);
int device_cu_count(int device);

}  // namespace qd
