// Host-side launchers of the batched decode step (qd_batch.hip): up to
// kBatchRows sequences, each at its own KV length, go through a layer
// together; the projections are skinny M <= 16 GEMMs on the FP32 matrix
// cores, so every weight is read from HBM once per batch step.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "qd_device.hpp"
#include "qd_kernels.hpp"

namespace qd {

constexpr int kBatchRows = 16;      // sequences per launch (the MFMA M dimension)
constexpr int kBatchLmParts = 512;  // LM-head workgroups = top-1 partials per sequence

// Buffers and geometry of one batched step. Row b of every activation buffer
// belongs to sequence slot slot[b], which consumes token[b] at KV position
// pos[b] (the host tracks positions, so the kernels take them as arguments);
// the KV cache is indexed by slot (slot s, layer l at
// k_cache + (s * layers + l) * capacity * kv_dim).
struct BatchLaunch {
  int rows;                     // 1 .. kBatchRows
  uint32_t slot[kBatchRows];
  uint32_t pos[kBatchRows];
  uint32_t token[kBatchRows];
  SeqState *states;             // [max_batch]; the argmax kernel writes slot[b]'s
  float *hidden;                // [kBatchRows][896] residual stream
  float *q;                     // [kBatchRows][nq * 64] rotated queries
  float *attn;                  // [kBatchRows][nq * 64]
  float *act;                   // [kBatchRows][4864]
  float *part;                  // [kBatchRows][nq][kAttnMaxChunks][kPartStride]
  float *split;                 // split-K tile partials (kBatchSplitFloats)
  uint32_t *counters;           // arrival counters (kBatchCounters), zero between launches
  float *k_cache;               // whole cache
  float *v_cache;
  const float *rope_cos;        // [capacity, 32]
  const float *rope_sin;
  int layers;
  int capacity;
  int nq;
  int nkv;
  float eps;
};

// Workspace sizes of BatchLaunch::split and ::counters.
constexpr int kBatchSplitFloats = 4 * 128 * (256 + 16);
constexpr int kBatchCounters = 1024;

struct BatchTail {
  const float *final_norm;
  const float *head;     // [vocab, 896]
  float *logits;         // [max_batch][vocab]: batch row b writes the row of its slot, slot[b]
  float *part_val;       // [kBatchRows][kBatchLmParts]
  uint32_t *part_idx;
  uint32_t *out_token;   // [kBatchRows] greedy token of each row
  float *out_top;        // [kBatchRows] its logit
  int vocab;
};

// The scratch of one batched group: every buffer of BatchLaunch and
// BatchTail that is neither an input nor an output of the step. Carved in
// this order from one block, each region 256-byte aligned.
struct BatchWorkspace {
  float *hidden;        // [kBatchRows][896]
  float *q;             // [kBatchRows][nq * 64]
  float *attn;          // [kBatchRows][nq * 64]
  float *act;           // [kBatchRows][4864]
  float *part;          // [kBatchRows][nq][kAttnMaxChunks][kPartStride]
  float *split;         // [kBatchSplitFloats]
  uint32_t *counters;   // [kBatchCounters], zero before a step
  float *part_val;      // [kBatchRows][kBatchLmParts]
  uint32_t *part_idx;   // [kBatchRows][kBatchLmParts]
  uint32_t *out_token;  // [kBatchRows]
  float *out_top;       // [kBatchRows]
};
// Bytes a BatchWorkspace for nq query heads takes; carves one from `base`
// (256-byte aligned, at least that many bytes).
size_t batch_workspace_bytes(int nq);
BatchWorkspace carve_batch_workspace(void *base, int nq);

// The library's static batch workspace (a file-scope device array of
// kBatchScratchBytes, one copy per GPU, held until the process ends): its
// address on `device`, looked up once per device with hipGetSymbolAddress
// while that device is current. nullptr (and *err set) on failure.
constexpr size_t kBatchScratchBytes = size_t(9) << 18;  // 2.25 MiB
void *batch_scratch(int device, hipError_t *err);
// Host lock of a device's static batch workspace: a step that uses the
// workspace holds it from its first launch until its stream is synchronised.
std::mutex &batch_scratch_lock(int device);
// Zeroes a workspace's arrival counters with a fill kernel (a step expects
// them zero; a step that stopped early can leave them set).
hipError_t launch_batch_clear_counters(hipStream_t s, uint32_t *counters);

// Kernels of the batched step, for per-kernel event timing.
enum BatchKernelId : int {
  kBEmbed = 0,
  kBQkvRope,
  kBAttn,
  kBOproj,
  kBGateUp,
  kBDown,
  kBLmHead,
  kBArgmax,
  kBatchKernelCount
};
const char *batch_kernel_name(int id);

hipError_t launch_batch_embed(hipStream_t s, const BatchLaunch &b, const float *embed, int vocab,
                              Marker *m = nullptr);
hipError_t launch_batch_layer(hipStream_t s, const BatchLaunch &b, const LayerPtrs &w, int layer,
                              Marker *m = nullptr);
hipError_t launch_batch_tail(hipStream_t s, const BatchLaunch &b, const BatchTail &t,
                             Marker *m = nullptr);

}  // namespace qd
