// Host-side launchers of the decode-step kernels (qd_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qd_device.hpp"

namespace qd {

// Arguments of one decoder layer for one sequence slot.
struct LayerLaunch {
  LayerPtrs w;
  const float *rope_cos;  // [capacity, 32]
  const float *rope_sin;
  SeqState *st;
  float *hidden;   // [hidden]
  float *q;        // [heads*64]
  float *attn;     // [heads*64]
  float *act;      // [intermediate]
  float *k_cache;  // this layer's [capacity, kv_heads*64]
  float *v_cache;
  float *part;     // split-KV partials [16][heads][66]
  int capacity;  // KV positions of the slot; kernels skip positions beyond
  int attn_parts;  // chunk geometry: attn_chunks(length, attn_parts, kAttnGrain)
  int weights_dtype;  // storage of w's decoder matrices (wqkv, wo, wg, wu, wd): kWeights*
  int nq;
  int nkv;
  float eps;
};

struct TailLaunch {
  const float *hidden;
  const float *final_norm;
  const float *head;  // [vocab, hidden]
  SeqState *st;
  float *logits;      // [vocab] or [history][vocab]
  int history;        // nonzero: logits + generated * vocab
  int vocab;
  float eps;
  float *part_val;    // [parts]
  uint32_t *part_idx;
  int parts;          // LM-head workgroups
  uint32_t *out_tokens;
};

// Kernels of the stream-ordered step, for per-kernel event timing.
enum KernelId : int {
  kKEmbed = 0,
  kKQkvRope,
  kKAttnPartial,
  kKAttnCombine,
  kKOproj,
  kKGateUp,
  kKDown,
  kKLmHead,
  kKArgmax,
  kKernelCount
};
const char *kernel_name(int id);

// Optional hook called around every launch (profiling).
struct Marker {
  virtual void before(int kernel) = 0;
  virtual void after(int kernel) = 0;
  virtual ~Marker() = default;
};

bool shape_supported(int hidden, int intermediate, int heads, int kv_heads,
                     int head_dim);
hipError_t launch_embed(hipStream_t s, const float *emb, const SeqState *st,
                        float *hidden, int hidden_size, int vocab,
                        Marker *m = nullptr);
hipError_t launch_layer(hipStream_t s, const LayerLaunch &p, Marker *m = nullptr);
hipError_t launch_tail(hipStream_t s, const TailLaunch &p, Marker *m = nullptr);
// Best-of-`iters` streaming read and copy bandwidth (GB/s, bytes moved per
// second) over a `bytes` buffer on `device` (current), with temporary buffers.
hipError_t probe_hbm(int device, size_t bytes, uint32_t iters, double *read_gbs, double *copy_gbs);
// Sets a slot's state to a step-mode token at `position` (device side).
hipError_t launch_set_state(hipStream_t s, SeqState *st, uint32_t position, uint32_t token);
// Rewrites every NaN of x[0, n) (x 16-byte aligned) as 0x7FC00000.
hipError_t launch_canonical_nan(hipStream_t s, float *x, size_t n);

}  // namespace qd
