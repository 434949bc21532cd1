// Host-side interface of the resident decode megakernel (qd_roles.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qd_device.hpp"

namespace qd {

// Profiled intervals of workgroup 0, each stage split into waiting for its
// input and working: QKV, attention, O-proj (with merge), gate/up, down,
// LM head, argmax -> 14 entries (wait, work), then the attention work's
// sub-phases (K/V staging, math, emit) -> 17 entries.
constexpr int kResidentStages = 17;

// Role-split resident kernel: one 512-thread workgroup per CU. In placement
// order, positions [0, end[kRoleQkv]) compute QKV, [end[kRoleQkv],
// end[kRoleAttn]) attention, then O, gate/up and down; the QKV, attention and
// O ranks come in KV-group blocks of group_cus[] each. Workgroup b takes
// position b, or, with xcd_place, the position that puts group g's QKV,
// attention and O CUs on XCD g (Roles' placement()).
constexpr int kRoleThreads = 512;
constexpr int kMaxRoleGrid = 512;
enum ResidentRole : int { kRoleQkv = 0, kRoleAttn, kRoleO, kRoleGate, kRoleDown, kRoleCount };
struct RolePlan {
  int end[kRoleCount];  // cumulative role ends in placement order (ResidentArgs::role_end)
  int group_cus[3];     // QKV, attention and O CUs per KV group (each role has nkv times as many)
  int xcd_place;        // 1: KV group g's QKV, attention and O CUs all run on XCD g
};
// XCDs of the device. The dispatcher deals a launch's workgroups to the
// XCDs round-robin, but the XCD it starts from is not fixed (after HIP graph
// replays on a stream, workgroup 0 of the next launch has run on another XCD
// than 0), so the resident kernel takes each workgroup's placement position
// from the XCD it runs on.
constexpr int kXcds = 8;

// Bits of the kernel's error word (zero at launch). A CU that raises one
// stops; the CUs waiting on it give up after their own bounded polls, so
// every workgroup exits.
constexpr uint32_t kResidentWaitGaveUp = 1u;    // a hand-off poll exhausted its spin limit
constexpr uint32_t kResidentPlanOverfill = 2u;  // the host plan gave a CU more units than it holds
constexpr uint32_t kResidentPlacement = 4u;     // an XCD received more workgroups than grid / kXcds
// Polls before a hand-off wait gives up (several milliseconds; a healthy
// hand-off takes a few microseconds).
constexpr uint32_t kResidentSpinLimit = 1u << 21;

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
  void *top;                    // (value, tag) argmax partials [2 token parities][2 * grid]
  float *slots;                 // [layers][2][roles_slot_floats] hand-off slots, all bits set
                                //   (kSlotEmpty) at launch
  float *logits;                // [vocab] or [max_tokens][vocab]
  uint32_t *out_tokens;         // [max_tokens]
  SeqState *st;
  uint32_t *error;              // [1 + kXcds], zero at launch: kResident* bits, then each
                                //   XCD's count of workgroups that have taken a position
  uint64_t *stage_ticks;        // nullptr, or [kResidentStages] 100 MHz ticks
  uint64_t *trace;              // nullptr, or [grid][layers + 1][kResidentStages]
                                //   100 MHz timestamps of token trace_token
  uint32_t trace_token;
  int history;
  int capacity;
  int vocab;
  int layers;
  int nq;
  int nkv;
  float eps;
  uint32_t first_token;
  uint32_t start_position;
  uint32_t max_tokens;
  uint32_t eos;
  uint32_t epoch;               // launch epoch << kTagSeqBits, never 0
  uint32_t spin_limit;          // polls before a wait gives up
  int role_end[kRoleCount];     // RolePlan::end
  int group_cus[3];             // RolePlan::group_cus
  int attn_parts;               // chunk geometry: attn_chunks(length, attn_parts, kAttnGrain)
  int xcd_place;                // RolePlan::xcd_place
  int weights_dtype;            // kWeights*: storage of the layers' matrices (picks the instance)
  int attn_mode;                // attention role instance: 0 both chunk forms, 1 every chunk
                                //   of every token longer than one block (tiles only), 2 none
                                //   (one-block form only)
};

// Argmax partial tags: epoch << kTagSeqBits | (token * (5 * layers + 1) + stage + 1).
constexpr int kTagSeqBits = 20;

// Role kernel hand-off slots. Per (layer, token parity) one block of plain
// floats, in order: the QKV output [q | k | v], the attention partial
// records [heads][kAttnMaxChunks][kRoleRecStride] (m, l, 2 pad, acc[64]),
// h1 [hidden], the MLP activation [intermediate] and the layer output
// [hidden]. A slot holds kSlotEmpty until written: a NaN bit pattern (every
// payload bit set) that the kernels' arithmetic never produces, since the
// engine canonicalises every NaN it loads (weights, embeddings, K/V rows)
// to 0x7FC00000.
constexpr int kRoleRecStride = 68;
constexpr uint32_t kSlotEmpty = 0xFFFFFFFFu;
// The layer output is published in segments: down CU r writes its rows
// (at most kHidSegment) padded to whole float4s in floats
// [kHidSegment * r, kHidSegment * (r + 1)), so no float4 has two writers.
constexpr int kHidSegment = 16;
constexpr size_t roles_slot_floats(int hidden, int inter, int heads, int kv_heads) {
  return size_t(heads + 2 * kv_heads) * 64 + size_t(heads) * kAttnMaxChunks * kRoleRecStride +
         size_t(kv_heads) * hidden + size_t(inter) + size_t(kHidSegment) * kMaxRoleGrid;
}

int device_cu_count(int device);

// Role split of `grid` CUs for generations reaching context `max_length`;
// false when the model shape has no role kernel or the grid cannot hold one
// layer's weights on chip.
bool plan_roles(int grid, int hidden, int inter, int heads, int kv_heads, int max_length,
                RolePlan *plan);
hipError_t launch_roles(hipStream_t s, const ResidentArgs &args, int grid);
// Prepares a resident launch in one dispatch: error[0 .. kXcds] zero, the
// parity-0 block ([slot_floats] floats at slots + 2 * l * slot_floats) of
// each of `layers` layers all kSlotEmpty, and, when top is not null, its
// top_pairs (value, tag) pairs zero.
hipError_t launch_roles_prepare(hipStream_t s, uint32_t *error, float *slots, size_t slot_floats,
                               int layers, void *top, int top_pairs);
// Largest co-resident grid of the role kernel for decoder matrices stored as
// `weights_dtype` (kWeights*) on `device` (0 if the query fails).
int roles_max_grid(int device, int weights_dtype);

}  // namespace qd
