// Resident decode megakernel, role-split form. One cooperative launch of one
// 512-thread workgroup per CU runs every token of a greedy generation (all
// decoder layers, the LM head, the argmax and the embedding feedback); it is
// the MI355X counterpart of the reference's persistent-graph resident loop
// (include/lrrt/persistent_graph/compiled_scheduler.hpp:108-217 driving
// benchmarks/qwen_stateful_graph_kernel.cpp:661-1083).
//
// Why roles. A decode step is a chain of dependent hand-offs between CUs
// (QKV -> attention -> O -> gate/up -> down -> next layer); on MI355X each
// device-scope hand-off costs ~0.5 us idle and 1-1.6 us while HBM streams,
// and a CU's vector memory pipe returns data in issue order, so a poll issued
// behind a burst of weight loads waits for all of them. The grid is therefore
// split into five roles, each owning one stage of every layer:
//
//   QKV   attention RMSNorm + packed QKV + bias + RoPE -> q, new K/V (+ cache)
//   ATTN  one unit per (KV head, chunk): the group's query heads over the
//         chunk's positions, online softmax -> partial records
//   O     merges the partial records itself, O projection + residual -> h1
//   GATE  MLP RMSNorm + gate/up + SiLU -> act
//   DOWN  down projection + residual -> next layer's hidden
//
// Every role CU keeps one layer's share of its weights on chip (LDS, filled
// by global_load_lds DMA, plus register slots). Right after computing layer l
// it issues the loads of its layer l+1 share, and only then polls for its
// next input: that input arrives about one layer later, by which time the
// loads have landed, so polls never queue behind weight traffic while HBM
// streams the other roles' shares. Sizing gives every role CU about the same
// bytes per layer, so all CUs stream at the same rate.
//
// Hand-offs go through plain FP32 slots, one block per (layer, token
// parity), which hold kSlotEmpty (all bits set) until written: a consumer
// polls 16-byte device-scope (sc1) loads until no word of each float4 it
// needs is empty. The writers of token t clear their slots in the other
// parity's block (token t + 1's). That block held token t - 1's values, and
// every CU finished token t - 1 before any CU started token t, because each
// waits for token t - 1's argmax, which needs every CU's LM-head partial.
// The host fills every slot with kSlotEmpty before a launch. The argmax
// partials are (value, tag) pairs, double-buffered by token parity (the tag
// names the launch epoch and the token).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <type_traits>

#include "qd_attention.hpp"
#include "qd_device.hpp"
#include "qd_device_math.hpp"
#include "qd_resident.hpp"

namespace qd {
namespace {

using namespace dev;

constexpr int kT = kRoleThreads;  // threads per workgroup
constexpr int kW = kT / kWave;    // waves per workgroup
// 160 KiB of LDS per CU, less what the runtime's own block reductions use.
constexpr int kLdsBytes = 160 * 1024 - 512;
constexpr int kAttnCap = 256;     // positions of an attention window staged in LDS

// Register slots per wave: row-pair units of the K=H roles, rows of DOWN.
#ifndef QD_SLOTS_Q
#define QD_SLOTS_Q 3
#endif
#ifndef QD_SLOTS_O
#define QD_SLOTS_O 5
#endif
#ifndef QD_SLOTS_G
#define QD_SLOTS_G 3
#endif
#ifndef QD_DOWN_REG_F4
#define QD_DOWN_REG_F4 18
#endif
constexpr int kSlotsQ = QD_SLOTS_Q, kSlotsO = QD_SLOTS_O, kSlotsG = QD_SLOTS_G;

// Wave index as a wave-uniform (scalar) value: unit indices, slot branches
// and row addresses derived from it stay in SGPRs.
__device__ __forceinline__ int wave_u() { return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); }

// Barriers. HIP's __syncthreads() carries a workgroup-scope fence, which on
// this target waits for every outstanding vector memory operation (weight
// DMA in flight, device-scope stores not yet acknowledged) before the
// barrier, and __syncthreads_and() also re-reads the workgroup size from
// memory. The waves of a role CU only share LDS, so their barrier waits
// for LDS operations alone; a wave that needs its own vector memory
// operations finished (LDS filled by its DMA) says so with vm_wait().
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// vm_wait is the s_waitcnt builtin (vmcnt 0; expcnt and lgkmcnt at their
// no-wait maxima), not inline asm: the compiler's wait insertion sees it, so
// after it no LDS access is guarded against a DMA already waited for.
constexpr unsigned kWaitVmcnt0 = 0x0F70u;
__device__ __forceinline__ void vm_wait() {
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  asm volatile("" ::: "memory");
}
// Prefetch pacing: after each prefetch load a wave waits until at most
// kPaceDepth of its vector memory operations are outstanding (0: no limit).
// A role issues its next-layer weights right after it publishes; unpaced,
// the gate/up CUs alone put ~35 MB of loads in flight at once, queued ahead
// of the hand-off polls of other roles. Depth 8 completes every role's share
// well before its next input arrives (depths 1 to 8 measured within 0.5 %).
#ifndef QD_PACE
#define QD_PACE 8
#endif
constexpr unsigned kPaceDepth = QD_PACE;
static_assert(kPaceDepth < 64, "vmcnt is six bits");
__device__ __forceinline__ void pace() {
  if constexpr (kPaceDepth > 0)
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0 | (kPaceDepth & 15u) | ((kPaceDepth >> 4) << 14));
}
// Whole-workgroup AND (flags: one LDS word per wave). The ballot is taken
// with the whole wave active, then lane 0 records it. Successive calls
// alternate between two flag sets (Roles::flag_set), so one barrier
// suffices: a wave writes the set of call k + 2 only after passing call
// k + 1's barrier, which every wave reaches only after reading call k's.
__device__ __forceinline__ bool block_all(bool v, uint32_t *flags) {
  const uint32_t wave_all = __builtin_amdgcn_ballot_w64(!v) == 0 ? 1u : 0u;
  if (lane_id() == 0) flags[wave_u()] = wave_all;
  lds_barrier();
  uint32_t all = 1u;
#pragma unroll
  for (int w = 0; w < kW; ++w) all &= flags[w];
  return all != 0u;
}

// Where a bounded wait reports that it gave up, and after how many polls.
struct Wait {
  uint32_t *error;
  uint32_t limit;
};

struct Pair2 {
  float v0;
  uint32_t t0;
  float v1;
  uint32_t t1;
};
typedef unsigned int u32x2 __attribute__((vector_size(8)));
typedef __attribute__((address_space(3))) void lds_void;

// (value, tag) vector with device-scope access; bounds-checked by the
// buffer descriptor.
struct TagVec {
  __amdgpu_buffer_rsrc_t r;
  __device__ TagVec(void *base, uint32_t elems)
      : r(__builtin_amdgcn_make_buffer_rsrc(base, 0, static_cast<int>(elems * 8u), kRsrcWord3)) {}
  __device__ void put(uint32_t i, float v, uint32_t tag) const {
    const u32x2 x = {__builtin_bit_cast(unsigned, v), tag};
    __builtin_amdgcn_raw_buffer_store_b64(x, r, i * 8u, 0, kPolicySc1);
  }
  __device__ Pair2 get2(uint32_t pair) const {
    return __builtin_bit_cast(Pair2,
                              __builtin_amdgcn_raw_buffer_load_b128(r, pair * 16u, 0, kPolicySc1));
  }
};

// Float4 i of a small global vector (norm gains, an embedding row) through
// the global address space: a flat load would count against lgkmcnt too,
// and while one is pending the compiler waits for every vector memory
// operation (vmcnt(0)) wherever it waits for any.
__device__ __forceinline__ float4 ld_global4(const float *p, int i) {
  const gf32x4 v = ((global_f32x4 *)p)[i];
  return make_float4(v.x, v.y, v.z, v.w);
}

struct Lds {
  const float *p;
  __device__ float ld(uint32_t i) const { return p[i]; }
  __device__ float4 ld4(uint32_t i4) const { return reinterpret_cast<const float4 *>(p)[i4]; }
};

// 1 KiB global -> LDS copy without registers: lane l's 16 bytes from `src`
// land at dst + 16 l (dst wave-uniform). Counted by vmcnt like any load.
template <int kPolicy>
__device__ __forceinline__ void dma16(const void *src, void *dst) {
#if __HIP_DEVICE_COMPILE__
  __builtin_amdgcn_global_load_lds(src, (lds_void *)dst, 16, 0, kPolicy);
#endif
}

// Profiling state in LDS (see Clock): stage totals and the traced token's
// stamps (per layer: input arrived, outputs published; then LM head/argmax).
constexpr int kMaxTraceLayers = 24;
constexpr int kStampsPerLayer = 5;  // input arrived, outputs published, 3 sub-phases
struct ClockLds {
  uint64_t ticks[kResidentStages];
  uint64_t stamps[kStampsPerLayer * kMaxTraceLayers + 4];
};

struct Common {
  float vec[1024];   // gathered input vector (hidden, h1, residual rows)
  float xn[1024];    // normalised GEMV operand / merged attention
  uint32_t flags[2][kW];                // block_all, two alternating sets
  float bv[kW];
  uint32_t bi[kW];
  float top[2 * kMaxRoleGrid];          // argmax partials (value, index bits); in the
                                        //   layers, a role's outputs staged for their stores
  ClockLds clock;                       // profiling (profiled variant only)
};
static_assert(offsetof(Common, xn) == offsetof(Common, vec) + sizeof(Common::vec),
              "h1 partials stage in vec and then xn");
// The kernel's one LDS block, at namespace scope so the per-role functions
// (called from the kernel) address it as LDS.
__shared__ __attribute__((aligned(16))) unsigned char roles_lds[kLdsBytes];

constexpr int kRegionOffset = (static_cast<int>(sizeof(Common)) + 255) / 256 * 256;
constexpr int kRegionBytes = kLdsBytes - kRegionOffset;

// Whole-workgroup gather of `pairs` tagged pairs: map(p, src_pair, dst)
// names pair p's source pair index and its destination float index (two
// consecutive floats). Returns false when the wait gave up (error raised).
// Each wave polls its own items until they are all complete, with no
// workgroup barrier between its polls; one barrier at the end makes the
// whole destination visible to every wave. (The same holds for gather4 and
// gather4_put.)
template <int kMaxPer, typename Map>
__device__ bool gather_map(const TagVec &src, int pairs, uint32_t tag, float *dst, Wait wait,
                           uint32_t *flags, Map map) {
  const int t = threadIdx.x;
  uint32_t pending = 0;
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k)
    if (t + k * kT < pairs) pending |= 1u << k;
  bool ok = true;
  for (uint32_t spin = 0;; ++spin) {
    Pair2 got[kMaxPer];
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k)
      if ((pending >> k) & 1u) {
        uint32_t s;
        int d;
        map(t + k * kT, s, d);
        got[k] = src.get2(s);
      }
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      if (((pending >> k) & 1u) && got[k].t0 == tag && got[k].t1 == tag) {
        uint32_t s;
        int d;
        map(t + k * kT, s, d);
        dst[d] = got[k].v0;
        dst[d + 1] = got[k].v1;
        pending &= ~(1u << k);
      }
    }
    // Every wave's earlier vector memory operations (its LDS DMA above all)
    // are complete when the gather returns.
    vm_wait();
    if (__builtin_amdgcn_ballot_w64(pending != 0) == 0) break;
    if (spin > wait.limit) {
      if (lane_id() == 0) atomicOr(wait.error, kResidentWaitGaveUp);
      ok = false;
      break;
    }
  }
  return block_all(ok, flags);
}

// Contiguous gather: elements [first, first + n) (first and n even) -> dst.
template <int kMaxPer>
__device__ bool gather(const TagVec &src, uint32_t first, int n, uint32_t tag, float *dst,
                       Wait wait, uint32_t *flags) {
  return gather_map<kMaxPer>(src, n / 2, tag, dst, wait, flags, [&](int p, uint32_t &s, int &d) {
    s = first / 2 + p;
    d = 2 * p;
  });
}

// One (layer, token parity) block of hand-off slots: plain floats with
// device-scope access, kSlotEmpty until written; bounds-checked by the
// buffer descriptor.
// Hand-off slots. Loads are sc1 (served by the reader's L2 within its XCD,
// coherently across XCDs); stores are sc1 (written through to memory) unless
// the slots are XCD-local: every writer and reader of them runs on one XCD,
// whose L2 is then the point of coherence and plain stores suffice.
struct Slots {
  __amdgpu_buffer_rsrc_t r;
  bool local;
  __device__ Slots(float *base, uint32_t floats, bool xcd_local = false)
      : r(__builtin_amdgcn_make_buffer_rsrc(base, 0, static_cast<int>(floats * 4u), kRsrcWord3)),
        local(xcd_local) {}
  __device__ void st32(uint32_t i, uint32_t v) const {
    if (local)
      __builtin_amdgcn_raw_buffer_store_b32(v, r, i * 4u, 0, 0);
    else
      __builtin_amdgcn_raw_buffer_store_b32(v, r, i * 4u, 0, kPolicySc1);
  }
  __device__ void st128(uint32_t i4, u32x4 v) const {
    if (local)
      __builtin_amdgcn_raw_buffer_store_b128(v, r, i4 * 16u, 0, 0);
    else
      __builtin_amdgcn_raw_buffer_store_b128(v, r, i4 * 16u, 0, kPolicySc1);
  }
  __device__ void put(uint32_t i, float v) const { st32(i, __builtin_bit_cast(unsigned, v)); }
  __device__ void clear(uint32_t i) const { st32(i, kSlotEmpty); }
  __device__ void put4(uint32_t i4, float4 v) const {
    const f32x4 x = {v.x, v.y, v.z, v.w};
    st128(i4, __builtin_bit_cast(u32x4, x));
  }
  __device__ void clear4(uint32_t i4) const {
    const u32x4 x = {kSlotEmpty, kSlotEmpty, kSlotEmpty, kSlotEmpty};
    st128(i4, x);
  }
  __device__ void st(uint32_t i, float v) const { put(i, v); }
  __device__ void st4(uint32_t i4, float4 v) const { put4(i4, v); }
  __device__ u32x4 get4(uint32_t i4) const {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, i4 * 16u, 0, kPolicySc1));
  }
};
struct Quad {
  uint32_t w[4];
};

// Whole-workgroup wait for n4 float4s of hand-off slots: map(p, s4, d4)
// names float4 p's slot index and its destination index in dst. A float4
// is complete when none of its words is kSlotEmpty. Returns false when the
// wait gave up (error raised).
template <int kMaxPer, typename Map>
__device__ bool gather4(const Slots &src, int n4, float4 *dst, Wait wait, uint32_t *flags,
                        Map map) {
  const int t = threadIdx.x;
  uint32_t pending = 0;
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k)
    if (t + k * kT < n4) pending |= 1u << k;
  bool ok = true;
  for (uint32_t spin = 0;; ++spin) {
    Quad got[kMaxPer];
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k)
      if ((pending >> k) & 1u) {
        int s, d;
        map(t + k * kT, s, d);
        got[k] = __builtin_bit_cast(Quad, src.get4(s));
      }
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      const Quad &g = got[k];
      if (((pending >> k) & 1u) && g.w[0] != kSlotEmpty && g.w[1] != kSlotEmpty &&
          g.w[2] != kSlotEmpty && g.w[3] != kSlotEmpty) {
        int s, d;
        map(t + k * kT, s, d);
        dst[d] = make_float4(__uint_as_float(g.w[0]), __uint_as_float(g.w[1]), __uint_as_float(g.w[2]),
                             __uint_as_float(g.w[3]));
        pending &= ~(1u << k);
      }
    }
    // Every wave's earlier vector memory operations (its LDS DMA and its
    // slot clears above all) are complete when the gather returns.
    vm_wait();
    if (__builtin_amdgcn_ballot_w64(pending != 0) == 0) break;
    if (spin > wait.limit) {
      if (lane_id() == 0) atomicOr(wait.error, kResidentWaitGaveUp);
      ok = false;
      break;
    }
  }
  return block_all(ok, flags);
}

// Contiguous float4s [first4, first4 + n4) of a slot block -> dst[0, n4).
template <int kMaxPer>
__device__ bool gather4c(const Slots &src, int first4, int n4, float *dst, Wait wait,
                         uint32_t *flags) {
  return gather4<kMaxPer>(src, n4, reinterpret_cast<float4 *>(dst), wait, flags,
                          [&](int p, int &s, int &d) {
                            s = first4 + p;
                            d = p;
                          });
}

// Whole-workgroup wait for `items` float4s of hand-off slots, item p =
// threadIdx.x + k * kT held in the thread's k-th place: live(p, k, s4) names
// its slot index and returns false for an item with nothing to wait for;
// put(k, v) consumes a complete float4. Returns false when the wait gave up
// (error raised).
template <int kMaxPer, typename Live, typename Put>
__device__ bool gather4_put(const Slots &src, int items, Wait wait, uint32_t *flags, Live live, Put put) {
  const int t = threadIdx.x;
  uint32_t pending = 0;
  int slot[kMaxPer];
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k) {
    slot[k] = 0;
    if (t + k * kT < items && live(t + k * kT, k, slot[k])) pending |= 1u << k;
  }
  bool ok = true;
  for (uint32_t spin = 0;; ++spin) {
    Quad got[kMaxPer];
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k)
      if ((pending >> k) & 1u) got[k] = __builtin_bit_cast(Quad, src.get4(slot[k]));
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      const Quad &g = got[k];
      if (((pending >> k) & 1u) && g.w[0] != kSlotEmpty && g.w[1] != kSlotEmpty &&
          g.w[2] != kSlotEmpty && g.w[3] != kSlotEmpty) {
        put(k, make_float4(__uint_as_float(g.w[0]), __uint_as_float(g.w[1]), __uint_as_float(g.w[2]),
                           __uint_as_float(g.w[3])));
        pending &= ~(1u << k);
      }
    }
    vm_wait();
    if (__builtin_amdgcn_ballot_w64(pending != 0) == 0) break;
    if (spin > wait.limit) {
      if (lane_id() == 0) atomicOr(wait.error, kResidentWaitGaveUp);
      ok = false;
      break;
    }
  }
  return block_all(ok, flags);
}

// Publishing a role's outputs. A role CU's outputs are fixed runs of slot
// elements; each thread owns at most one float4 of them (OutMap, computed
// once per launch): its float4 index q in the destination, which of its
// four elements belong to this CU (the float4s at the ends of a run are
// shared with neighbouring workgroups) and where the values sit in the LDS
// stage. A whole float4 goes out with one 16-byte store, a shared one
// element by element. Memory then sees whole-line writes rather than
// scattered words (scattered 4-byte writes from the lanes slowed a hand-off
// by 0.5-1.3 us). The thread reads its float4 from LDS before it stores:
// the compiler makes an LDS read wait for every earlier store (vmcnt
// counts stores and guards the DMA).
struct OutMap {
  int q = -1;         // float4 index in the destination, -1: none
  int soff = 0;       // float4 index in the stage
  uint32_t mask = 0;  // elements of float4 q this CU owns
  int tag = 0;        // caller's label for the run
  // Float4 `item` of the run [first, first + n) (stage[j] holding element
  // sbase + j, sbase a multiple of 4); returns the run's float4 count.
  __device__ int take(int first, int n, int sbase, int item, int run_tag) {
    const int q0 = first >> 2, cnt = ((first + n + 3) >> 2) - q0;
    if (item >= 0 && item < cnt) {
      q = q0 + item;
      soff = (4 * q - sbase) >> 2;
      mask = 0;
      for (int k = 0; k < 4; ++k)
        if (4 * q + k >= first && 4 * q + k < first + n) mask |= 1u << k;
      tag = run_tag;
    }
    return cnt;
  }
};
// Stores v (this thread's float4 of a run) to dst at float4 q + off4.
template <typename Dst>
__device__ __forceinline__ void put_quad(const Dst &dst, const OutMap &m, float4 v, int off4 = 0) {
  if (m.mask == 0xFu) {
    dst.st4(static_cast<uint32_t>(m.q + off4), v);
  } else {
    const float x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if ((m.mask >> k) & 1u) dst.st(static_cast<uint32_t>(4 * (m.q + off4) + k), x[k]);
  }
}
// Sets this thread's elements of a run of slots to kSlotEmpty.
__device__ __forceinline__ void clear_quad(const Slots &dst, const OutMap &m) {
  if (m.mask == 0xFu) {
    dst.clear4(static_cast<uint32_t>(m.q));
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if ((m.mask >> k) & 1u) dst.clear(static_cast<uint32_t>(4 * m.q + k));
  }
}

// Profiling clock kept by thread 0 (profiled variant only). Totals and the
// traced token's stamps live in LDS and reach global memory only when the
// traced token ends and at exit: a global store here would make the role's
// next LDS read wait for it (the compiler guards LDS reads behind the DMA
// with vmcnt, which also counts stores), distorting what is measured.

template <bool kProfile>
struct Clock {
  ClockLds *lds = nullptr;
  uint64_t prev = 0;
  bool tracing = false;
  int layer = 0;
  __device__ void start(ClockLds *c) {
    if (kProfile && threadIdx.x == 0) {
      lds = c;
      for (int s = 0; s < kResidentStages; ++s) lds->ticks[s] = 0;
      prev = wall_clock64();
    }
  }
  __device__ void at(bool trace_this_token, int l) {
    if (kProfile) {
      tracing = trace_this_token;
      layer = l;
    }
  }
  // Role stages 2r (input arrived) and 2r+1 (outputs published) per layer;
  // stages from 2*kRoleCount on belong to the token's LM head and argmax.
  __device__ void lap(int stage) {
    if (kProfile && threadIdx.x == 0) {
      const uint64_t now = wall_clock64();
      lds->ticks[stage] += now - prev;
      prev = now;
      if (tracing) {
        if (stage < 2 * kRoleCount) {
          if (layer < kMaxTraceLayers) lds->stamps[kStampsPerLayer * layer + (stage & 1)] = now;
        } else {
          lds->stamps[kStampsPerLayer * kMaxTraceLayers + (stage - 2 * kRoleCount)] = now;
        }
      }
    }
  }
  // Sub-phase stamp k (0..2) of the traced token's current layer (trace only).
  __device__ void mark(int k) {
    if (kProfile && threadIdx.x == 0 && tracing && layer < kMaxTraceLayers)
      lds->stamps[kStampsPerLayer * layer + 2 + k] = wall_clock64();
  }
  // Timeline of the traced token: row[l][stage] for this CU's role stages,
  // its sub-phases in the last three stage slots, and the LM head / argmax
  // stages.
  __device__ void flush_trace(uint64_t *trace, int wg, int layers, int role) const {
    if (!kProfile || !trace || threadIdx.x != 0) return;
    uint64_t *row = trace + static_cast<size_t>(wg) * (layers + 1) * kResidentStages;
    for (int l = 0; l < layers && l < kMaxTraceLayers; ++l) {
      const uint64_t *st = lds->stamps + kStampsPerLayer * l;
      row[l * kResidentStages + 2 * role] = st[0];
      row[l * kResidentStages + 2 * role + 1] = st[1];
      for (int k = 0; k < 3; ++k) row[l * kResidentStages + kResidentStages - 3 + k] = st[2 + k];
    }
    for (int j = 0; j < 4; ++j)
      row[layers * kResidentStages + 2 * kRoleCount + j] =
          lds->stamps[kStampsPerLayer * kMaxTraceLayers + j];
  }
  // Stage totals: the first CU of each role reports its role's stages, CU 0
  // the LM head and argmax stages.
  __device__ void publish(uint64_t *out, int role, bool first_of_role) const {
    if (!kProfile || !out || threadIdx.x != 0) return;
    if (first_of_role) {
      out[2 * role] = lds->ticks[2 * role];
      out[2 * role + 1] = lds->ticks[2 * role + 1];
    }
    if (blockIdx.x == 0)
      for (int s = 2 * kRoleCount; s < kResidentStages; ++s) out[s] = lds->ticks[s];
  }
};

// ---- K=H row-pair roles (QKV, O, gate/up) ----------------------------------
// A CU owns units [u0, u0 + n); local unit k belongs to wave k % kW. Units
// k < kW*S sit in register slot k / kW of their wave; the next Lcap units in
// LDS (unit k - kW*S, in slot-layout order); any further unit is loaded from
// global memory when computed (only if the plan over-fills a CU).
//
// Registers and LDS always hold FP32, so the arithmetic of a layer is the
// same code whatever the stored type W. FP32 weights are loaded as they
// are (LDS by DMA). BF16 / FP16 weights are widened while prefetching: the
// register units' slots arrive raw and are widened by settle(), which a
// role calls before it waits for its input; the LDS units pass through a
// wave's registers (load, widen, LDS store), so their HBM bytes are halved
// and nothing is widened inside a layer's dot products.
template <int H, int S, int LdsUnits, typename W>
struct PairRole {
  // Units held in LDS: what the region holds, at most what the eight unit
  // sums of a wave (compute) can carry.
  static constexpr int Lcap = LdsUnits < (8 - S) * kW ? LdsUnits : (8 - S) * kW;
  using WT = WReg<W>;
  using R = typename WT::type;
  using Slot = typename WSlot<W>::type;
  static constexpr bool kNarrow = sizeof(R) == 8;
  static constexpr int NJ = PairSlots<H>::NJ;
  static constexpr int K4 = PairSlots<H>::K4;
  static constexpr int UnitBytes = NJ * 1024;  // FP32 slots, slot-layout order
  float4 wv[S][NJ];
  R raw[kNarrow ? S : 1][NJ];  // narrow register units as loaded, until settle()
  unsigned char *units = nullptr;
  int n = 0;

  // Slot c of a row pair's run of 2 K4 slots (zero past it).
  __device__ static R load_slot(const Slot *a4, const Slot *b4, int c, int lane) {
    const int f = c * kWave + lane;
    if (c * kWave + kWave <= K4) return ld_slot(a4 + f);
    if (c * kWave >= K4) return f < 2 * K4 ? ld_slot(b4 + (f - K4)) : WT::zero();
    return ld_slot(f < K4 ? a4 + f : b4 + (f - K4));
  }

  template <typename Rows>
  __device__ void prefetch_regs(Rows rows) {
    const int w = wave_u(), lane = lane_id();
#pragma unroll
    for (int j = 0; j < S; ++j) {
      const int k = w + kW * j;
      if (k < n) {
        const W *ra, *rb;
        rows(k, ra, rb);
        const Slot *a4 = reinterpret_cast<const Slot *>(ra);
        const Slot *b4 = reinterpret_cast<const Slot *>(rb);
#pragma unroll
        for (int c = 0; c < NJ; ++c) {
          if constexpr (kNarrow)
            raw[j][c] = load_slot(a4, b4, c, lane);
          else
            wv[j][c] = load_slot(a4, b4, c, lane);
        }
        pace();
      } else {
        // An empty slot is still redefined, so its previous contents are
        // not kept live across the code between two prefetches.
#pragma unroll
        for (int c = 0; c < NJ; ++c) {
          if constexpr (kNarrow)
            raw[j][c] = WT::zero();
          else
            wv[j][c] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
  }
  // Narrow register units: widen the prefetched slots (waits for them).
  __device__ void settle() {
    if constexpr (kNarrow) {
#pragma unroll
      for (int j = 0; j < S; ++j)
#pragma unroll
        for (int c = 0; c < NJ; ++c) wv[j][c] = pin(WT::widen(raw[j][c]));
    }
  }
  template <typename Rows>
  __device__ void prefetch_lds(Rows rows) {
    const int lane = lane_id();
    if constexpr (!kNarrow) {
      for (int k = kW * S + wave_u(); k < n && k - kW * S < Lcap; k += kW) {
        const W *ra, *rb;
        rows(k, ra, rb);
        const Slot *a4 = reinterpret_cast<const Slot *>(ra);
        const Slot *b4 = reinterpret_cast<const Slot *>(rb);
        unsigned char *dst = units + (k - kW * S) * UnitBytes;
#pragma unroll
        for (int c = 0; c < NJ; ++c) {
          const int f = c * kWave + lane;
          const Slot *src = f < K4 ? a4 + f : (f < 2 * K4 ? b4 + (f - K4) : a4);
          dma16<kPolicyNt>(src, dst + c * 1024);
          pace();
        }
      }
    } else {
      // Two units in flight: unit k's slots are widened and stored while
      // unit k + kW's loads are outstanding.
      R cur[NJ], nxt[NJ];
      int k = kW * S + wave_u();
      auto fetch = [&](int kk, R (&buf)[NJ]) {
        const W *ra, *rb;
        rows(kk, ra, rb);
        const Slot *a4 = reinterpret_cast<const Slot *>(ra);
        const Slot *b4 = reinterpret_cast<const Slot *>(rb);
#pragma unroll
        for (int c = 0; c < NJ; ++c) buf[c] = load_slot(a4, b4, c, lane);
      };
      auto live = [&](int kk) { return kk < n && kk - kW * S < Lcap; };
      if (live(k)) fetch(k, cur);
      for (; live(k); k += kW) {
        if (live(k + kW)) fetch(k + kW, nxt);
        float4 *dst = reinterpret_cast<float4 *>(units + (k - kW * S) * UnitBytes);
#pragma unroll
        for (int c = 0; c < NJ; ++c) dst[c * kWave + lane] = WT::widen(cur[c]);
#pragma unroll
        for (int c = 0; c < NJ; ++c) cur[c] = nxt[c];
      }
    }
  }
  // Every unit's two sums are computed before any epilogue runs: the
  // epilogues publish with device-scope stores, and on this target vmcnt
  // counts stores too, so an LDS read issued after a store (the compiler
  // guards LDS reads behind the pending DMA with vmcnt(0)) would wait for
  // the store's round trip.
  // prep(k) returns the per-unit constants the epilogue needs from LDS; it
  // is read before the unit's epilogue stores for the same reason.
  static constexpr int kLdsPerWave = (Lcap + kW - 1) / kW;
  template <typename Prep, typename Epi, typename Mid>
  __device__ void compute(const float4 (&xv)[NJ], Prep prep, Epi epi, Mid mid) const {
    const int w = wave_u(), lane = lane_id();
    constexpr int kUnits = S + kLdsPerWave;
    static_assert(kUnits <= 8, "unit sums travel as values 0..7 and 8..15");
    // Per-lane partials of every unit: unit j's first row as value j, its
    // second row as value 8 + j (zeros where the wave has no unit).
    float part[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) part[i] = 0.f;
#pragma unroll
    for (int j = 0; j < S; ++j) pair_partial<H>(wv[j], xv, part[j], part[8 + j]);
#pragma unroll
    for (int i = 0; i < kLdsPerWave; ++i) {
      const int k = kW * S + w + kW * i;
      if (k < n && k - kW * S < Lcap) {
        const float4 *src = reinterpret_cast<const float4 *>(units + (k - kW * S) * UnitBytes);
        float4 wl[NJ];
#pragma unroll
        for (int c = 0; c < NJ; ++c) wl[c] = src[c * kWave + lane];
        pair_partial<H>(wl, xv, part[S + i], part[8 + S + i]);
      }
    }
    // All the wave's sums at once, each bit-identical to wave_sum (lane l
    // holds value l mod 16): unit j's sums finish in lane j, where all the
    // wave's epilogues then run at once.
    const float tot = wave_sum_multi<16>(part);
    mid();
    const float ma = tot;
    const float mb = __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, tot), 0x108 /* row_shl:8 */, 0xf, 0xf,
                                           false));
    const int k = lane < S ? w + kW * lane : kW * S + w + kW * (lane - S);
    if (lane < kUnits && k < n && (lane < S || k - kW * S < Lcap)) epi(k, ma, mb, prep(k));
  }
  // Units this CU can hold (the host plan never assigns more).
  static constexpr int capacity() { return kW * S + Lcap; }
};

// ---- K=I rows, column slices (down) -----------------------------------------
// A CU owns rows [u0, u0 + n). Wave w owns column slice w of every row
// (slots [c0, c0 + ns) of the row's NJ float4 slots, dot_row_sliced's
// slices): rows [0, kRegF4 / ns) of its slice sit in register slots, the
// rest in the wave's own LDS area. Each wave waits for its own slice of the
// activation (straight into registers) and leaves every row's per-lane
// slice sums in LDS; wave w then finishes rows w, w + 8, ... (per lane
// combine_slices over the waves' sums, then wave_sum: dot_row_sliced's
// order). Registers are indexed with the slice width as a template constant.
template <int I, typename W>
struct DownRole {
  using WT = WReg<W>;
  using R = typename WT::type;
  using Slot = typename WSlot<W>::type;
  static constexpr bool kNarrow = sizeof(R) == 8;
  static constexpr int NJ = RowSlots<I>::NJ;
  static constexpr int kNsLo = NJ / kRowSlices, kNsHi = (NJ + kRowSlices - 1) / kRowSlices;
  // Weight float4s per lane held in registers (a wider budget for the
  // wide slices made the compiler keep the array in scratch).
  __host__ __device__ static constexpr int reg_f4(int) { return kRegF4; }
  static constexpr int kRegF4 = QD_DOWN_REG_F4;
  static constexpr int kMaxRows = 16;
  static_assert(kRowSlices == kW && kNsLo >= 1, "one slice per wave");
  // LDS 1 KiB slot-rows of the CU's n rows (what the registers do not hold).
  __host__ __device__ static constexpr int lds_rows(int n) {
    int total = 0;
    for (int w = 0; w < kRowSlices; ++w) {
      const int ns = row_slice_begin(NJ, w + 1) - row_slice_begin(NJ, w);
      total += (n > reg_f4(ns) / ns ? n - reg_f4(ns) / ns : 0) * ns;
    }
    return total;
  }
  __host__ __device__ static constexpr int capacity() {
    int n = kMaxRows;
    // LDS rows, then the per-lane slice sums of every row.
    while (n > 0 && lds_rows(n) * kWave * 16 + n * kRowSlices * kWave * 4 > kRegionBytes) --n;
    return n;
  }
  // Registers and LDS hold FP32 whatever W is (PairRole's scheme): narrow
  // register rows arrive in raw and are widened by settle(); narrow LDS
  // rows pass through the wave's registers and are widened on the way.
  float4 wr[kRegF4];
  R raw[kNarrow ? kRegF4 : 1];
  float4 *lw = nullptr;   // this wave's LDS rows: ((r - nr) * ns + s) * 64 + lane
  int n = 0, c0 = 0, ns = 0, nr = 0;

  __device__ void init(int rows, float4 *region_f4) {
    n = rows;
    const int w = wave_u();
    c0 = row_slice_begin(NJ, w);
    ns = row_slice_begin(NJ, w + 1) - c0;
    nr = reg_f4(ns) / ns;
    int off = 0;
    for (int v = 0; v < w; ++v) {
      const int nsv = row_slice_begin(NJ, v + 1) - row_slice_begin(NJ, v);
      off += (n > reg_f4(nsv) / nsv ? n - reg_f4(nsv) / nsv : 0) * nsv;
    }
    lw = region_f4 + off * kWave;
  }
  template <int Ns, typename Row>
  __device__ void prefetch_regs_ns(Row row) {
    constexpr int Nr = reg_f4(Ns) / Ns;
    const int lane = lane_id();
#pragma unroll
    for (int r = 0; r < Nr; ++r) {
#pragma unroll
      for (int s = 0; s < Ns; ++s) {
        const Slot *src = reinterpret_cast<const Slot *>(row(r)) + (c0 + s) * kWave + lane;
        if constexpr (kNarrow)
          raw[r * Ns + s] = r < n ? ld_slot(src) : WT::zero();
        else
          wr[r * Ns + s] = r < n ? ld_slot(src) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      pace();
    }
  }
  template <typename Row>
  __device__ void prefetch_regs(Row row) {
    if (ns == kNsHi) prefetch_regs_ns<kNsHi>(row); else prefetch_regs_ns<kNsLo>(row);
  }
  // Narrow register rows: widen the prefetched slots (waits for them).
  __device__ void settle() {
    if constexpr (kNarrow) {
#pragma unroll
      for (int i = 0; i < kRegF4; ++i) wr[i] = pin(WT::widen(raw[i]));
    }
  }
  template <typename Row>
  __device__ void prefetch_lds(Row row) {
    const int lane = lane_id();
    if constexpr (!kNarrow) {
      for (int r = nr; r < n; ++r)
        for (int s = 0; s < ns; ++s) {
          dma16<kPolicyNt>(reinterpret_cast<const Slot *>(row(r)) + (c0 + s) * kWave + lane,
                           lw + ((r - nr) * ns + s) * kWave);
          pace();
        }
    } else {
      // A row's slots (at most kNsHi) in flight while the previous row's
      // are widened and stored.
      R cur[kNsHi], nxt[kNsHi];
      auto fetch = [&](int r, R (&buf)[kNsHi]) {
        const Slot *src = reinterpret_cast<const Slot *>(row(r)) + c0 * kWave + lane;
#pragma unroll
        for (int s = 0; s < kNsHi; ++s)
          if (s < ns) buf[s] = ld_slot(src + s * kWave);
      };
      if (nr < n) fetch(nr, cur);
      for (int r = nr; r < n; ++r) {
        if (r + 1 < n) fetch(r + 1, nxt);
#pragma unroll
        for (int s = 0; s < kNsHi; ++s)
          if (s < ns) lw[((r - nr) * ns + s) * kWave + lane] = WT::widen(cur[s]);
#pragma unroll
        for (int s = 0; s < kNsHi; ++s) cur[s] = nxt[s];
      }
    }
  }
  // Per-lane slice sums of every row with this wave's activation slice xa:
  // row r's lands in part[(r * kW + wave) * 64 + lane]. The register rows
  // are computed unconditionally (rows past n hold zeros); the LDS rows go
  // in batches of kBatch whose reads are all issued before their products,
  // so a batch waits for LDS once (indices past the last row are clamped to
  // it and their sums discarded).
  static constexpr int kBatch = 4;
  template <int Ns>
  __device__ void sums_ns(const float4 (&xa)[kNsHi], float *part) const {
    constexpr int Nr = reg_f4(Ns) / Ns;
    const int lane = lane_id(), w = wave_u();
    float acc[Nr];
#pragma unroll
    for (int r = 0; r < Nr; ++r) {
      acc[r] = 0.f;
#pragma unroll
      for (int s = 0; s < Ns; ++s) acc[r] = fma4(wr[r * Ns + s], xa[s], acc[r]);
    }
#pragma unroll
    for (int r = 0; r < Nr; ++r)
      if (r < n) part[(r * kW + w) * kWave + lane] = acc[r];
#pragma unroll
    for (int b = Nr; b < kMaxRows; b += kBatch) {
      if (b >= n) break;
      float4 lr[kBatch][Ns];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        const int r = min(b + i, n - 1);
#pragma unroll
        for (int s = 0; s < Ns; ++s) lr[i][s] = lw[((r - Nr) * Ns + s) * kWave + lane];
      }
      float bacc[kBatch];
#pragma unroll
      for (int i = 0; i < kBatch; ++i) {
        bacc[i] = 0.f;
#pragma unroll
        for (int s = 0; s < Ns; ++s) bacc[i] = fma4(lr[i][s], xa[s], bacc[i]);
      }
#pragma unroll
      for (int i = 0; i < kBatch; ++i)
        if (b + i < n) part[((b + i) * kW + w) * kWave + lane] = bacc[i];
    }
  }
  __device__ void sums(const float4 (&xa)[kNsHi], float *part) const {
    if (ns == kNsHi) sums_ns<kNsHi>(xa, part); else sums_ns<kNsLo>(xa, part);
  }
};

// Balanced split of `total` items over `parts`: part r gets [begin, end).
__device__ __forceinline__ int split_begin(int total, int parts, int r) {
  return static_cast<int>((static_cast<int64_t>(total) * r) / parts);
}

template <int H, int I, int NQ, int NKV, typename W = float>
struct Shape {
  static constexpr int QD = NQ * kHeadDim;
  static constexpr int KVD = NKV * kHeadDim;
  static constexpr int G = NQ / NKV;
  static constexpr int QkvRows = QD + 2 * KVD;
  static constexpr int QkvUnits = QkvRows / 2;
  static constexpr int OUnits = H / 2;
  static constexpr int UnitBytes = PairSlots<H>::NJ * 1024;
  static constexpr int RowBytes = RowSlots<I>::NJ * kWave * 16;
  // QKV region: units, biases (whole float4 DMA rows), cos|sin row.
  static constexpr int BiasF4 = (QkvRows / 4 + kWave - 1) / kWave * kWave;
  static constexpr int LQ = (kRegionBytes - BiasF4 * 16 - kWave * 16) / UnitBytes;
  // Partial records of every head (the slot block's attention outputs).
  static constexpr int PartFloats = NQ * kAttnMaxChunks * kRoleRecStride;
  // O is split by KV group: an O CU of group g takes the g-th QDG columns
  // (its G query heads) of every row, so its units are row pairs of QDG
  // columns, and its region holds units and its group's records.
  static constexpr int QDG = G * kHeadDim;
  static constexpr int OUnitBytes = PairSlots<QDG>::NJ * 1024;
  static constexpr int PartFloatsG = G * kAttnMaxChunks * kRoleRecStride;
  static constexpr int LO = (kRegionBytes - PartFloatsG * 4) / OUnitBytes;
  static constexpr int LG = kRegionBytes / UnitBytes;
  static_assert(QkvRows % 2 == 0 && H % 2 == 0, "row pairs");
  static_assert(G <= kW && NQ % NKV == 0, "one wave per query head of a group");
  static_assert(LQ > 0 && LO > 0 && LG > 0, "LDS plan");
  static_assert(H <= 1024 && QD <= 1024, "common vectors");
};

// The attention CU's LDS: the group's queries and this step's K/V row, one
// window of K (float4 columns) and V rows, and each wave's probability
// tile. After a chunk's
// tiles the K window holds the wave partials (AttnStage).
struct AttnRegion {
  float qs[kW * kHeadDim];
  float kn[kHeadDim];
  float vn[kHeadDim];
  float4 kt[(kHeadDim / 4) * kAttnCap];
  float vr[kAttnCap * kHeadDim];
  float ps[kW * kAttnPsFloats];
};
static_assert(sizeof(AttnRegion) <= kRegionBytes, "attention region");
static_assert(kAttnSlots == kW && kAttnCap % (kAttnSlots * kAttnTile) == 0, "a window holds whole rounds of tiles");
static_assert(kAttnStageFloats * 4 <= sizeof(AttnRegion::kt), "wave partials staged over the K window");
// V element d of window row j (rows of kHeadDim floats).
__device__ __forceinline__ int attn_v_slot(int j, int d) { return j * kHeadDim + d; }

// One role CU's view of the launch: arguments, LDS, tagged vectors, the
// token state, and the pieces every role shares (the per-token loop, the LM
// head and the argmax). Each role runs its own loop (run_*), so the register
// slots of one role are never live in another role's code.
template <int H, int I, int NQ, int NKV, bool kProfile, typename W>
struct Roles {
  using Sh = Shape<H, I, NQ, NKV, W>;
  static constexpr int QD = Sh::QD, KVD = Sh::KVD, GROUP = Sh::G;
  static constexpr int NJ = PairSlots<H>::NJ;

  const ResidentArgs &a;
  Common &cm;
  unsigned char *region;
  int rank, nrole, wg, lane, wv, grid;  // wg: placement position (the trace row)
  uint32_t per_token;
  TagVec ttop;
  Clock<kProfile> clock;
  uint32_t token, generated = 0, stop_reason = 0;
  float top = 0.f;
  uint32_t flag_parity = 0;
  // The block_all flag set of the next workgroup-wide AND (every wave makes
  // the same sequence of calls).
  __device__ uint32_t *flag_set() {
    flag_parity ^= 1u;
    return cm.flags[flag_parity];
  }

  __device__ Roles(const ResidentArgs &args, unsigned char *lds, int rank_, int nrole_, int wg_)
      : a(args),
        cm(*reinterpret_cast<Common *>(lds)),
        region(lds + kRegionOffset),
        rank(rank_),
        nrole(nrole_),
        wg(wg_),
        lane(lane_id()),
        wv(wave_u()),
        grid(gridDim.x),
        per_token(5u * args.layers + 1u),
        ttop(args.top, 4 * gridDim.x),
        token(args.first_token) {
    clock.start(&cm.clock);
  }

  __device__ uint32_t tag(uint32_t seq) const { return a.epoch | (seq + 1u); }
  __device__ Wait wt() const { return Wait{a.error, a.spin_limit}; }
  // Hand-off vectors inside a slot block (kRoleRecStride-float records).
  static constexpr int kOffQkv = 0;
  static constexpr int kOffPart = QD + 2 * KVD;
  static constexpr int kOffH1 = kOffPart + Sh::PartFloats;
  static constexpr int kOffAct = kOffH1 + NKV * H;
  static constexpr int kOffHid = kOffAct + I;
  static constexpr int kHidFloats = kHidSegment * kMaxRoleGrid;
  static constexpr int kSlotFloats = kOffHid + kHidFloats;
  static_assert(kSlotFloats == roles_slot_floats(H, I, NQ, NKV) && kOffPart % 4 == 0 && H % 4 == 0 &&
                    I % 4 == 0 && kRoleRecStride % 4 == 0,
                "slot layout");
  // A vector of layer l's slot block for token t (the block of t's parity).
  // Token t's writers also clear their slots in the other parity's block
  // (token t + 1's): every CU has finished token t - 1, whose values it
  // held, before any CU starts token t (each waits for the argmax), and the
  // clears are complete (vmcnt) before the writer's next gather returns.
  __device__ Slots slots(int l, uint32_t t, int off, int n, bool xcd_local = false) const {
    return Slots(a.slots + (static_cast<size_t>(l) * 2 + (t & 1u)) * kSlotFloats + off,
                 static_cast<uint32_t>(n), xcd_local);
  }
  // The QKV outputs and the attention records stay inside KV group g's
  // CUs, which the XCD placement puts on XCD g: XCD-local slots then.
  __device__ Slots s_qkv(int l, uint32_t t) const { return slots(l, t, kOffQkv, QD + 2 * KVD, a.xcd_place); }
  __device__ Slots s_part(int l, uint32_t t) const {
    return slots(l, t, kOffPart, Sh::PartFloats, a.xcd_place);
  }
  // Group g's partial of the attention block's output: the O rows over
  // group g's heads (group 0's with the residual added); h1 is their sum in
  // group order.
  __device__ Slots s_h1(int l, uint32_t t, int g) const { return slots(l, t, kOffH1 + g * H, H); }
  // Float4s [first4, first4 + n4) of h1 -> dst, summed in group order (dst
  // and the following NKV - 1 runs of kH1Stride4 float4s are the staging).
  static constexpr int kH1Stride4 = 256;
  static_assert(4 * kH1Stride4 >= H && NKV <= 2, "h1 partials staged in Common's vec and xn");
  __device__ bool gather_h1(uint32_t t, int l, int first4, int n4, float *dst) {
    if (!gather4<(NKV * H / 4 + kT - 1) / kT>(slots(l, t, kOffH1, NKV * H), NKV * n4,
                                              reinterpret_cast<float4 *>(dst), wt(),
                                              flag_set(), [&](int p, int &s4, int &d4) {
                                                const int g = p / n4, q = p % n4;
                                                s4 = g * (H / 4) + first4 + q;
                                                d4 = g * kH1Stride4 + q;
                                              }))
      return false;
    for (int i = threadIdx.x; i < 4 * n4; i += kT) {
      float v = dst[i];
#pragma unroll
      for (int g = 1; g < NKV; ++g) v += dst[g * 4 * kH1Stride4 + i];
      dst[i] = v;
    }
    lds_barrier();
    return true;
  }
  __device__ Slots s_act(int l, uint32_t t) const { return slots(l, t, kOffAct, I); }
  __device__ Slots s_hid(int l, uint32_t t) const { return slots(l, t, kOffHid, kHidFloats); }
  // The down role's split of the layer output: CU r of ndown() owns rows
  // [down_begin(r), down_begin(r + 1)), published as segment r.
  __device__ int ndown() const { return a.role_end[kRoleDown] - a.role_end[kRoleGate]; }
  // split_begin(H, R, r) without an integer division: H r < 2^24 is exact
  // in float, the product with 1/R is within one of the quotient, and one
  // correction step makes it exact.
  __device__ static int down_begin(int r, int R, float inv_r) {
    const int num = H * r;
    int q = static_cast<int>(static_cast<float>(num) * inv_r);
    q -= q * R > num ? 1 : 0;
    q += (q + 1) * R <= num ? 1 : 0;
    return q;
  }
  static_assert(H * kMaxRoleGrid < (1 << 24), "exact float products");
  // Rows [row0, row0 + nrows) of layer l's output -> dst[row - row0]: the
  // segments of the down CUs owning them, whole float4s polled like any
  // hand-off, each valid row scattered to its place.
  static constexpr int kHidMaxPer = 2;
  __device__ bool gather_hid(uint32_t t, int l, int row0, int nrows, float *dst) {
    const int R = ndown();
    const float inv_r = 1.f / static_cast<float>(R);
    // Owner of row i: the largest r with split_begin(H, R, r) <= i
    // (a division by the constant H).
    auto owner = [&](int i) { return ((i + 1) * R - 1) / H; };
    const int r_lo = owner(row0);
    const int items = 4 * (owner(row0 + nrows - 1) - r_lo + 1);
    // Item p: float4 q of segment r; rows [b, e) of that float4 land in dst.
    int first[kHidMaxPer], count[kHidMaxPer];
    return gather4_put<kHidMaxPer>(
        s_hid(l, t), items, wt(), flag_set(),
        [&](int p, int k, int &s4) {
          const int r = r_lo + p / 4, q = p % 4;
          s4 = (kHidSegment / 4) * r + q;
          const int b = down_begin(r, R, inv_r) + 4 * q;
          const int e = min(down_begin(r + 1, R, inv_r), b + 4);
          first[k] = b;
          count[k] = e - b;
          return e > b;
        },
        [&](int k, float4 v) {
          const int b = first[k], c = count[k];
          const float x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int row = b + j;
            if (j < c && row >= row0 && row < row0 + nrows) dst[row - row0] = x[j];
          }
        });
  }
  // The host plan never gives a CU more units than it holds on chip; a plan
  // that did is reported as an error (the other CUs' waits then give up).
  __device__ bool fits(int n, int capacity) const {
    if (n <= capacity) return true;
    if (threadIdx.x == 0) atomicOr(a.error, kResidentPlanOverfill);
    return false;
  }
  __device__ uint32_t seqno(uint32_t t, int l, int s) const { return t * per_token + 5u * l + s; }
  // Layer l's weight pointers, read through the scalar cache (the table is
  // written once before any launch): a vector load of it would be waited
  // for with vmcnt, i.e. behind every store and DMA issued before it.
  __device__ LayerPtrs layer(int l) const {
    typedef const __attribute__((address_space(4))) uint64_t kword;
    kword *src = (kword *)(reinterpret_cast<uint64_t>(a.layer_ptrs) + sizeof(LayerPtrs) * l);
    LayerPtrs r;
    uint64_t *dst = reinterpret_cast<uint64_t *>(&r);
#pragma unroll
    for (size_t i = 0; i < sizeof(LayerPtrs) / 8; ++i) dst[i] = src[i];
    return r;
  }
  __device__ const float *kv_layer(const float *base, int l) const {
    return base + static_cast<size_t>(l) * a.capacity * KVD;
  }

  // The per-token loop. layer(t, l, position) runs one layer of this role
  // (including the prefetch of its next share) and returns false when a
  // wait gave up; pre_lds(l, position) / pre_regs(l) issue a layer's share.
  // defer_first: the role issues even the LDS part of the next token's
  // layer-0 share after the LM head (its last layer ends right before the
  // LM head's input poll, which would otherwise queue behind it).
  template <typename Layer, typename PreLds, typename PreRegs>
  __device__ void loop(int role, bool defer_first, Layer layer, PreLds pre_lds, PreRegs pre_regs) {
    pre_lds(0, static_cast<int>(a.start_position));
    pre_regs(0);
    clock.lap(2 * role + 1);
    for (uint32_t t = 0; t < a.max_tokens; ++t) {
      const int position = static_cast<int>(a.start_position + t);
      if (token >= static_cast<uint32_t>(a.vocab) || position >= a.capacity) break;
      const bool traced = a.trace != nullptr && t == a.trace_token;
      for (int l = 0; l < a.layers; ++l) {
        clock.at(traced, l);
        if (!layer(t, l, position)) return;
      }
      clock.at(traced, a.layers);
      if (!lm_head(t)) return;
      if (defer_first) pre_lds(0, position + 1);
      pre_regs(0);  // register share of layer 0 for the next token
      if (!argmax(t)) return;
      if (traced) clock.flush_trace(a.trace, wg, a.layers, role);
      generated = t + 1;
      if (blockIdx.x == 0 && threadIdx.x == 0)
        *(__attribute__((address_space(1))) uint32_t *)(a.out_tokens + t) = token;
      if (token == UINT32_MAX) break;  // every logit NaN
      if (token == a.eos) {
        stop_reason = 2u;
        break;
      }
      if (generated >= a.max_tokens) {
        stop_reason = 1u;
        break;
      }
    }
    clock.publish(a.stage_ticks, role, rank == 0);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      SeqState *st = a.st;
      st->position = a.start_position + generated;
      st->token = token;
      st->generated = generated;
      st->stop_reason = stop_reason;
      st->stopped = 1u;
      st->top_logit = top;
      st->eos = a.eos;
      st->max_tokens = a.max_tokens;
      st->mode = kModeGenerate;
    }
  }

  // ---- LM head + per-CU top-1 (every CU) ------------------------------------
  __device__ bool lm_head(uint32_t t) {
    const uint32_t par = t & 1u;
    const uint32_t tag_top = tag(t * per_token + 5u * a.layers);
    const int units = (a.vocab + 1) / 2;
    const int gw = static_cast<int>(blockIdx.x) * kW + wv;
    const int stride = grid * kW;
    auto load = [&](int u, float4 (&w)[NJ]) {
      if (u < units) {
        const float *ra = a.head + static_cast<size_t>(2 * u) * H;
        const float *rb = 2 * u + 1 < a.vocab ? ra + H : ra;
        load_pair_weights<H>(ra, rb, w);
      }
    };
    float4 w0[NJ], w1[NJ], w2[NJ];
    float4 gv[NJ];
    load_pair_gain<H>(a.final_norm, gv);
    load(gw, w0);
    __builtin_amdgcn_sched_barrier(0);
    if (!gather_hid(t, a.layers - 1, 0, H, cm.vec)) return false;
    clock.lap(2 * kRoleCount);
    float4 xv[NJ];
    const float inv = norm_scale(load_pair_operand_gain<H>(Lds{cm.vec}, gv, xv), H, a.eps);
    float best = -INFINITY;
    uint32_t best_i = UINT32_MAX;
    float *logits = a.logits + (a.history ? static_cast<size_t>(t) * a.vocab : 0);
    auto step = [&](int u, const float4 (&w)[NJ]) {
      float sa, sb;
      pair_dot<H>(w, xv, sa, sb);
      sa *= inv;
      sb *= inv;
      const int r0 = 2 * u;
      const bool has1 = r0 + 1 < a.vocab;
      if (lane == 0) {
        typedef __attribute__((address_space(1))) float gfloat;
        gfloat *out = (gfloat *)(logits + r0);
        out[0] = sa;
        if (has1) out[1] = sb;
      }
      if (better(sa, r0, best, best_i)) {
        best = sa;
        best_i = r0;
      }
      if (has1 && better(sb, r0 + 1, best, best_i)) {
        best = sb;
        best_i = r0 + 1;
      }
    };
    load(gw + stride, w1);
    for (int u = gw; u < units; u += 3 * stride) {
      load(u + 2 * stride, w2);
      step(u, w0);
      if (u + stride >= units) break;
      load(u + 3 * stride, w0);
      step(u + stride, w1);
      if (u + 2 * stride >= units) break;
      load(u + 4 * stride, w1);
      step(u + 2 * stride, w2);
    }
    if (lane == 0) {
      cm.bv[wv] = best;
      cm.bi[wv] = best_i;
    }
    lds_barrier();
    if (threadIdx.x == 0) {
      for (int v = 1; v < kW; ++v) {
        if (better(cm.bv[v], cm.bi[v], best, best_i)) {
          best = cm.bv[v];
          best_i = cm.bi[v];
        }
      }
      ttop.put(par * 2 * grid + 2 * blockIdx.x, best, tag_top);
      ttop.put(par * 2 * grid + 2 * blockIdx.x + 1, __builtin_bit_cast(float, best_i), tag_top);
    }
    lds_barrier();  // cm.bv/bi are reused by the argmax
    clock.lap(2 * kRoleCount + 1);
    return true;
  }

  // ---- argmax over the workgroup partials (every CU) ------------------------
  __device__ bool argmax(uint32_t t) {
    const uint32_t par = t & 1u;
    const uint32_t tag_top = tag(t * per_token + 5u * a.layers);
    if (!gather<(kMaxRoleGrid + kT - 1) / kT>(ttop, par * 2 * grid, 2 * grid, tag_top, cm.top,
                                              wt(), flag_set()))
      return false;
    clock.lap(2 * kRoleCount + 2);
    float best = -INFINITY;
    uint32_t best_i = UINT32_MAX;
    for (int p = threadIdx.x; p < grid; p += kT) {
      const float v = cm.top[2 * p];
      const uint32_t i = __builtin_bit_cast(uint32_t, cm.top[2 * p + 1]);
      if (better(v, i, best, best_i)) {
        best = v;
        best_i = i;
      }
    }
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
      const float ov = __shfl_xor(best, o, kWave);
      const uint32_t oi = __shfl_xor(best_i, o, kWave);
      if (better(ov, oi, best, best_i)) {
        best = ov;
        best_i = oi;
      }
    }
    if (lane == 0) {
      cm.bv[wv] = best;
      cm.bi[wv] = best_i;
    }
    lds_barrier();
    best = cm.bv[0];
    best_i = cm.bi[0];
    for (int v = 1; v < kW; ++v) {
      if (better(cm.bv[v], cm.bi[v], best, best_i)) {
        best = cm.bv[v];
        best_i = cm.bi[v];
      }
    }
    lds_barrier();
    token = best_i;
    top = best;
    clock.lap(2 * kRoleCount + 3);
    return true;
  }

  // Floats [4 first4, 4 (first4 + n4)) of layer l's input (the previous
  // layer's output, or this token's embedding row at l = 0) -> dst.
  __device__ bool layer_input(uint32_t t, int l, int first4, int n4, float *dst) {
    if (l == 0) {
      const float *e = a.embed + static_cast<size_t>(token) * H;
      for (int c = threadIdx.x; c < n4; c += kT) reinterpret_cast<float4 *>(dst)[c] = ld_global4(e, first4 + c);
      vm_wait();
      lds_barrier();
      return true;
    }
    return gather_hid(t, l - 1, 4 * first4, min(4 * n4, H - 4 * first4), dst);
  }

  // ---- QKV ------------------------------------------------------------------
  __device__ void run_qkv() {
    // The role's CUs come in KV-group blocks of group_cus[0]. Group g's
    // units, in order: its G query heads, then K head g, then V head g (32
    // units = one packed head each; unit u is rows (u / 32) * 64 + u % 32
    // and 32 further on); each of the group's CUs takes a run of them.
    const int gq = a.group_cus[0];
    const int g = rank / gq, rr = rank % gq;
    constexpr int GU = (GROUP + 2) * kRotary;
    const int j0 = split_begin(GU, gq, rr);
    PairRole<H, kSlotsQ, Sh::LQ, W> rq;
    rq.n = split_begin(GU, gq, rr + 1) - j0;
    rq.units = region;
    if (!fits(rq.n, rq.capacity())) return;
    // Packed head of the group's local head lh (0..G-1 query, G: K, G+1: V).
    auto head_of = [&](int lh) { return lh < GROUP ? GROUP * g + lh : (lh == GROUP ? NQ + g : NQ + NKV + g); };
    auto unit_of = [&](int j) { return head_of(j / kRotary) * kRotary + j % kRotary; };
    float4 *q_bias = reinterpret_cast<float4 *>(region + Sh::LQ * Sh::UnitBytes);
    float4 *q_cs = q_bias + Sh::BiasF4;
    auto rows = [&](int l) {
      const W *base = reinterpret_cast<const W *>(layer(l).wqkv);
      return [=](int k, const W *&ra, const W *&rb) {
        const int u = unit_of(j0 + k);
        const int row = (u / kRotary) * kHeadDim + u % kRotary;
        ra = base + static_cast<size_t>(row) * H;
        rb = ra + static_cast<size_t>(kRotary) * H;
      };
    };
    // Biases of every packed row and the cos|sin row of the position
    // (clamped to the table) travel with the weights.
    auto pre_lds = [&](int l, int position) {
      rq.prefetch_lds(rows(l));
      if (wv != 0) return;
      const float4 *b4 = reinterpret_cast<const float4 *>(layer(l).bqkv);
      for (int i = 0; i < Sh::BiasF4 / kWave; ++i) {
        const int f = i * kWave + lane;
        dma16<kPolicyNt>(b4 + (f < Sh::QkvRows / 4 ? f : 0), q_bias + i * kWave);
      }
      const int p = min(position, a.capacity - 1);
      const float4 *c4 = reinterpret_cast<const float4 *>(a.rope_cos + static_cast<size_t>(p) * kRotary);
      const float4 *s4 = reinterpret_cast<const float4 *>(a.rope_sin + static_cast<size_t>(p) * kRotary);
      constexpr int R4 = kRotary / 4;
      dma16<kPolicyNt>(lane < R4 ? c4 + lane : (lane < 2 * R4 ? s4 + (lane - R4) : c4), q_cs);
    };
    auto pre_regs = [&](int l) { rq.prefetch_regs(rows(l)); };
    // Each local head lh this CU touches is two runs of its packed head's
    // slots (rows ib.. and 32 + ib..), staged at 64 (lh - lh0); thread i owns
    // float4 i of those runs taken in order (tagged with the packed head).
    const int lh0 = j0 / kRotary;
    OutMap om;
    {
      int item = threadIdx.x;
      for (int lh = lh0; lh <= (j0 + rq.n - 1) / kRotary; ++lh) {
        const int h = head_of(lh);
        const int sb = h * kHeadDim - kHeadDim * (lh - lh0);
        const int ib = max(j0, lh * kRotary) - lh * kRotary;
        const int ie = min(j0 + rq.n, (lh + 1) * kRotary) - lh * kRotary;
        item -= om.take(h * kHeadDim + ib, ie - ib, sb, item, h);
        item -= om.take(h * kHeadDim + kRotary + ib, ie - ib, sb, item, h);
      }
    }
    loop(kRoleQkv, false, [&](uint32_t t, int l, int position) {
      const LayerPtrs lw = layer(l);
      const Slots out = s_qkv(l, t);
      if (om.q >= 0) clear_quad(s_qkv(l, t + 1), om);
      float4 gv[NJ];
      load_pair_gain<H>(lw.attn_norm, gv);
      rq.settle();
      if (!layer_input(t, l, 0, H / 4, cm.vec)) return false;
      clock.lap(2 * kRoleQkv);
      float4 xv[NJ];
      const float inv = norm_scale(load_pair_operand_gain<H>(Lds{cm.vec}, gv, xv), H, a.eps);
      clock.mark(0);
      const float *bias = reinterpret_cast<const float *>(q_bias);
      const float *cs = reinterpret_cast<const float *>(q_cs);
      const Coherent kcache(kv_layer(a.k_cache, l), static_cast<uint32_t>(a.capacity) * KVD * 4u);
      const Coherent vcache(kv_layer(a.v_cache, l), static_cast<uint32_t>(a.capacity) * KVD * 4u);
      float *stage = cm.top;
      rq.compute(xv, [&](int k) {
        const int u = unit_of(j0 + k);
        const int ra = (u / kRotary) * kHeadDim + u % kRotary;
        return make_float4(bias[ra], bias[ra + kRotary], cs[u % kRotary], cs[kRotary + u % kRotary]);
      }, [&](int k, float sa, float sb, float4 c) {
        const int j = j0 + k;
        const int head = head_of(j / kRotary);
        const int slot = kHeadDim * (j / kRotary - lh0) + j % kRotary;
        const float x0 = fmaf(sa, inv, c.x);
        const float x1 = fmaf(sb, inv, c.y);
        if (head < NQ + NKV) {
          const float cv = c.z, sv = c.w;
          rope_rotate(x0, x1, cv, sv, stage[slot], stage[slot + kRotary]);
        } else {
          stage[slot] = x0;
          stage[slot + kRotary] = x1;
        }
      }, [&] { clock.mark(1); });
      lds_barrier();
      if (om.q >= 0) {
        // The slots and, for a K or V head, the cache row (slot e of K head
        // g is cache element position * KVD + e - QD, of V head g
        // position * KVD + e - QD - KVD).
        const float4 v = reinterpret_cast<const float4 *>(stage)[om.soff];
        put_quad(out, om, v);
        if (om.tag >= NQ + NKV)
          put_quad(vcache, om, v, (position * KVD - QD - KVD) / 4);
        else if (om.tag >= NQ)
          put_quad(kcache, om, v, (position * KVD - QD) / 4);
      }
      clock.mark(2);
      lds_barrier();  // LDS units, biases and cos|sin are rewritten next
      clock.lap(2 * kRoleQkv + 1);
      if (l + 1 < a.layers) {
        pre_lds(l + 1, position);
        pre_regs(l + 1);
      } else {
        pre_lds(0, position + 1);
      }
      return true;
    }, pre_lds, pre_regs);
  }

  // ---- attention ----------------------------------------------------------
  // Chunk c of KV group g is handled by the group's attention CU c % na. A
  // chunk's K (by float4 columns) and V rows are staged in LDS in windows of
  // kAttnCap positions; the first window of a CU's first chunk is loaded
  // ahead with the other roles' weights.
  __device__ void attn_dma(int l, int g, int wb, int we, AttnRegion &ar) {
    const float *kc = kv_layer(a.k_cache, l);
    const float *vc = kv_layer(a.v_cache, l);
    const int nrow = we - wb;
    const int nblk = (nrow + kWave - 1) / kWave;
    for (int i = wv; i < (kHeadDim / 4) * nblk; i += kW) {
      const int blk = i / (kHeadDim / 4), d4 = i % (kHeadDim / 4);
      const int pos = min(wb + blk * kWave + lane, a.capacity - 1);
      dma16<kPolicySc1>(kc + static_cast<size_t>(pos) * KVD + g * kHeadDim + 4 * d4,
                        ar.kt + d4 * kAttnCap + blk * kWave);
    }
    for (int i = wv; i < (nrow + 3) / 4; i += kW) {
      const int pos = min(wb + 4 * i + lane / 16, a.capacity - 1);
      dma16<kPolicySc1>(vc + static_cast<size_t>(pos) * KVD + g * kHeadDim + 4 * (lane % 16),
                        ar.vr + 4 * i * kHeadDim);
    }
  }

  // kMode (ResidentArgs::attn_mode): 0, both chunk forms; 1, every chunk of
  // the launch is longer than one block, so the one-block (vector ALU) form
  // is left out of the instance; 2, no chunk is, so the MFMA tiles and their
  // register window are left out. Each instance's code then gets the role's
  // registers to itself.
  template <int kMode>
  __device__ void run_attn() {
    static_assert(GROUP <= kAttnMaxGroup, "an attention tile takes up to 8 heads per KV group");
    AttnRegion &ar = *reinterpret_cast<AttnRegion *>(region);
    // The role's CUs come in KV-group blocks of group_cus[1]: CU rr of group
    // g takes the group's chunks rr, rr + group_cus[1], ...
    const int na = a.group_cus[1];
    const int g = rank / na, rr = rank % na;
    // The second window of a CU's first chunk is loaded a layer ahead too,
    // into registers: wave w's tile of it (tile kAttnSlots + w of the chunk),
    // this lane's K half (kw2) and its V element of each position (vw2), the
    // tile's arithmetic being attn_tile's (attn_tile_ops).
    float4 kw2[kHeadDim / 8];
    float vw2[kAttnTile];
    auto pre_lds = [&](int l, int position) {
      const int length = position + 1;
      const int chunks = attn_chunks(length, a.attn_parts, kAttnGrain), cl = attn_chunk_len(length, a.attn_parts, kAttnGrain);
      if (rr >= chunks || position >= a.capacity) return;
      const int begin = rr * cl, end = min(length, begin + cl);
      attn_dma(l, g, begin, min(end, begin + kAttnCap), ar);
      const int t0 = begin + kAttnCap + wv * kAttnTile;
      if (kMode != 2 && t0 < end) {
        const Coherent kc(kv_layer(a.k_cache, l), static_cast<uint32_t>(a.capacity) * KVD * 4u);
        const Coherent vc(kv_layer(a.v_cache, l), static_cast<uint32_t>(a.capacity) * KVD * 4u);
        const int pk = min(t0 + (lane & 31), end - 1);
        const uint32_t k4 = (static_cast<uint32_t>(pk) * KVD + g * kHeadDim + (kHeadDim / 2) * (lane >> 5)) / 4;
#pragma unroll
        for (int i = 0; i < kHeadDim / 8; ++i) kw2[i] = kc.ld4(k4 + i);
#pragma unroll
        for (int k = 0; k < kAttnTile; ++k)
          vw2[k] = vc.ld(static_cast<uint32_t>(min(t0 + k, end - 1)) * KVD + g * kHeadDim + lane);
      }
    };
    auto pre_regs = [](int) {};
    loop(kRoleAttn, false, [&](uint32_t t, int l, int position) {
      const int length = position + 1;
      const int chunks = attn_chunks(length, a.attn_parts, kAttnGrain), cl = attn_chunk_len(length, a.attn_parts, kAttnGrain);
      const Slots in = s_qkv(l, t), out = s_part(l, t);
      // Record (h, c) is kRoleRecStride floats at (h * kAttnMaxChunks + c) *
      // kRoleRecStride: whole float4s.
      constexpr int kRec4 = kRoleRecStride / 4;
      {
        // The group's records token t + 1 reads (its own chunk count),
        // spread over the group's CUs like its chunks. This holds however the
        // count moves: it drops when the chunk length grows (context 1024 ->
        // 1025) and regrows later, which leaves older records in slots beyond
        // it.
        const Slots next = s_part(l, t + 1);
        const int chunks_next = attn_chunks(length + 1, a.attn_parts, kAttnGrain);
        for (int c = rr; c < chunks_next; c += na) {
          for (int e = threadIdx.x; e < GROUP * kRec4; e += kT)
            next.clear4(((g * GROUP + e / kRec4) * kAttnMaxChunks + c) * kRec4 + e % kRec4);
        }
      }
      bool first_unit = true;
      float *ps = ar.ps + wv * kAttnPsFloats;
      float *kst = reinterpret_cast<float *>(ar.kt);
      const AttnStage stage{kst, kst + kAttnSlots * kMaxGroup, kst + 2 * kAttnSlots * kMaxGroup};
      for (int c = rr; c < chunks; c += na) {
        const int begin = c * cl;
        const int end = min(length, begin + cl);
        const bool has_new = position >= begin && position < end;
        if (!first_unit) {
          lds_barrier();
          attn_dma(l, g, begin, min(end, begin + kAttnCap), ar);
        }
        // The group's queries, then this step's K and V rows (float4s).
        constexpr int q4 = GROUP * kHeadDim / 4, r4 = kHeadDim / 4;
        const int n4 = q4 + (has_new ? 2 * r4 : 0);
        if (!gather4<(q4 + 2 * r4 + kT - 1) / kT>(in, n4, reinterpret_cast<float4 *>(ar.qs), wt(),
                                                  flag_set(), [&](int p, int &s, int &d) {
              if (p < q4) {
                s = g * q4 + p;
                d = p;
              } else if (p < q4 + r4) {
                s = (QD + g * kHeadDim) / 4 + (p - q4);
                d = kW * r4 + (p - q4);
              } else {
                s = (QD + KVD + g * kHeadDim) / 4 + (p - q4 - r4);
                d = kW * r4 + r4 + (p - q4 - r4);
              }
            }))
          return false;
        if (first_unit) clock.lap(2 * kRoleAttn);
        if constexpr (kMode == 2) {
          if (!attn_single_block(cl)) {  // the host's mode would be wrong
            if (threadIdx.x == 0) atomicOr(a.error, kResidentPlanOverfill);
            return false;
          }
        }
        if (kMode == 2 || (kMode == 0 && attn_single_block(cl))) {
          // One block (the window, loaded ahead): wave h takes head h, its
          // query in registers, and stores the head's record (m, l, two pad
          // words, acc[64]) itself: one contiguous 256-byte store of acc and
          // one of the head words.
          if (position >= begin && position < end) {
            const int j = position - begin;
            if (threadIdx.x < kHeadDim / 4)
              ar.kt[threadIdx.x * kAttnCap + j] = reinterpret_cast<const float4 *>(ar.kn)[threadIdx.x];
            if (threadIdx.x < kHeadDim) ar.vr[attn_v_slot(j, threadIdx.x)] = ar.vn[threadIdx.x];
          }
          lds_barrier();
          clock.mark(0);
          if (wv < GROUP) {
            float4 q[kHeadDim / 4];
#pragma unroll
            for (int d4 = 0; d4 < kHeadDim / 4; ++d4)
              q[d4] = reinterpret_cast<const float4 *>(ar.qs + wv * kHeadDim)[d4];
            PLds pb{ps + 4, kWave};
            float bm[1], bl[1], ba[1];
            attn_block_valu<1>([&](int d4, int j) { return ar.kt[d4 * kAttnCap + j]; },
                               [&](int, int d4) { return q[d4]; },
                               [&](int j, int d) { return ar.vr[attn_v_slot(j, d)]; }, pb, 0, end - begin - 1, bm,
                               bl, ba);
            float M = -INFINITY, L = 0.f, A = 0.f;
            attn_fold(bm[0], bl[0], ba[0], M, L, A);
            clock.mark(1);
            const uint32_t rec = ((g * GROUP + wv) * kAttnMaxChunks + c) * kRoleRecStride;
            out.put(rec + 4 + lane, A);
            if (lane < 4) out.put(rec + lane, lane == 0 ? M : lane == 1 ? L : 0.f);
          }
          clock.mark(2);
          first_unit = false;
          continue;
        }
        float4 qa[kHeadDim / 4];
        attn_query([&](int h, int d4) { return reinterpret_cast<const float4 *>(ar.qs + h * kHeadDim)[d4]; },
                   GROUP, qa);
        // Wave w's running partial over the chunk's tiles w, w + kW, ...,
        // window by window.
        AttnAcc acc;
        acc.init();
        for (int wb = begin; wb < end; wb += kAttnCap) {
          const int we = min(end, wb + kAttnCap);
          if (first_unit && wb == begin + kAttnCap) {
            // The second window from registers (no LDS, no barrier). When
            // the new position lies in this chunk it is the chunk's last
            // (end - 1), where the tile's reads past the end are clamped
            // too: those take the gathered row instead of the prefetched
            // cache row, as the LDS windows do.
            const int t0 = wb + wv * kAttnTile;
            if (t0 < end) {
              const int knew = has_new ? position - t0 : kAttnTile;
              const int hq = lane >> 5;
              const bool kfresh = (lane & 31) >= knew;
              const float vfresh = ar.vn[lane];
              attn_tile_ops(
                  qa,
                  [&](int i) {
                    // The fresh row as a register value (pin): a choice
                    // between two loads would be folded into one load
                    // through a generic pointer, keeping kw2 in scratch.
                    float4 f = reinterpret_cast<const float4 *>(ar.kn)[(kHeadDim / 8) * hq + i];
                    pin(f);
                    return kfresh ? f : kw2[i];
                  },
                  [&](int k) { return k >= knew ? vfresh : vw2[k]; }, ps, t0, end, acc);
            }
            continue;
          }
          if (wb != begin) {
            lds_barrier();
            attn_dma(l, g, wb, we, ar);
            vm_wait();
            lds_barrier();
          }
          if (position >= wb && position < we) {
            const int j = position - wb;
            if (threadIdx.x < kHeadDim / 4)
              ar.kt[threadIdx.x * kAttnCap + j] = reinterpret_cast<const float4 *>(ar.kn)[threadIdx.x];
            if (threadIdx.x < kHeadDim) ar.vr[attn_v_slot(j, threadIdx.x)] = ar.vn[threadIdx.x];
          }
          lds_barrier();
          if (wb == begin) clock.mark(0);
          attn_slot_tiles(qa, [&](int pos, int d4) { return ar.kt[d4 * kAttnCap + (pos - wb)]; },
                          [&](int pos, int d) { return ar.vr[attn_v_slot(pos - wb, d)]; }, ps, begin, wb, we, end,
                          wv, acc);
        }
        clock.mark(1);
        // The wave partials replace the K window, then wave h folds head
        // h's in slot order (lane = dim) and stores the head's record (m,
        // l, two pad words, acc[64]): one contiguous 256-byte store of acc
        // and one of the head words. A reader takes a float4 once none of
        // its words is kSlotEmpty, so it never sees a partly written one.
        lds_barrier();
        stage.put(wv, GROUP, acc);
        lds_barrier();
        if (wv < GROUP) {
          float M, L, A;
          attn_slot_merge(stage, (end - begin + kAttnTile - 1) / kAttnTile, wv, lane, M, L, A);
          const uint32_t rec = ((g * GROUP + wv) * kAttnMaxChunks + c) * kRoleRecStride;
          out.put(rec + 4 + lane, A);
          if (lane < 4) out.put(rec + lane, lane == 0 ? M : lane == 1 ? L : 0.f);
        }
        clock.mark(2);
        first_unit = false;
      }
      if (first_unit) clock.lap(2 * kRoleAttn);
      lds_barrier();  // K/V windows and queries are rewritten next
      clock.lap(2 * kRoleAttn + 1);
      if (l + 1 < a.layers)
        pre_lds(l + 1, position);
      else
        pre_lds(0, position + 1);
      return true;
    }, pre_lds, pre_regs);
  }

  // ---- O projection ---------------------------------------------------------
  __device__ void run_o() {
    // The role's CUs come in KV-group blocks of group_cus[2]; a group's CUs
    // split every output row pair, each over the group's QDG columns.
    constexpr int QDG = Sh::QDG;
    const int gn = a.group_cus[2];
    const int g = rank / gn, rr = rank % gn;
    const int u0 = split_begin(Sh::OUnits, gn, rr);
    PairRole<QDG, kSlotsO, Sh::LO, W> ro;
    ro.n = split_begin(Sh::OUnits, gn, rr + 1) - u0;
    ro.units = region;
    if (!fits(ro.n, ro.capacity())) return;
    // The group's partial records in LDS: record (head 7g + j, c) at
    // (j * kAttnMaxChunks + c) * kRoleRecStride. The merge reads chunks
    // beyond the token's count too (discarded by a select); the zero fill
    // keeps what they read finite until some token has gathered them.
    float *parts = reinterpret_cast<float *>(region + Sh::LO * Sh::OUnitBytes);
    for (int i = threadIdx.x; i < Sh::PartFloatsG; i += kT) parts[i] = 0.f;
    auto rows = [&](int l) {
      const W *base = reinterpret_cast<const W *>(layer(l).wo) + g * QDG;
      return [=](int k, const W *&ra, const W *&rb) {
        ra = base + static_cast<size_t>(2 * (u0 + k)) * QD;
        rb = ra + QD;
      };
    };
    auto pre_lds = [&](int l, int) { ro.prefetch_lds(rows(l)); };
    auto pre_regs = [&](int l) { ro.prefetch_regs(rows(l)); };
    OutMap om;  // rows [2 u0, 2 u0 + 2 n), staged from element 2 u0 rounded down to 4
    om.take(2 * u0, 2 * ro.n, (2 * u0) & ~3, threadIdx.x, 0);
    loop(kRoleO, false, [&](uint32_t t, int l, int position) {
      const int C = attn_chunks(position + 1, a.attn_parts, kAttnGrain);
      const Slots out = s_h1(l, t, g);
      if (om.q >= 0) clear_quad(s_h1(l, t + 1, g), om);
      // Group 0 adds the residual: rows [2 u0, 2 u0 + 2 n) of the layer
      // input, in the float4s covering them (row r at cm.vec[r - 4 f4]).
      const int f4 = (2 * u0) / 4, e4 = (2 * (u0 + ro.n) + 3) / 4;
      const int roff = 2 * u0 - 4 * f4;
      ro.settle();
      if (g == 0 && !layer_input(t, l, f4, e4 - f4, cm.vec)) return false;
      // The partial records of the group's heads over C chunks; one pass
      // covers sixteen chunks.
      constexpr int kRec4 = kRoleRecStride / 4;
      constexpr int kPer = (GROUP * kAttnMaxChunks * kRec4 + kT - 1) / kT;
      static_assert(kPer <= 8, "partial gather pass");
      const Slots in = s_part(l, t);
      const int n4 = GROUP * C * kRec4;
      if (!gather4<kPer>(in, n4, reinterpret_cast<float4 *>(parts), wt(), flag_set(), [&](int p, int &s, int &d) {
            const int rec = p / kRec4, k = p % kRec4;
            const int j = rec / C, c = rec % C;
            s = ((g * GROUP + j) * kAttnMaxChunks + c) * kRec4 + k;
            d = (j * kAttnMaxChunks + c) * kRec4 + k;
          }))
        return false;
      clock.lap(2 * kRoleO);
      // Merge, in attn_merge's arithmetic: wave j takes the group's head j.
      // Lane c of each 16-lane row (one per chunk place) forms the head's M
      // (row16_max), w_c = 2^(m_c - M) (zero past C) and den (row16_sum of
      // the products w_c l_c, in every lane); lane d then folds its dim's
      // numerator over the chunks in order, w_c read from lane c. Specialised
      // on the exact C; the record reads are issued first, and no step waits
      // for another wave.
      static_assert(kHeadDim == kWave && GROUP <= kW && kAttnMaxChunks == 16, "merge layout");
      if (wv < GROUP) {
        auto merge = [&](auto c_tag) {
          constexpr int kC = decltype(c_tag)::value;
          const float *rec = parts + wv * kAttnMaxChunks * kRoleRecStride;
          float av[kC];
#pragma unroll
          for (int c = 0; c < kC; ++c) av[c] = rec[c * kRoleRecStride + 4 + lane];
          const int c = lane & (kAttnMaxChunks - 1);
          const float2 ml = *reinterpret_cast<const float2 *>(rec + c * kRoleRecStride);
          const bool in = c < C;
          const float mx = row16_max(in ? ml.x : -INFINITY);
          const float w = in ? exp2_fast(ml.x - mx) : 0.f;
          const float den = row16_sum(in ? __fmul_rn(w, ml.y) : 0.f);
          float num = 0.f;
#pragma unroll
          for (int k = 0; k < kC; ++k) num = fmaf(read_lane(w, k), av[k], num);
          cm.xn[wv * kHeadDim + lane] = num / den;
        };
        switch (C) {
#define QD_MERGE_CASE(n) \
  case n:                \
    merge(std::integral_constant<int, n>{}); \
    break;
          QD_MERGE_CASE(1) QD_MERGE_CASE(2) QD_MERGE_CASE(3) QD_MERGE_CASE(4)
          QD_MERGE_CASE(5) QD_MERGE_CASE(6) QD_MERGE_CASE(7) QD_MERGE_CASE(8)
          QD_MERGE_CASE(9) QD_MERGE_CASE(10) QD_MERGE_CASE(11) QD_MERGE_CASE(12)
          QD_MERGE_CASE(13) QD_MERGE_CASE(14) QD_MERGE_CASE(15)
          default: merge(std::integral_constant<int, 16>{}); break;
#undef QD_MERGE_CASE
        }
      }
      lds_barrier();
      float4 xv[PairSlots<QDG>::NJ];
      load_pair_operand<QDG>(Lds{cm.xn}, xv);
      float *stage = cm.top;  // row 2 u0 + j at stage[j + roff]
      clock.mark(0);
      ro.compute(xv,
                 [&](int k) {
                   return g == 0 ? make_float4(cm.vec[roff + 2 * k], cm.vec[roff + 2 * k + 1], 0.f, 0.f)
                                 : make_float4(0.f, 0.f, 0.f, 0.f);
                 },
                 [&](int k, float sa, float sb, float4 c) {
                   stage[2 * k + roff] = g == 0 ? c.x + sa : sa;
                   stage[2 * k + 1 + roff] = g == 0 ? c.y + sb : sb;
                 },
                 [&] { clock.mark(1); });
      lds_barrier();
      if (om.q >= 0) put_quad(out, om, reinterpret_cast<const float4 *>(stage)[om.soff]);
      clock.mark(2);
      lds_barrier();
      clock.lap(2 * kRoleO + 1);
      if (l + 1 < a.layers) {
        pre_lds(l + 1, position);
        pre_regs(l + 1);
      } else {
        pre_lds(0, position + 1);
      }
      return true;
    }, pre_lds, pre_regs);
  }

  // ---- gate/up + SiLU -------------------------------------------------------
  __device__ void run_gate() {
    // Whole float4s of the activation per CU, so no float4 has two writers.
    static_assert(I % 4 == 0, "activation in float4s");
    const int u0 = 4 * split_begin(I / 4, nrole, rank);
    PairRole<H, kSlotsG, Sh::LG, W> rg;
    rg.n = 4 * split_begin(I / 4, nrole, rank + 1) - u0;
    rg.units = region;
    if (!fits(rg.n, rg.capacity())) return;
    auto rows = [&](int l) {
      const LayerPtrs lp = layer(l);
      const W *g = reinterpret_cast<const W *>(lp.wg), *u = reinterpret_cast<const W *>(lp.wu);
      return [=](int k, const W *&ra, const W *&rb) {
        ra = g + static_cast<size_t>(u0 + k) * H;
        rb = u + static_cast<size_t>(u0 + k) * H;
      };
    };
    auto pre_lds = [&](int l, int) { rg.prefetch_lds(rows(l)); };
    auto pre_regs = [&](int l) { rg.prefetch_regs(rows(l)); };
    OutMap om;  // units [u0, u0 + n), staged from u0 rounded down to 4
    om.take(u0, rg.n, u0 & ~3, threadIdx.x, 0);
    loop(kRoleGate, false, [&](uint32_t t, int l, int position) {
      const Slots out = s_act(l, t);
      if (om.q >= 0) clear_quad(s_act(l, t + 1), om);
      float *stage = cm.top;  // unit u0 + k at stage[k + (u0 & 3)]
      float4 gv[NJ];
      load_pair_gain<H>(layer(l).mlp_norm, gv);
      rg.settle();
      if (!gather_h1(t, l, 0, H / 4, cm.vec)) return false;
      clock.lap(2 * kRoleGate);
      float4 xv[NJ];
      const float inv = norm_scale(load_pair_operand_gain<H>(Lds{cm.vec}, gv, xv), H, a.eps);
      clock.mark(0);
      rg.compute(xv, [](int) { return make_float4(0.f, 0.f, 0.f, 0.f); },
                 [&](int k, float gs, float us, float4) {
                   stage[k + (u0 & 3)] = silu_mul(gs * inv, us * inv);
                 },
                 [&] { clock.mark(1); });
      lds_barrier();
      if (om.q >= 0) put_quad(out, om, reinterpret_cast<const float4 *>(stage)[om.soff]);
      clock.mark(2);
      lds_barrier();
      clock.lap(2 * kRoleGate + 1);
      if (l + 1 < a.layers) {
        pre_lds(l + 1, position);
        pre_regs(l + 1);
      } else {
        pre_lds(0, position + 1);
      }
      return true;
    }, pre_lds, pre_regs);
  }

  // ---- down + residual ------------------------------------------------------
  __device__ void run_down() {
    const int u0 = split_begin(H, nrole, rank);
    DownRole<I, W> rd;
    const int n = split_begin(H, nrole, rank + 1) - u0;
    if (!fits(n, DownRole<I, W>::capacity())) return;
    rd.init(n, reinterpret_cast<float4 *>(region));
    auto row = [&](int l) {
      const W *base = reinterpret_cast<const W *>(layer(l).wd);
      return [=](int k) { return base + static_cast<size_t>(u0 + k) * I; };
    };
    auto pre_lds = [&](int l, int) { rd.prefetch_lds(row(l)); };
    auto pre_regs = [&](int l) { rd.prefetch_regs(row(l)); };
    // This CU's output segment: float4s [seg4, seg4 + 4) of the layer
    // output, rows u0 + k at element k, padded with zeros; thread q < pub4
    // publishes float4 q.
    static_assert(DownRole<I, W>::kMaxRows <= kHidSegment, "a down CU's rows fit its segment");
    const int seg4 = (kHidSegment / 4) * rank, pub4 = (n + 3) / 4;
    const bool pub = static_cast<int>(threadIdx.x) < pub4;
    const int hb4 = u0 / 4;                       // float4s of h1 covering [u0, u0 + n)
    const int hn4 = (u0 + n + 3) / 4 - hb4;
    // Per-lane slice sums [row][wave][lane], after this CU's LDS rows.
    float *part = reinterpret_cast<float *>(region) + DownRole<I, W>::lds_rows(n) * kWave * 4;
    float *stage = cm.top;  // row u0 + k at stage[k]
    loop(kRoleDown, true, [&](uint32_t t, int l, int position) {
      const Slots out = s_hid(l, t);
      if (pub) s_hid(l, t + 1).clear4(seg4 + threadIdx.x);
      rd.settle();
      if (!gather_h1(t, l, hb4, hn4, cm.vec)) return false;
      // This wave's slice of the activation, straight into registers.
      float4 xa[DownRole<I, W>::kNsHi];
      bool ok = true;
      {
        const Slots src = s_act(l, t);
        uint32_t pending = (1u << rd.ns) - 1u;
        for (uint32_t spin = 0; ok; ++spin) {
          Quad got[DownRole<I, W>::kNsHi];
#pragma unroll
          for (int s = 0; s < DownRole<I, W>::kNsHi; ++s)
            if ((pending >> s) & 1u) got[s] = __builtin_bit_cast(Quad, src.get4((rd.c0 + s) * kWave + lane));
#pragma unroll
          for (int s = 0; s < DownRole<I, W>::kNsHi; ++s) {
            const Quad &g = got[s];
            if (((pending >> s) & 1u) && g.w[0] != kSlotEmpty && g.w[1] != kSlotEmpty &&
                g.w[2] != kSlotEmpty && g.w[3] != kSlotEmpty) {
              xa[s] = make_float4(__uint_as_float(g.w[0]), __uint_as_float(g.w[1]), __uint_as_float(g.w[2]),
                                  __uint_as_float(g.w[3]));
              pending &= ~(1u << s);
            }
          }
          vm_wait();
          if (__builtin_amdgcn_ballot_w64(pending != 0) == 0) break;
          if (spin > a.spin_limit) {
            if (lane == 0) atomicOr(a.error, kResidentWaitGaveUp);
            ok = false;
          }
        }
      }
      clock.lap(2 * kRoleDown);
      clock.mark(0);
      if (ok) rd.sums(xa, part);
      clock.mark(1);
      if (!block_all(ok, flag_set())) return false;
      // Wave w finishes rows w and w + kW (at most kMaxRows = 2 kW rows): the
      // slice sums of both rows are read at once and reduced together
      // (wave_sum_multi: row w's sum in lane 0, row w + kW's in lane 1).
      static_assert(DownRole<I, W>::kMaxRows <= 2 * kW, "two rows per wave");
      if (wv < n) {
        const int k1 = min(wv + kW, n - 1);
        float p0[kRowSlices], p1[kRowSlices];
#pragma unroll
        for (int w = 0; w < kRowSlices; ++w) {
          p0[w] = part[(wv * kW + w) * kWave + lane];
          p1[w] = part[(k1 * kW + w) * kWave + lane];
        }
        const float two[2] = {combine_slices(p0), combine_slices(p1)};
        const float sum = wave_sum_multi<2>(two);
        const int k = wv + kW * lane;
        if (lane < 2 && k < n) stage[k] = cm.vec[u0 + k - 4 * hb4] + sum;
      }
      if (static_cast<int>(threadIdx.x) >= n && static_cast<int>(threadIdx.x) < 4 * pub4) stage[threadIdx.x] = 0.f;
      lds_barrier();
      if (pub) out.put4(seg4 + threadIdx.x, reinterpret_cast<const float4 *>(stage)[threadIdx.x]);
      clock.mark(2);
      lds_barrier();
      clock.lap(2 * kRoleDown + 1);
      if (l + 1 < a.layers) {  // layer 0 of the next token follows the LM head
        pre_lds(l + 1, position);
        pre_regs(l + 1);
      }
      return true;
    }, pre_lds, pre_regs);
  }
};

// Each role's loop is its own (non-inlined) function so the register
// allocator sizes each role separately instead of one body holding all five.
// kRoleAttnLong / kRoleAttnShort: the attention role of a launch whose
// chunks all exceed one block / all fit one (ResidentArgs::attn_mode).
constexpr int kRoleAttnLong = kRoleCount, kRoleAttnShort = kRoleCount + 1;
template <int H, int I, int NQ, int NKV, bool kProfile, typename W, int kRole>
__device__ __attribute__((noinline)) void run_role(const void *kernarg, int rank, int nrole, int wg) {
  // The launch arguments, copied with scalar loads from the kernel's
  // argument segment (whose address the kernel passes: a callee has no
  // kernarg segment pointer of its own, and the address of the kernel's
  // by-value parameter would name a private stack copy) into a local the
  // compiler keeps in SGPRs.
  ResidentArgs a;
  {
    typedef const __attribute__((address_space(4))) uint32_t kword;
    // readfirstlane returns a signed int: each half is taken as uint32_t
    // before widening, or bit 31 of the low half would sign-extend into the
    // high half and the address would be non-canonical.
    const uint64_t addr = reinterpret_cast<uint64_t>(kernarg);
    const uint64_t lo =
        static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr)));
    const uint64_t hi =
        static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(addr >> 32)));
    kword *src = (kword *)((hi << 32) | lo);
    uint32_t *dst = reinterpret_cast<uint32_t *>(&a);
#pragma unroll
    for (size_t i = 0; i < sizeof(ResidentArgs) / 4; ++i) dst[i] = src[i];
  }
  Roles<H, I, NQ, NKV, kProfile, W> r(a, roles_lds, __builtin_amdgcn_readfirstlane(rank),
                                   __builtin_amdgcn_readfirstlane(nrole),
                                   __builtin_amdgcn_readfirstlane(wg));
  if constexpr (kRole == kRoleQkv) r.run_qkv();
  if constexpr (kRole == kRoleAttn) r.template run_attn<0>();
  if constexpr (kRole == kRoleAttnLong) r.template run_attn<1>();
  if constexpr (kRole == kRoleAttnShort) r.template run_attn<2>();
  if constexpr (kRole == kRoleO) r.run_o();
  if constexpr (kRole == kRoleGate) r.run_gate();
  if constexpr (kRole == kRoleDown) r.run_down();
}

// Placement position of workgroup b. With xcd_place, XCD x < nkv holds KV
// group x's QKV, attention and O CUs as its first G = sum(group_cus)
// workgroups (b / kXcds < G), in that order; the other workgroups take the
// gate/up and down positions in workgroup order.
__device__ __forceinline__ int placement(const ResidentArgs &a, int b) {
  if (!a.xcd_place) return b;
  const int n0 = a.group_cus[0], n1 = a.group_cus[1], n2 = a.group_cus[2];
  const int G = n0 + n1 + n2;
  const int x = b % kXcds, i = b / kXcds;
  if (x < a.nkv && i < G) {
    if (i < n0) return x * n0 + i;
    if (i < n0 + n1) return a.nkv * n0 + x * n1 + (i - n0);
    return a.nkv * (n0 + n1) + x * n2 + (i - n0 - n1);
  }
  int before = 0;  // group workgroups with a lower index
  for (int xx = 0; xx < a.nkv; ++xx) before += min(G, b > xx ? (b - xx + kXcds - 1) / kXcds : 0);
  return a.nkv * G + (b - before);
}

__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xFu;
}

template <int H, int I, int NQ, int NKV, bool kProfile, typename W>
__global__ __launch_bounds__(kT, 1) void roles_kernel(ResidentArgs a) {
  const void *kernarg = (const void *)__builtin_amdgcn_kernarg_segment_ptr();
  // With XCD placement a workgroup's position is i * kXcds + x, x the XCD it
  // runs on and i its arrival order there (a ticket from a.error[1 + x]),
  // whatever XCD the dispatcher started the launch from. An XCD dealt more
  // than grid / kXcds workgroups stops the extra ones (their waiting peers
  // give up): the intra-XCD hand-offs rely on the placement.
  int wg = blockIdx.x;
  if (a.xcd_place) {
    uint32_t *ticket = reinterpret_cast<uint32_t *>(roles_lds);
    const uint32_t x = xcc_id();
    if (threadIdx.x == 0) *ticket = x < kXcds ? atomicAdd(a.error + 1 + x, 1u) : ~0u;
    __syncthreads();
    const uint32_t i = *ticket;
    __syncthreads();  // every wave has read the ticket before the LDS is reused
    if (i >= gridDim.x / kXcds) {
      if (threadIdx.x == 0) atomicOr(a.error, kResidentPlacement);
      return;
    }
    wg = static_cast<int>(i * kXcds + x);
  }
  const int b = placement(a, wg);
  int role = 0;
  while (role < kRoleCount - 1 && b >= a.role_end[role]) ++role;
  const int rbeg = role ? a.role_end[role - 1] : 0;
  const int rank = b - rbeg, nrole = a.role_end[role] - rbeg;
  switch (role) {
    case kRoleQkv:
      run_role<H, I, NQ, NKV, kProfile, W, kRoleQkv>(kernarg, rank, nrole, wg);
      break;
    case kRoleAttn:
      if (a.attn_mode == 1)
        run_role<H, I, NQ, NKV, kProfile, W, kRoleAttnLong>(kernarg, rank, nrole, wg);
      else if (a.attn_mode == 2)
        run_role<H, I, NQ, NKV, kProfile, W, kRoleAttnShort>(kernarg, rank, nrole, wg);
      else
        run_role<H, I, NQ, NKV, kProfile, W, kRoleAttn>(kernarg, rank, nrole, wg);
      break;
    case kRoleO:
      run_role<H, I, NQ, NKV, kProfile, W, kRoleO>(kernarg, rank, nrole, wg);
      break;
    case kRoleGate:
      run_role<H, I, NQ, NKV, kProfile, W, kRoleGate>(kernarg, rank, nrole, wg);
      break;
    default:
      run_role<H, I, NQ, NKV, kProfile, W, kRoleDown>(kernarg, rank, nrole, wg);
      break;
  }
}

using Qwen = Shape<896, 4864, 14, 2>;
// The kernel instance for the decoder matrices' storage (kWeights*).
template <typename W>
const void *roles_fn_as(bool profile) {
  return profile ? reinterpret_cast<const void *>(&roles_kernel<896, 4864, 14, 2, true, W>)
                 : reinterpret_cast<const void *>(&roles_kernel<896, 4864, 14, 2, false, W>);
}
const void *roles_fn(bool profile, int weights_dtype) {
  switch (weights_dtype) {
    case kWeightsBf16: return roles_fn_as<Bf16>(profile);
    case kWeightsF16: return roles_fn_as<F16>(profile);
    default: return roles_fn_as<float>(profile);
  }
}

// What a resident launch expects at its start, in one dispatch: the error
// word and the XCD tickets zero, and parity 0's block of every layer's
// hand-off slots empty (token 0's). Parity 1's blocks need no clearing:
// token 0's writers clear their slots there before any CU starts token 1.
// With `top`, the argmax tag arena is zeroed too.
__global__ __launch_bounds__(256) void roles_prepare_kernel(uint32_t *error, uint4 *slots,
                                                            uint32_t block_u4, uint2 *top,
                                                            uint32_t top_pairs) {
  const uint32_t t = threadIdx.x + blockIdx.x * blockDim.x, n = gridDim.x * blockDim.x;
  if (blockIdx.y == 0) {
    if (t < 1 + kXcds) error[t] = 0u;
    for (uint32_t i = t; i < top_pairs; i += n) top[i] = make_uint2(0u, 0u);
  }
  uint4 *blk = slots + size_t(blockIdx.y) * 2 * block_u4;
  for (uint32_t i = t; i < block_u4; i += n) blk[i] = make_uint4(kSlotEmpty, kSlotEmpty, kSlotEmpty, kSlotEmpty);
}

}  // namespace

bool plan_roles(int grid, int hidden, int inter, int heads, int kv_heads, int max_length,
                RolePlan *plan) {
  if (hidden != 896 || inter != 4864 || heads != 14 || kv_heads != 2) return false;
  if (grid > kMaxRoleGrid || max_length < 1) return false;
  // Units per role, their capacity per CU (LDS + register slots) and bytes.
  // O: each of the KV groups covers every row pair (Roles::run_o).
  const int units[4] = {Qwen::QkvUnits, kv_heads * Qwen::OUnits, inter, hidden};
  const int cap[4] = {Qwen::LQ + kW * kSlotsQ, Qwen::LO + kW * kSlotsO, Qwen::LG + kW * kSlotsG,
                      DownRole<4864, float>::capacity()};
  const double bytes[4] = {double(units[0]) * Qwen::UnitBytes, double(units[1]) * Qwen::OUnitBytes,
                           double(units[2]) * Qwen::UnitBytes, double(units[3]) * Qwen::RowBytes};
  const double total = bytes[0] + bytes[1] + bytes[2] + bytes[3];
  // CUs a role needs to hold its units: the gate role splits whole float4s
  // of the activation (4 units), the others single units.
  // QKV and O work in KV groups (Roles::run_qkv, run_o): each group's CUs
  // hold the group's share.
  auto need_of = [&](int r) {
    if (r == 0) return kv_heads * ((units[0] / kv_heads + cap[0] - 1) / cap[0]);
    if (r == 1) return kv_heads * ((Qwen::OUnits + cap[1] - 1) / cap[1]);
    const int g = r == 2 ? 4 : 1;
    return ((units[r] + g - 1) / g + cap[r] / g - 1) / (cap[r] / g);
  };
  int floor_weights = 0;
  for (int r = 0; r < 4; ++r) floor_weights += need_of(r);
  // One attention CU per (KV head, chunk) unit of the longest context, or
  // as many as the weight roles leave (an attention CU then takes several
  // units, the later ones staged after its query arrives). A long context
  // gets a chunk per window of kAttnCap positions (up to kAttnMaxChunks),
  // so each chunk's tiles run as one round on the CU's waves.
  const int chunks = std::max(attn_chunks(max_length),
                              std::min(kAttnMaxChunks, (max_length + kAttnCap - 1) / kAttnCap));
  int n_attn = std::min(kv_heads * chunks, grid - floor_weights);
  n_attn -= n_attn % kv_heads;  // whole KV groups
  if (n_attn < kv_heads) return false;
  const int rest = grid - n_attn;
  int n[4], used = 0;
  for (int r = 0; r < 4; ++r) {
    const int need = need_of(r);
    n[r] = std::max(need, static_cast<int>(rest * bytes[r] / total));
    n[r] = std::min(n[r], units[r]);
    used += n[r];
  }
  if (rest <= 0) return false;
  // Hand out or take back the remainder by the largest per-CU share.
  while (used != rest) {
    int pick = -1;
    double best = used < rest ? -1.0 : 1e30;
    for (int r = 0; r < 4; ++r) {
      const double share = bytes[r] / n[r];
      const int need = need_of(r);
      if (used < rest && n[r] < units[r] && share > best) {
        best = share;
        pick = r;
      }
      if (used > rest && n[r] > need && bytes[r] / (n[r] - 1) < best) {
        best = bytes[r] / (n[r] - 1);
        pick = r;
      }
    }
    if (pick < 0) return false;
    n[pick] += used < rest ? 1 : -1;
    used += used < rest ? 1 : -1;
  }
  // QKV and O in whole KV groups; the gate role gives or takes the rest.
  for (int r = 0; r < 2; ++r) {
    const int d = (kv_heads - n[r] % kv_heads) % kv_heads;
    if (d == 0) continue;
    if (n[2] - d >= need_of(2)) {
      n[r] += d;
      n[2] -= d;
    } else if (n[r] - (kv_heads - d) >= need_of(r)) {
      n[r] -= kv_heads - d;
      n[2] += kv_heads - d;
    } else {
      return false;
    }
  }
  plan->group_cus[0] = n[0] / kv_heads;
  plan->group_cus[1] = n_attn / kv_heads;
  plan->group_cus[2] = n[1] / kv_heads;
  plan->xcd_place = grid % kXcds == 0 && kv_heads <= kXcds &&
                    plan->group_cus[0] + plan->group_cus[1] + plan->group_cus[2] <= grid / kXcds;
  plan->end[kRoleQkv] = n[0];
  plan->end[kRoleAttn] = n[0] + n_attn;
  plan->end[kRoleO] = plan->end[kRoleAttn] + n[1];
  plan->end[kRoleGate] = plan->end[kRoleO] + n[2];
  plan->end[kRoleDown] = plan->end[kRoleGate] + n[3];
  // The layer output's segments are gathered with at most two float4s per
  // thread (Roles::kHidMaxPer).
  if (4 * n[3] > 2 * kT) return false;
  return plan->end[kRoleDown] == grid;
}

hipError_t launch_roles(hipStream_t s, const ResidentArgs &args, int grid) {
  void *params[] = {const_cast<ResidentArgs *>(&args)};
  if (args.weights_dtype != kWeightsF32 && args.weights_dtype != kWeightsBf16 &&
      args.weights_dtype != kWeightsF16)
    return hipErrorInvalidValue;
  return hipLaunchCooperativeKernel(roles_fn(args.stage_ticks || args.trace, args.weights_dtype), dim3(grid), dim3(kT),
                                    params, 0, s);
}

hipError_t launch_roles_prepare(hipStream_t s, uint32_t *error, float *slots, size_t slot_floats,
                               int layers, void *top, int top_pairs) {
  if (slot_floats % 4 != 0 || reinterpret_cast<uintptr_t>(slots) % 16 != 0 || layers < 1 ||
      layers > 65535)
    return hipErrorInvalidValue;
  const uint32_t block_u4 = static_cast<uint32_t>(slot_floats / 4);
  const dim3 grid((block_u4 + 4 * 256 - 1) / (4 * 256), static_cast<uint32_t>(layers));
  hipLaunchKernelGGL(roles_prepare_kernel, grid, dim3(256), 0, s, error,
                     reinterpret_cast<uint4 *>(slots), block_u4, static_cast<uint2 *>(top),
                     top ? static_cast<uint32_t>(top_pairs) : 0u);
  return hipGetLastError();
}

int device_cu_count(int device) {
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return 0;
  return cus;
}

int roles_max_grid(int device, int weights_dtype) {
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return 0;
  // Every instance of the storage type must fit (the profiled one included).
  int lo = 1 << 30;
  for (bool profile : {false, true}) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, roles_fn(profile, weights_dtype), kT, 0) !=
        hipSuccess)
      return 0;
    lo = std::min(lo, per_cu);
  }
  return cus * lo;
}

}  // namespace qd
