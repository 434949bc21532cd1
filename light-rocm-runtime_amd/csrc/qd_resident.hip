// Resident decode megakernel: one cooperative launch runs every token of a
// greedy generation -- all decoder layers, the LM head, the argmax and the
// embedding feedback. It is the MI355X counterpart of the reference's
// persistent-graph resident loop (include/lrrt/persistent_graph/
// compiled_scheduler.hpp:108-217 driving benchmarks/
// qwen_stateful_graph_kernel.cpp:661-1083), built around what the hardware
// measures: a grid barrier on 256 CUs costs ~1.5 us and every dependent
// device-scope memory round trip ~1 us, so the kernel has no barriers at
// all. It is a dataflow graph over tagged vectors:
//
//   every value one workgroup hands to another is stored as an 8-byte
//   (value, tag) pair with a device-scope (sc1) store; the tag names the
//   launch epoch and the (token, layer, stage) that produced it. A consumer
//   polls the pairs it needs until every tag matches, then proceeds. A
//   producer never waits for its stores to complete, and a consumer issues
//   its next weight loads before it starts polling, so HBM streaming
//   overlaps the hand-off latency.
//
// Stage map per layer (whole output rows per wave, rows spread over every
// wave of the grid):
//   A  attention RMSNorm + packed QKV + bias + RoPE -> q, new K/V (+ cache)
//   B  split-KV GQA attention per (query head, chunk); the unit of a head's
//      last chunk merges the head's partials -> attn
//   C  O projection + residual -> h1
//   D  MLP RMSNorm + gate/up + SiLU -> act      (every workgroup takes part)
//   E  down projection + residual -> hidden
// Tail: final RMSNorm + LM head + per-workgroup top-1 -> every workgroup
// reduces the partials to the sampled token and feeds it back.
//
// Reuse safety: a tagged buffer is rewritten only after stage D of a later
// layer, and every workgroup finishes reading the previous version before
// its own stage D, which every later producer transitively waits for.
#include <hip/hip_runtime.h>

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

constexpr uint32_t kSpinLimit = 1u << 21;  // polls before a wait gives up

struct Pair2 {
  float v0;
  uint32_t t0;
  float v1;
  uint32_t t1;
};
typedef unsigned int u32x2 __attribute__((vector_size(8)));

// Vector of (value, tag) elements with device-scope access.
struct TagVec {
  __amdgpu_buffer_rsrc_t r;
  __device__ TagVec(void *base, uint32_t elems)
      : r(__builtin_amdgcn_make_buffer_rsrc(base, 0, static_cast<int>(elems * 8u),
                                            kRsrcWord3)) {}
  __device__ void put(uint32_t i, float v, uint32_t tag) const {
    const u32x2 x = {__builtin_bit_cast(unsigned, v), tag};
    __builtin_amdgcn_raw_buffer_store_b64(x, r, i * 8u, 0, kPolicySc1);
  }
  __device__ Pair2 get2(uint32_t pair) const {
    return __builtin_bit_cast(
        Pair2, __builtin_amdgcn_raw_buffer_load_b128(r, pair * 16u, 0, kPolicySc1));
  }
};

struct Lds {
  const float *p;
  __device__ float ld(uint32_t i) const { return p[i]; }
  __device__ float4 ld4(uint32_t i4) const { return reinterpret_cast<const float4 *>(p)[i4]; }
};

// One head's K or V row staged in LDS, addressed like a full cache row
// (float4 index i4 of [kv_heads*64]) for head `head`.
struct LdsHeadRow {
  const float *p;
  int head;
  __device__ float4 ld4(uint32_t i4) const {
    return reinterpret_cast<const float4 *>(p)[i4 - head * (kHeadDim / 4)];
  }
};

// This thread's float4 of an RMSNorm gain vector (threads past N/4 get 0),
// loaded ahead of the activation it scales.
template <int N>
__device__ __forceinline__ float4 load_gain4(const float *gain) {
  return threadIdx.x < N / 4 ? reinterpret_cast<const float4 *>(gain)[threadIdx.x]
                             : make_float4(0.f, 0.f, 0.f, 0.f);
}

// "Row pairs over all waves" loop with a 4-deep weight pipeline: while a
// unit is reduced, the wave's next three units are already loading; the
// operand x (K floats in LDS) is held in registers in the slot layout. rows(u, a, b) gives unit u's two
// row pointers; epi(u, sa, sb) consumes the sums (every lane holds them).
// w0 must hold the weights of unit `first` when first < units.
template <int K, typename Rows, typename Epi>
__device__ __forceinline__ void run_pairs(int first, int stride, int units, const float *x,
                                          float4 (&w0)[PairSlots<K>::NJ], Rows rows,
                                          Epi epi) {
  constexpr int NJ = PairSlots<K>::NJ;
  if (first >= units) return;
  float4 xv[NJ];
  load_pair_operand<K>(Lds{x}, xv);
  float4 w1[NJ], w2[NJ], w3[NJ];
  auto load = [&](int u, float4 (&w)[NJ]) {
    if (u < units) {
      const float *ra, *rb;
      rows(u, ra, rb);
      load_pair_weights<K>(ra, rb, w);
    }
  };
  auto step = [&](int u, const float4 (&w)[NJ]) {
    float sa, sb;
    pair_dot<K>(w, xv, sa, sb);
    epi(u, sa, sb);
  };
  load(first + stride, w1);
  load(first + 2 * stride, w2);
  for (int u = first; u < units; u += 4 * stride) {
    load(u + 3 * stride, w3);
    step(u, w0);
    if (u + stride >= units) break;
    load(u + 4 * stride, w0);
    step(u + stride, w1);
    if (u + 2 * stride >= units) break;
    load(u + 5 * stride, w1);
    step(u + 2 * stride, w2);
    if (u + 3 * stride >= units) break;
    load(u + 6 * stride, w2);
    step(u + 3 * stride, w3);
  }
}

// Profiling clock (profiled kernel variant only), kept by thread 0 of each
// workgroup in LDS: per-stage totals (published for workgroup 0), and
// optionally a timeline of every workgroup for one token
// (row[layer * kResidentStages + stage] = time the stage ended; the tail
// stages use layer = layers).
template <bool kProfile>
struct StageClock {
  uint64_t *ticks = nullptr;  // LDS [kResidentStages]
  uint64_t prev = 0;
  uint64_t *row = nullptr;
  bool tracing = false;
  int layer = 0;
  __device__ void start(uint64_t *lds_ticks, uint64_t *trace, int layers) {
    if (kProfile && threadIdx.x == 0) {
      ticks = lds_ticks;
      for (int s = 0; s < kResidentStages; ++s) ticks[s] = 0;
      prev = wall_clock64();
      if (trace) row = trace + static_cast<size_t>(blockIdx.x) * (layers + 1) * kResidentStages;
    }
  }
  __device__ void lap(int stage) {
    if (kProfile && threadIdx.x == 0) {
      const uint64_t now = wall_clock64();
      ticks[stage] += now - prev;
      prev = now;
      if (tracing) row[layer * kResidentStages + stage] = now;
    }
  }
  __device__ void at(uint32_t token, uint32_t trace_token, int l) {
    if (kProfile) {
      tracing = row != nullptr && token == trace_token;
      layer = l;
    }
  }
  __device__ void publish(uint64_t *out) const {
    if (kProfile && out && blockIdx.x == 0 && threadIdx.x == 0)
      for (int s = 0; s < kResidentStages; ++s) out[s] = ticks[s];
  }
};

struct Shared {
  float xs[4864];                              // staged activation vector
  float hs[1024];                              // residual vector
  float hid[1024];                             // the layer's input hidden vector
  float xn[1024];                              // RMSNorm output (GEMV operand)
  float parts[kAttnMaxChunks * kPartStride];   // a head's partials at its owner unit
  AttnLds attn;
  float red[kWavesPerBlock];
  float bv[kWavesPerBlock];
  uint32_t bi[kWavesPerBlock];
  float top[2 * kMaxResidentGrid];
  uint64_t ticks[kResidentStages];             // profiling totals (thread 0)
};

// Whole-workgroup gather: waits until elements [first, first + n) of src
// (n even, first even) all carry `tag` and copies their values to dst[0..n).
// ahead() runs first: the stage's weight prefetch, which then streams while
// the inputs are awaited. Returns false when the wait gave up (error word
// raised).
template <int kMaxPer, typename Ahead>
__device__ bool gather(const TagVec &src, uint32_t first, int n, uint32_t tag, float *dst,
                       uint32_t *error, Ahead ahead) {
  const int pairs = n / 2;
  const int t = threadIdx.x;
  uint32_t pending = 0;
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k)
    if (t + k * kBlock < pairs) pending |= 1u << k;
  ahead();
  __builtin_amdgcn_sched_barrier(0);
  for (uint32_t spin = 0;; ++spin) {
    Pair2 got[kMaxPer];
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k)
      if ((pending >> k) & 1u) got[k] = src.get2(first / 2 + t + k * kBlock);
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
      if (((pending >> k) & 1u) && got[k].t0 == tag && got[k].t1 == tag) {
        const int p = t + k * kBlock;
        dst[2 * p] = got[k].v0;
        dst[2 * p + 1] = got[k].v1;
        pending &= ~(1u << k);
      }
    }
    if (__syncthreads_and(pending == 0)) return true;
    if (spin > kSpinLimit) {
      if (t == 0) atomicOr(error, 1u);
      return false;
    }
  }
}

template <int kMaxPer>
__device__ bool gather(const TagVec &src, uint32_t first, int n, uint32_t tag, float *dst,
                       uint32_t *error) {
  return gather<kMaxPer>(src, first, n, tag, dst, error, [] {});
}

template <int H, int I, int QD, bool kProfile>
__global__ __launch_bounds__(kBlock, 1) void resident_decode_kernel(ResidentArgs a) {
  static_assert(I <= 4864 && H <= 1024, "LDS staging sizes");
  __shared__ Shared sh;
  const int kv_dim = a.nkv * kHeadDim;
  const int group = a.nq / a.nkv;
  const int gw = blockIdx.x * kWavesPerBlock + wave_id();
  const int nwaves = gridDim.x * kWavesPerBlock;
  const int lane = lane_id();
  const int wgw = static_cast<int>(blockIdx.x) * kWavesPerBlock;  // first wave of the WG
  const uint32_t per_token = 6u * a.layers + 1u;
  // Per query head h: its query, then this step's K and V rows of its KV
  // head (repeated for every head of the group).
  constexpr int qkv_block = 3 * kHeadDim;
  const TagVec tqkv(a.qkv, a.nq * qkv_block);
  const TagVec tpart(a.part, kAttnMaxChunks * a.nq * kPartStride);
  const TagVec tattn(a.attn, QD);
  const TagVec th1(a.h1, H);
  const TagVec tact(a.act, I);
  const TagVec thid(a.hidden, H);
  const TagVec ttop(a.top, 2 * gridDim.x);
  auto tag = [&](uint32_t seq) { return a.epoch | (seq + 1u); };
  // The layer's input hidden vector into sh.hid (embedding row at layer 0),
  // with the caller's prefetch queued behind the first poll.
  auto fetch_hidden = [&](int l, uint32_t tag_prev, const float *embed_row, auto ahead) {
    if (l == 0) {
      ahead();
      for (int c = threadIdx.x; c < H; c += kBlock) sh.hid[c] = embed_row[c];
      __syncthreads();
      return true;
    }
    return gather<(H / 2 + kBlock - 1) / kBlock>(thid, 0, H, tag_prev, sh.hid, a.error, ahead);
  };

  uint32_t token = a.first_token;
  uint32_t generated = 0;
  uint32_t stop_reason = 0;
  float top = 0.f;
  StageClock<kProfile> clock;
  clock.start(sh.ticks, a.trace, a.layers);

  for (uint32_t t = 0; t < a.max_tokens; ++t) {
    const int position = static_cast<int>(a.start_position + t);
    if (token >= static_cast<uint32_t>(a.vocab) || position >= a.capacity) break;
    const int length = position + 1;
    const int chunk_len = attn_chunk_len(length);
    const int chunks = attn_chunks(length);
    const float *embed_row = a.embed + static_cast<size_t>(token) * H;
    const uint32_t s0 = t * per_token;

    for (int l = 0; l < a.layers; ++l) {
      clock.at(t, a.trace_token, l);
      const LayerPtrs w = a.layer_ptrs[l];
      float *kc = a.k_cache + static_cast<size_t>(l) * a.capacity * kv_dim;
      float *vc = a.v_cache + static_cast<size_t>(l) * a.capacity * kv_dim;
      const uint32_t tag_q = tag(s0 + 6 * l + 0);
      const uint32_t tag_p = tag(s0 + 6 * l + 1);
      const uint32_t tag_m = tag(s0 + 6 * l + 2);
      const uint32_t tag_h1 = tag(s0 + 6 * l + 3);
      const uint32_t tag_act = tag(s0 + 6 * l + 4);
      const uint32_t tag_hid = tag(s0 + 6 * l + 5);
      const uint32_t tag_prev = l ? tag(s0 + 6 * (l - 1) + 5) : 0u;
      bool have_hidden = false;

      // ---- A: RMSNorm + QKV + bias + RoPE ------------------------------------
      {
        const int units = (a.nq + 2 * a.nkv) * kRotary;
        if (wgw < units) {
          auto rows = [&](int u, const float *&ra, const float *&rb) {
            const int row = (u / kRotary) * kHeadDim + u % kRotary;
            ra = w.wqkv + static_cast<size_t>(row) * H;
            rb = ra + static_cast<size_t>(kRotary) * H;
          };
          // Unit constants (bias pair, rotation) fetched with the weights.
          auto consts = [&](int u, float4 &cv) {
            const int head = u / kRotary, i = u % kRotary;
            const int ra = head * kHeadDim + i;
            cv.x = w.bqkv[ra];
            cv.y = w.bqkv[ra + kRotary];
            const bool rot = head < a.nq + a.nkv;
            cv.z = rot ? a.rope_cos[position * kRotary + i] : 1.f;
            cv.w = rot ? a.rope_sin[position * kRotary + i] : 0.f;
          };
          float4 w0[PairSlots<H>::NJ];
          float4 c0 = make_float4(0.f, 0.f, 1.f, 0.f);
          float4 g;
          if (!fetch_hidden(l, tag_prev, embed_row, [&] {
                if (gw < units) {
                  const float *ra, *rb;
                  rows(gw, ra, rb);
                  load_pair_weights<H>(ra, rb, w0);
                  consts(gw, c0);
                }
                g = load_gain4<H>(w.attn_norm);
              }))
            return;
          have_hidden = true;
          clock.lap(0);
          const float inv = block_inv_rms<H>(Lds{sh.hid}, a.eps, sh.red);
          norm_to_lds<H>(sh.hid, inv, g, sh.xn);
          __syncthreads();
          {
            const Coherent kcache(kc, static_cast<uint32_t>(a.capacity) * kv_dim * 4u);
            const Coherent vcache(vc, static_cast<uint32_t>(a.capacity) * kv_dim * 4u);
            run_pairs<H>(gw, nwaves, units, sh.xn, w0, rows, [&](int u, float sa, float sb) {
              if (lane != 0) return;
              float4 cv = c0;
              if (u != gw) consts(u, cv);
              const int head = u / kRotary, i = u % kRotary;
              const float x0 = sa + cv.x;
              const float x1 = sb + cv.y;
              if (head < a.nq + a.nkv) {
                const float first = x0 * cv.z - x1 * cv.w;
                const float second = x1 * cv.z + x0 * cv.w;
                if (head < a.nq) {
                  tqkv.put(head * qkv_block + i, first, tag_q);
                  tqkv.put(head * qkv_block + i + kRotary, second, tag_q);
                } else {
                  const int kvh = head - a.nq;
                  const int o = kvh * kHeadDim + i;
                  for (int h = kvh * group; h < (kvh + 1) * group; ++h) {
                    tqkv.put(h * qkv_block + kHeadDim + i, first, tag_q);
                    tqkv.put(h * qkv_block + kHeadDim + i + kRotary, second, tag_q);
                  }
                  kcache.st(position * kv_dim + o, first);
                  kcache.st(position * kv_dim + o + kRotary, second);
                }
              } else {
                const int kvh = head - a.nq - a.nkv;
                const int o = kvh * kHeadDim + i;
                for (int h = kvh * group; h < (kvh + 1) * group; ++h) {
                  tqkv.put(h * qkv_block + 2 * kHeadDim + i, x0, tag_q);
                  tqkv.put(h * qkv_block + 2 * kHeadDim + i + kRotary, x1, tag_q);
                }
                vcache.st(position * kv_dim + o, x0);
                vcache.st(position * kv_dim + o + kRotary, x1);
              }
            });
          }
        }
      }
      clock.lap(1);

      // ---- B: split-KV attention, one (query head, chunk) per unit -----------
      {
        const int units = a.nq * chunks;
        const Coherent kcache(kc, static_cast<uint32_t>(a.capacity) * kv_dim * 4u);
        const Coherent vcache(vc, static_cast<uint32_t>(a.capacity) * kv_dim * 4u);
        for (int u = blockIdx.x; u < units; u += gridDim.x) {
          const int h = u / chunks, chunk = u % chunks;
          const int g = h / group;
          const int begin = chunk * chunk_len;
          const int end = min(length, begin + chunk_len);
          const bool has_new = position >= begin && position < end;
          bool ok = true;
          // The unit holding this step's position also takes its K/V row,
          // which follows the query in the same tagged block.
          const LdsHeadRow knew{sh.attn.qkv + kHeadDim, g};
          const LdsHeadRow vnew{sh.attn.qkv + 2 * kHeadDim, g};
          attn_partial_unit<kWavesPerBlock>(
              kcache, vcache, knew, vnew, has_new ? position : -1, g, kv_dim, begin, end,
              sh.attn,
              [&](auto request_rows) {
                ok = gather<1>(tqkv, h * qkv_block, has_new ? qkv_block : kHeadDim, tag_q,
                               sh.attn.qkv, a.error, request_rows);
                clock.lap(2);
              },
              [&](float m, float lsum, float acc, int d) {
                if (has_new) {
                  // The owner keeps its own record in LDS for the merge.
                  float *rec = sh.parts + chunk * kPartStride;
                  rec[2 + d] = acc;
                  if (d == 0) {
                    rec[0] = m;
                    rec[1] = lsum;
                  }
                } else {
                  const uint32_t rec = (h * kAttnMaxChunks + chunk) * kPartStride;
                  tpart.put(rec + 2 + d, acc, tag_p);
                  if (d == 0) {
                    tpart.put(rec, m, tag_p);
                    tpart.put(rec + 1, lsum, tag_p);
                  }
                }
              },
              [&](int phase) {
                if (phase < 3) clock.lap(kResidentStages - 3 + phase);
              });
          if (!ok) return;
          if (has_new) {
            // Owner of the head (its last chunk, which waits longest for this
            // step's K/V row): merge the other chunks' partials with its own.
            if (!gather<(kAttnMaxChunks * kPartStride / 2 + kBlock - 1) / kBlock>(
                    tpart, h * kAttnMaxChunks * kPartStride, chunk * kPartStride, tag_p, sh.parts,
                    a.error))
              return;
            if (threadIdx.x < kHeadDim) {
              const int d = threadIdx.x;
              tattn.put(h * kHeadDim + d,
                        attn_merge([&](int c, int k) { return sh.parts[c * kPartStride + k]; },
                                   chunks, d),
                        tag_m);
            }
          }
          __syncthreads();
        }
      }
      clock.lap(3);

      // ---- C: O projection + residual -----------------------------------------
      {
        constexpr int units = H / 2;
        if (wgw < units) {
          auto rows = [&](int u, const float *&ra, const float *&rb) {
            ra = w.wo + static_cast<size_t>(2 * u) * QD;
            rb = ra + QD;
          };
          float4 w0[PairSlots<QD>::NJ];
          if (!have_hidden && !fetch_hidden(l, tag_prev, embed_row, [] {})) return;
          if (!gather<(QD / 2 + kBlock - 1) / kBlock>(tattn, 0, QD, tag_m, sh.xs, a.error, [&] {
                if (gw < units) {
                  const float *ra, *rb;
                  rows(gw, ra, rb);
                  load_pair_weights<QD>(ra, rb, w0);
                }
              }))
            return;
          clock.lap(4);
          {
            run_pairs<QD>(gw, nwaves, units, sh.xs, w0, rows, [&](int u, float sa, float sb) {
              if (lane != 0) return;
              th1.put(2 * u, sh.hid[2 * u] + sa, tag_h1);
              th1.put(2 * u + 1, sh.hid[2 * u + 1] + sb, tag_h1);
            });
          }
        }
      }
      clock.lap(5);

      // ---- D: RMSNorm + gate/up + SiLU (every workgroup) ----------------------
      {
        auto rows = [&](int u, const float *&ra, const float *&rb) {
          ra = w.wg + static_cast<size_t>(u) * H;
          rb = w.wu + static_cast<size_t>(u) * H;
        };
        float4 w0[PairSlots<H>::NJ];
        float4 g;
        if (!gather<(H / 2 + kBlock - 1) / kBlock>(th1, 0, H, tag_h1, sh.hs, a.error, [&] {
              if (gw < I) {
                const float *ra, *rb;
                rows(gw, ra, rb);
                load_pair_weights<H>(ra, rb, w0);
              }
              g = load_gain4<H>(w.mlp_norm);
            }))
          return;
        clock.lap(6);
        const float inv = block_inv_rms<H>(Lds{sh.hs}, a.eps, sh.red);
        norm_to_lds<H>(sh.hs, inv, g, sh.xn);
        __syncthreads();
        {
          run_pairs<H>(gw, nwaves, I, sh.xn, w0, rows, [&](int u, float gt, float up) {
            if (lane == 0) tact.put(u, gt / (1.f + expf(-gt)) * up, tag_act);
          });
        }
      }
      clock.lap(7);

      // ---- E: down projection + residual --------------------------------------
      {
        if (wgw < H) {
          // A wave's first two rows are requested before the wait.
          float4 wrow[RowSlots<I>::NJ];
          if (!gather<(I / 2 + kBlock - 1) / kBlock>(tact, 0, I, tag_act, sh.xs, a.error, [&] {
                if (gw < H) load_row_weights<I>(w.wd + static_cast<size_t>(gw) * I, wrow);
              }))
            return;
          clock.lap(8);
          for (int r = gw; r < H; r += nwaves) {
            if (r != gw) load_row_weights<I>(w.wd + static_cast<size_t>(r) * I, wrow);
            const float s = row_dot_lds<I>(wrow, sh.xs);
            if (lane == 0) thid.put(r, sh.hs[r] + s, tag_hid);
          }
        }
      }
      clock.lap(9);
    }

    // ---- LM head + top-1 ---------------------------------------------------------
    clock.at(t, a.trace_token, a.layers);
    const uint32_t tag_last = tag(s0 + 6 * (a.layers - 1) + 5);
    const uint32_t tag_top = tag(s0 + 6 * a.layers);
    {
      const int units = (a.vocab + 1) / 2;
      auto rows = [&](int u, const float *&ra, const float *&rb) {
        ra = a.head + static_cast<size_t>(2 * u) * H;
        rb = 2 * u + 1 < a.vocab ? ra + H : ra;
      };
      float4 w0[PairSlots<H>::NJ];
      float4 g;
      if (!gather<(H / 2 + kBlock - 1) / kBlock>(thid, 0, H, tag_last, sh.xs, a.error, [&] {
            if (gw < units) {
              const float *ra, *rb;
              rows(gw, ra, rb);
              load_pair_weights<H>(ra, rb, w0);
            }
            g = load_gain4<H>(a.final_norm);
          }))
        return;
      clock.lap(10);
      const float inv = block_inv_rms<H>(Lds{sh.xs}, a.eps, sh.red);
      norm_to_lds<H>(sh.xs, inv, g, sh.xn);
      __syncthreads();
      float best = -INFINITY;
      uint32_t best_i = UINT32_MAX;
      {
        float *logits = a.logits + (a.history ? static_cast<size_t>(t) * a.vocab : 0);
        run_pairs<H>(gw, nwaves, units, sh.xn, w0, rows, [&](int u, float sa, float sb) {
          const int r0 = 2 * u;
          const bool has1 = r0 + 1 < a.vocab;
          if (lane == 0) {
            logits[r0] = sa;
            if (has1) logits[r0 + 1] = sb;
          }
          if (better(sa, r0, best, best_i)) {
            best = sa;
            best_i = r0;
          }
          if (has1 && better(sb, r0 + 1, best, best_i)) {
            best = sb;
            best_i = r0 + 1;
          }
        });
      }
      if (lane == 0) {
        sh.bv[wave_id()] = best;
        sh.bi[wave_id()] = best_i;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        for (int wv = 1; wv < kWavesPerBlock; ++wv) {
          if (better(sh.bv[wv], sh.bi[wv], best, best_i)) {
            best = sh.bv[wv];
            best_i = sh.bi[wv];
          }
        }
        ttop.put(2 * blockIdx.x, best, tag_top);
        ttop.put(2 * blockIdx.x + 1, __builtin_bit_cast(float, best_i), tag_top);
      }
    }
    clock.lap(11);

    // ---- argmax over the workgroup partials (every workgroup) ----------------
    {
      if (!gather<(kMaxResidentGrid + kBlock - 1) / kBlock>(ttop, 0, 2 * gridDim.x, tag_top,
                                                            sh.top, a.error))
        return;
      clock.lap(12);
      float best = -INFINITY;
      uint32_t best_i = UINT32_MAX;
      for (uint32_t p = threadIdx.x; p < gridDim.x; p += blockDim.x) {
        const float v = sh.top[2 * p];
        const uint32_t i = __builtin_bit_cast(uint32_t, sh.top[2 * p + 1]);
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
        sh.bv[wave_id()] = best;
        sh.bi[wave_id()] = best_i;
      }
      __syncthreads();
      best = sh.bv[0];
      best_i = sh.bi[0];
      for (int wv = 1; wv < kWavesPerBlock; ++wv) {
        if (better(sh.bv[wv], sh.bi[wv], best, best_i)) {
          best = sh.bv[wv];
          best_i = sh.bi[wv];
        }
      }
      __syncthreads();
      token = best_i;
      top = best;
    }
    clock.lap(13);
    generated = t + 1;
    if (blockIdx.x == 0 && threadIdx.x == 0) a.out_tokens[t] = token;
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
  clock.publish(a.stage_ticks);
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

}  // namespace

hipError_t launch_resident(hipStream_t s, const ResidentArgs &args, int grid) {
  void *params[] = {const_cast<ResidentArgs *>(&args)};
  const void *fn =
      (args.stage_ticks || args.trace)
          ? reinterpret_cast<const void *>(&resident_decode_kernel<896, 4864, 896, true>)
          : reinterpret_cast<const void *>(&resident_decode_kernel<896, 4864, 896, false>);
  return hipLaunchCooperativeKernel(fn, dim3(grid), dim3(kBlock), params, 0, s);
}

int resident_max_grid(int device) {
  int cus = 0, per_cu = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &per_cu, reinterpret_cast<const void *>(&resident_decode_kernel<896, 4864, 896, true>),
          kBlock, 0) != hipSuccess)
    return 0;
  return cus * per_cu;
}

int device_cu_count(int device) {
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    return 0;
  return cus;
}

}  // namespace qd
