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
//   B  split-KV GQA attention partials per (KV head, chunk)
//   C  merge of the partials + O projection + residual -> h1
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

// Waits until elements [first, first + n) of src (n even, first even) all
// carry `tag` and copies their values to dst[0..n). Whole workgroup; returns
// false when the wait gave up (error word raised).
template <int kMaxPer>
__device__ bool gather(const TagVec &src, uint32_t first, int n, uint32_t tag,
                       float *dst, uint32_t *error) {
  const int pairs = n / 2;
  const int t = threadIdx.x;
  uint32_t pending = 0;
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k)
    if (t + k * kBlock < pairs) pending |= 1u << k;
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

// Polls elements [first, first + n) (n even, first even) until every tag
// matches, copying nothing: a cheap wait on the elements its producers write
// last, so a large vector is fetched only once it is nearly complete.
template <int kMaxPer>
__device__ bool await_tags(const TagVec &src, uint32_t first, int n, uint32_t tag,
                           uint32_t *error) {
  const int pairs = n / 2;
  const int t = threadIdx.x;
  uint32_t pending = 0;
#pragma unroll
  for (int k = 0; k < kMaxPer; ++k)
    if (t + k * kBlock < pairs) pending |= 1u << k;
  for (uint32_t spin = 0;; ++spin) {
    Pair2 got[kMaxPer];
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k)
      if ((pending >> k) & 1u) got[k] = src.get2(first / 2 + t + k * kBlock);
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k)
      if (((pending >> k) & 1u) && got[k].t0 == tag && got[k].t1 == tag) pending &= ~(1u << k);
    if (__syncthreads_and(pending == 0)) return true;
    if (spin > kSpinLimit) {
      if (t == 0) atomicOr(error, 1u);
      return false;
    }
  }
}

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

// "Row pairs over all waves" loop with a 4-deep weight pipeline: while a
// unit is reduced, the wave's next three units are already loading.
// rows(u, a, b) gives unit u's two row pointers; epi(u, sa, sb) consumes the
// sums (every lane holds them). w0 must hold the weights of unit `first`
// when first < units.
template <int K, typename Rows, typename Epi>
__device__ __forceinline__ void run_pairs(int first, int stride, int units,
                                          const float4 (&xv)[PairSlots<K>::NJ],
                                          float4 (&w0)[PairSlots<K>::NJ], Rows rows,
                                          Epi epi) {
  constexpr int NJ = PairSlots<K>::NJ;
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

template <bool kProfile>
struct StageClock {
  uint64_t ticks[kResidentStages] = {};
  uint64_t prev = 0;
  __device__ void start() {
    if (kProfile) prev = wall_clock64();
  }
  __device__ void lap(int stage) {
    if (kProfile) {
      const uint64_t now = wall_clock64();
      ticks[stage] += now - prev;
      prev = now;
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
  float parts[kAttnMaxChunks * kPartStride];   // one head's partials (mergers)
  AttnLds attn;
  float kvn[2 * kHeadDim];                     // this step's K/V row of one head
  float red[kWavesPerBlock];
  float bv[kWavesPerBlock];
  uint32_t bi[kWavesPerBlock];
  float top[2 * kMaxResidentGrid];
};

template <int H, int I, int QD, bool kProfile>
__global__ __launch_bounds__(kBlock, 1) void resident_decode_kernel(ResidentArgs a) {
  static_assert(I <= 4864 && H <= 1024, "LDS staging sizes");
  __shared__ Shared sh;
  const int kv_dim = a.nkv * kHeadDim;
  const int group = a.nq / a.nkv;
  const int gw = blockIdx.x * kWavesPerBlock + wave_id();
  const int nwaves = gridDim.x * kWavesPerBlock;
  const int lane = lane_id();
  const uint32_t per_token = 6u * a.layers + 1u;
  const TagVec tq(a.q, QD);
  const TagVec tkv(a.kvnew, 2 * kv_dim);
  const TagVec tpart(a.part, kAttnMaxChunks * a.nq * kPartStride);
  const TagVec tattn(a.attn, QD);
  const TagVec th1(a.h1, H);
  const TagVec tact(a.act, I);
  const TagVec thid(a.hidden, H);
  const TagVec ttop(a.top, 2 * gridDim.x);
  auto tag = [&](uint32_t seq) { return a.epoch | (seq + 1u); };

  uint32_t token = a.first_token;
  uint32_t generated = 0;
  uint32_t stop_reason = 0;
  float top = 0.f;
  StageClock<kProfile> clock;
  clock.start();

  for (uint32_t t = 0; t < a.max_tokens; ++t) {
    const int position = static_cast<int>(a.start_position + t);
    if (token >= static_cast<uint32_t>(a.vocab) || position >= a.capacity) break;
    const int length = position + 1;
    const int chunk_len = attn_chunk_len(length);
    const int chunks = attn_chunks(length);
    const float *embed_row = a.embed + static_cast<size_t>(token) * H;
    const uint32_t s0 = t * per_token;

    for (int l = 0; l < a.layers; ++l) {
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

      // ---- A: RMSNorm + QKV + bias + RoPE ------------------------------------
      {
        const int units = (a.nq + 2 * a.nkv) * kRotary;
        if (static_cast<int>(blockIdx.x) * kWavesPerBlock < units) {
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
          if (gw < units) {
            const float *ra, *rb;
            rows(gw, ra, rb);
            load_pair_weights<H>(ra, rb, w0);
            consts(gw, c0);
          }
          if (l == 0) {
            for (int c = threadIdx.x; c < H; c += kBlock) sh.xs[c] = embed_row[c];
            __syncthreads();
          } else if (!gather<2>(thid, 0, H, tag_prev, sh.xs, a.error)) {
            return;
          }
          clock.lap(0);
          const float inv = block_inv_rms<H>(Lds{sh.xs}, a.eps, sh.red);
          float4 xv[PairSlots<H>::NJ];
          load_pair_operand<H, true>(Lds{sh.xs}, inv, w.attn_norm, xv);
          const Coherent kcache(kc, static_cast<uint32_t>(a.capacity) * kv_dim * 4u);
          const Coherent vcache(vc, static_cast<uint32_t>(a.capacity) * kv_dim * 4u);
          run_pairs<H>(gw, nwaves, units, xv, w0, rows, [&](int u, float sa, float sb) {
            if (lane != 0) return;
            float4 cv = c0;
            if (u != gw) consts(u, cv);
            const int head = u / kRotary, i = u % kRotary;
            const int ra = head * kHeadDim + i, rb = ra + kRotary;
            const float x0 = sa + cv.x;
            const float x1 = sb + cv.y;
            if (head < a.nq + a.nkv) {
              const float first = x0 * cv.z - x1 * cv.w;
              const float second = x1 * cv.z + x0 * cv.w;
              if (head < a.nq) {
                tq.put(ra, first, tag_q);
                tq.put(rb, second, tag_q);
              } else {
                const int o = (head - a.nq) * kHeadDim + i;
                tkv.put(o, first, tag_q);
                tkv.put(o + kRotary, second, tag_q);
                kcache.st(position * kv_dim + o, first);
                kcache.st(position * kv_dim + o + kRotary, second);
              }
            } else {
              const int o = (head - a.nq - a.nkv) * kHeadDim + i;
              tkv.put(kv_dim + o, x0, tag_q);
              tkv.put(kv_dim + o + kRotary, x1, tag_q);
              vcache.st(position * kv_dim + o, x0);
              vcache.st(position * kv_dim + o + kRotary, x1);
            }
          });
        }
      }
      clock.lap(1);

      // ---- B: split-KV attention partials -------------------------------------
      {
        const int units = a.nkv * chunks;
        const Coherent kcache(kc, static_cast<uint32_t>(a.capacity) * kv_dim * 4u);
        const Coherent vcache(vc, static_cast<uint32_t>(a.capacity) * kv_dim * 4u);
        for (int u = blockIdx.x; u < units; u += gridDim.x) {
          const int g = u / chunks, chunk = u % chunks;
          const int begin = chunk * chunk_len;
          const int end = min(length, begin + chunk_len);
          const bool has_new = position >= begin && position < end;
          bool ok = true;
          const LdsHeadRow knew{sh.kvn, g};
          const LdsHeadRow vnew{sh.kvn + kHeadDim, g};
          attn_partial_unit(
              kcache, vcache, knew, vnew, has_new ? position : -1, g, group, kv_dim, begin, end,
              sh.attn,
              [&]() {
                ok = gather<2>(tq, g * group * kHeadDim, group * kHeadDim, tag_q, sh.attn.qs,
                               a.error);
                if (ok && has_new)
                  ok = gather<1>(tkv, g * kHeadDim, kHeadDim, tag_q, sh.kvn, a.error) &&
                       gather<1>(tkv, kv_dim + g * kHeadDim, kHeadDim, tag_q, sh.kvn + kHeadDim,
                                 a.error);
                clock.lap(2);
              },
              [&](int hl, float m, float lsum, float acc, int d) {
                const uint32_t rec = ((g * group + hl) * kAttnMaxChunks + chunk) * kPartStride;
                tpart.put(rec + 2 + d, acc, tag_p);
                if (d == 0) {
                  tpart.put(rec, m, tag_p);
                  tpart.put(rec + 1, lsum, tag_p);
                }
              });
          if (!ok) return;
          __syncthreads();
        }
      }
      clock.lap(3);

      // ---- M: merge of each query head's partials (one workgroup per head) ----
      {
        const int h = static_cast<int>(blockIdx.x) - (static_cast<int>(gridDim.x) - a.nq);
        if (h >= 0) {
          if (!gather<3>(tpart, h * kAttnMaxChunks * kPartStride, chunks * kPartStride, tag_p,
                         sh.parts, a.error))
            return;
          if (threadIdx.x < kHeadDim) {
            const int d = threadIdx.x;
            tattn.put(h * kHeadDim + d,
                      attn_merge([&](int c, int k) { return sh.parts[c * kPartStride + k]; },
                                 chunks, d),
                      tag_m);
          }
        }
      }

      // ---- C: O projection + residual -----------------------------------------
      {
        constexpr int units = H / 2;
        if (static_cast<int>(blockIdx.x) * kWavesPerBlock < units) {
          auto rows = [&](int u, const float *&ra, const float *&rb) {
            ra = w.wo + static_cast<size_t>(2 * u) * QD;
            rb = ra + QD;
          };
          float4 w0[PairSlots<QD>::NJ];
          if (gw < units) {
            const float *ra, *rb;
            rows(gw, ra, rb);
            load_pair_weights<QD>(ra, rb, w0);
          }
          if (l == 0) {
            for (int c = threadIdx.x; c < H; c += kBlock) sh.hs[c] = embed_row[c];
          } else if (!gather<2>(thid, 0, H, tag_prev, sh.hs, a.error)) {
            return;
          }
          if (!gather<2>(tattn, 0, QD, tag_m, sh.xs, a.error)) return;
          clock.lap(4);
          float4 xv[PairSlots<QD>::NJ];
          load_pair_operand<QD, false>(Lds{sh.xs}, 1.f, nullptr, xv);
          run_pairs<QD>(gw, nwaves, units, xv, w0, rows, [&](int u, float sa, float sb) {
            if (lane != 0) return;
            th1.put(2 * u, sh.hs[2 * u] + sa, tag_h1);
            th1.put(2 * u + 1, sh.hs[2 * u + 1] + sb, tag_h1);
          });
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
        if (gw < I) {
          const float *ra, *rb;
          rows(gw, ra, rb);
          load_pair_weights<H>(ra, rb, w0);
        }
        if (!gather<2>(th1, 0, H, tag_h1, sh.hs, a.error)) return;
        clock.lap(6);
        const float inv = block_inv_rms<H>(Lds{sh.hs}, a.eps, sh.red);
        float4 xv[PairSlots<H>::NJ];
        load_pair_operand<H, true>(Lds{sh.hs}, inv, w.mlp_norm, xv);
        run_pairs<H>(gw, nwaves, I, xv, w0, rows, [&](int u, float g, float up) {
          if (lane == 0) tact.put(u, g / (1.f + expf(-g)) * up, tag_act);
        });
      }
      clock.lap(7);

      // ---- E: down projection + residual --------------------------------------
      {
        if (static_cast<int>(blockIdx.x) * kWavesPerBlock < H) {
          float4 wrow[RowSlots<I>::NJ];
          if (gw < H) load_row_weights<I>(w.wd + static_cast<size_t>(gw) * I, wrow);
          const int probe = min(I, nwaves);
          if (!await_tags<4>(tact, I - probe, probe, tag_act, a.error)) return;
          if (!gather<10>(tact, 0, I, tag_act, sh.xs, a.error)) return;
          clock.lap(8);
          float4 xv[RowSlots<I>::NJ];
          load_row_operand<I>(Lds{sh.xs}, xv);
          for (int r = gw; r < H; r += nwaves) {
            if (r != gw) load_row_weights<I>(w.wd + static_cast<size_t>(r) * I, wrow);
            const float s = row_dot<I>(wrow, xv);
            if (lane == 0) thid.put(r, sh.hs[r] + s, tag_hid);
          }
        }
      }
      clock.lap(9);
    }

    // ---- LM head + top-1 ---------------------------------------------------------
    const uint32_t tag_last = tag(s0 + 6 * (a.layers - 1) + 5);
    const uint32_t tag_top = tag(s0 + 6 * a.layers);
    {
      const int units = (a.vocab + 1) / 2;
      auto rows = [&](int u, const float *&ra, const float *&rb) {
        ra = a.head + static_cast<size_t>(2 * u) * H;
        rb = 2 * u + 1 < a.vocab ? ra + H : ra;
      };
      float4 w0[PairSlots<H>::NJ];
      if (gw < units) {
        const float *ra, *rb;
        rows(gw, ra, rb);
        load_pair_weights<H>(ra, rb, w0);
      }
      if (!gather<2>(thid, 0, H, tag_last, sh.xs, a.error)) return;
      clock.lap(10);
      const float inv = block_inv_rms<H>(Lds{sh.xs}, a.eps, sh.red);
      float4 xv[PairSlots<H>::NJ];
      load_pair_operand<H, true>(Lds{sh.xs}, inv, a.final_norm, xv);
      float *logits = a.logits + (a.history ? static_cast<size_t>(t) * a.vocab : 0);
      float best = -INFINITY;
      uint32_t best_i = UINT32_MAX;
      run_pairs<H>(gw, nwaves, units, xv, w0, rows, [&](int u, float sa, float sb) {
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
      if (!gather<4>(ttop, 0, 2 * gridDim.x, tag_top, sh.top, a.error)) return;
      clock.lap(12);
      float best = -INFINITY;
      uint32_t best_i = UINT32_MAX;
      for (uint32_t p = threadIdx.x; p < gridDim.x; p += kBlock) {
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
      args.stage_ticks
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
