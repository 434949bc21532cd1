// GQA decode attention shared by the stream-ordered kernels and the resident
// megakernel, so both paths run the same arithmetic in the same order.
//
// Split-KV: the attended positions 0..L-1 are cut into chunks of
// attn_chunk_len(L) positions (a multiple of 64, at most kAttnMaxChunks
// chunks). A workgroup owns one (query head, chunk) unit and produces an
// online-softmax partial (max m, sum l, acc[64]); the heads of a group read
// the same K/V rows, the repeats served by the caches. A merge combines
// the partials of a head: out = sum_c 2^(m_c - M) acc_c / sum_c 2^(m_c - M) l_c
// (scores and maxima in base-2 units, see kScoreScaleLog2).
// Semantics: benchmarks/qwen_stateful_graph_kernel.cpp:554-600 (scale
// 1/sqrt(64), query head h reads KV head h / (heads / kv_heads), positions
// 0..kv_length inclusive).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qd_device.hpp"
#include "qd_device_math.hpp"

namespace qd {

namespace dev {

// Scores are kept in base-2 units, s * log2(e) / sqrt(64), so every
// softmax exponential is one v_exp_f32 (exp2) and the partial maxima m are
// base-2 too; e^(x / sqrt(64)) = 2^(x * log2(e) / sqrt(64)).
constexpr float kScoreScaleLog2 = 0.18033688011112042f;  // log2(e) / 8

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Probabilities of a block handed from lane u (position u) to every lane,
// four at a time: get(u4) returns those of positions 4 u4 .. 4 u4 + 3.
// Lane reads (v_readlane), for a kernel without LDS to spare.
struct PLanes {
  float p;
  __device__ void put(float v) { p = v; }
  __device__ float4 get(int u4) const {
    return make_float4(read_lane(p, 4 * u4), read_lane(p, 4 * u4 + 1), read_lane(p, 4 * u4 + 2),
                       read_lane(p, 4 * u4 + 3));
  }
};
// The same through 64 floats of the wave's own LDS: every lane writes its
// probability, then reads them as float4 broadcasts (no VALU per position).
struct PLds {
  float *buf;
  __device__ void put(float v) {
    buf[lane_id()] = v;
    // Lanes of the wave read each other's words: order the writes first.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  __device__ float4 get(int u4) const { return reinterpret_cast<const float4 *>(buf)[u4]; }
};

// One query head over the positions [0, n) of a chunk, computed by one wave;
// the resident role kernel (K/V staged in LDS) and the stream-ordered kernel
// (K/V read from the cache) both run it, so their partials are bit-identical.
// Blocks of 64 positions: lane = position for the scores (64-dim dot in
// order d = 0..63, scaled by kScoreScaleLog2), an online base-2 softmax
// (running max m, sum l), then P.V with lane = output dim: position u of the block feeds
// accumulator u % 4, the four combine as (a0 + a1) + (a2 + a3) and the block
// sum is added to the rescaled running acc. k4(d4, j) returns float4 d4 of
// position j's K row and v(j, d) element d of its V row; both are called
// only with j < n (the positions of a partial last block read row n - 1,
// with their probabilities masked to 0). pb hands the probabilities between
// lanes (PLanes or PLds: same values, same arithmetic). q holds the head's
// 64 query values; (m, l, acc) carry the state across calls, so a chunk may
// be walked in windows whose lengths are multiples of 64.
template <typename K4, typename V, typename PB>
__device__ __forceinline__ void attn_head_window(K4 k4, V v, PB pb, const float4 (&q)[kHeadDim / 4], int n,
                                                 float &m, float &l, float &acc) {
  const int lane = lane_id();
  for (int base = 0; base < n; base += kWave) {
    const int last = n - 1 - base;  // wave-uniform: positions past it are masked
    float4 kr[kHeadDim / 4];
#pragma unroll
    for (int d4 = 0; d4 < kHeadDim / 4; ++d4) kr[d4] = k4(d4, base + min(lane, last));
    float s = 0.f;
#pragma unroll
    for (int d4 = 0; d4 < kHeadDim / 4; ++d4) s = fma4(kr[d4], q[d4], s);
    const float sv = lane <= last ? __fmul_rn(s, kScoreScaleLog2) : -INFINITY;
    const float m_new = fmaxf(m, wave_max(sv));
    const float p = m_new == -INFINITY ? 0.f : exp2_fast(sv - m_new);
    const float corr = m_new == -INFINITY ? 1.f : exp2_fast(m - m_new);
    l = fmaf(l, corr, wave_sum(p));
    m = m_new;
    pb.put(p);
    float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u4 = 0; u4 < kWave / 4; ++u4) {
      const float4 pp = pb.get(u4);
      a[0] = fmaf(pp.x, v(base + min(4 * u4, last), lane), a[0]);
      a[1] = fmaf(pp.y, v(base + min(4 * u4 + 1, last), lane), a[1]);
      a[2] = fmaf(pp.z, v(base + min(4 * u4 + 2, last), lane), a[2]);
      a[3] = fmaf(pp.w, v(base + min(4 * u4 + 3, last), lane), a[3]);
    }
    acc = fmaf(acc, corr, (a[0] + a[1]) + (a[2] + a[3]));
  }
}

// Merge of one head's partials for output dim d; part(c, k) returns element
// k of chunk c's record (0: m, base 2; 1: l; 2 + d: acc):
// out = sum_c 2^(m_c - M) acc_c / sum_c 2^(m_c - M) l_c. The numerator folds
// the chunks in order (fma); the denominator sums the products
// 2^(m_c - M) l_c of all kAttnMaxChunks chunk places (zero past `chunks`) as
// the pairwise tree of row16_sum, the order the resident role kernel forms
// it in with one lane per chunk. Records are stored head major: record
// (h, c) at (h * kAttnMaxChunks + c) * kPartStride.
template <typename Part>
__device__ __forceinline__ float attn_merge(const Part &part, int chunks, int d) {
  static_assert(kAttnMaxChunks == 16, "one 16-lane row per head");
  float mx = -INFINITY;
  for (int c = 0; c < chunks; ++c) mx = fmaxf(mx, part(c, 0));
  float t[kAttnMaxChunks];
  float num = 0.f;
  for (int c = 0; c < kAttnMaxChunks; ++c) {
    t[c] = 0.f;
    if (c < chunks) {
      const float w = exp2_fast(part(c, 0) - mx);
      t[c] = __fmul_rn(w, part(c, 1));  // a rounded product: never contracted into the sums
      num = fmaf(w, part(c, 2 + d), num);
    }
  }
  float den = 0.f;
#pragma unroll
  for (int o = 0; o < kAttnMaxChunks; o += 8) {
    const float a = (t[o] + t[o + 1]) + (t[o + 2] + t[o + 3]);
    const float b = (t[o + 4] + t[o + 5]) + (t[o + 6] + t[o + 7]);
    den = o == 0 ? a + b : den + (a + b);
  }
  return num / den;
}

}  // namespace dev
}  // namespace qd
