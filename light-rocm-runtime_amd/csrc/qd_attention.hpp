// GQA decode attention shared by the stream-ordered kernels and the resident
// megakernel, so both paths run the same arithmetic in the same order.
//
// Split-KV: the attended positions 0..L-1 are cut into chunks of
// attn_chunk_len(L) positions (a multiple of 64, at most kAttnMaxChunks
// chunks), and chunks into blocks of 64. Each (query head, block) gets a
// softmax partial (max m, sum l, acc[64]), a chunk's blocks are folded in
// order into the chunk's partial, and a merge combines
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
// four at a time: get(hh, u4) returns head slot hh's probabilities of
// positions 4 u4 .. 4 u4 + 3. Lane reads (v_readlane), one head, for a
// kernel without LDS to spare.
struct PLanes {
  float p;
  __device__ void put(int, float v) { p = v; }
  __device__ void sync() {}
  __device__ float4 get(int, int u4) const {
    return make_float4(read_lane(p, 4 * u4), read_lane(p, 4 * u4 + 1), read_lane(p, 4 * u4 + 2),
                       read_lane(p, 4 * u4 + 3));
  }
};
// The same through the wave's own LDS (head slot hh at buf + hh * stride,
// 16-byte aligned): every lane writes its probabilities, then reads them as
// float4 broadcasts (no VALU per position).
struct PLds {
  float *buf;
  int stride;
  __device__ void put(int hh, float v) { buf[hh * stride + lane_id()] = v; }
  // Lanes of the wave read each other's words: order the writes first.
  __device__ void sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  __device__ float4 get(int hh, int u4) const { return reinterpret_cast<const float4 *>(buf + hh * stride)[u4]; }
};

// Softmax partial of one block of up to 64 positions (base .. base + last)
// for kNH query heads taken by one wave, the block's K/V shared by them; the
// resident role kernel (K/V staged in LDS, heads spread over the waves) and
// the stream-ordered kernel (one head per wave, K/V read from the cache)
// both run it, so their partials are bit-identical. Per head, with lane =
// position: the score is the 64-dim dot in order d = 0..63 scaled by
// kScoreScaleLog2 (positions past `last` masked to -inf), m = the block max
// (wave_max), p = 2^(s - m), l = wave_sum(p); then P.V with lane = output
// dim: position u feeds accumulator u % 4 and acc = (a0 + a1) + (a2 + a3).
// k4(d4, j): float4 d4 of position j's K row; q4(hh, d4): float4 d4 of head
// slot hh's query; v(j, d): element d of position j's V row (positions of a
// partial block read row base + last, their probabilities being 0); pb
// hands the probabilities between lanes (PLanes or PLds: same values).
template <int kNH, typename K4, typename Q4, typename V, typename PB>
__device__ __forceinline__ void attn_block(K4 k4, Q4 q4, V v, PB &pb, int base, int last, float (&m)[kNH],
                                           float (&l)[kNH], float (&acc)[kNH]) {
  const int lane = lane_id();
  float4 kr[kHeadDim / 4];
#pragma unroll
  for (int d4 = 0; d4 < kHeadDim / 4; ++d4) kr[d4] = k4(d4, base + min(lane, last));
  float sv[kNH];
#pragma unroll
  for (int hh = 0; hh < kNH; ++hh) {
    float s = 0.f;
#pragma unroll
    for (int d4 = 0; d4 < kHeadDim / 4; ++d4) s = fma4(kr[d4], q4(hh, d4), s);
    sv[hh] = lane <= last ? __fmul_rn(s, kScoreScaleLog2) : -INFINITY;
  }
#pragma unroll
  for (int hh = 0; hh < kNH; ++hh) {
    m[hh] = wave_max(sv[hh]);
    const float p = exp2_fast(sv[hh] - m[hh]);
    l[hh] = wave_sum(p);
    pb.put(hh, p);
  }
  pb.sync();
  float a[kNH][4];
#pragma unroll
  for (int hh = 0; hh < kNH; ++hh) a[hh][0] = a[hh][1] = a[hh][2] = a[hh][3] = 0.f;
#pragma unroll
  for (int u4 = 0; u4 < kWave / 4; ++u4) {
    float vj[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) vj[k] = v(base + min(4 * u4 + k, last), lane);
#pragma unroll
    for (int hh = 0; hh < kNH; ++hh) {
      const float4 pp = pb.get(hh, u4);
      a[hh][0] = fmaf(pp.x, vj[0], a[hh][0]);
      a[hh][1] = fmaf(pp.y, vj[1], a[hh][1]);
      a[hh][2] = fmaf(pp.z, vj[2], a[hh][2]);
      a[hh][3] = fmaf(pp.w, vj[3], a[hh][3]);
    }
  }
#pragma unroll
  for (int hh = 0; hh < kNH; ++hh) acc[hh] = (a[hh][0] + a[hh][1]) + (a[hh][2] + a[hh][3]);
}

// Folds a block partial (mb, lb, ab) into a chunk's running partial
// (M, L, A), blocks taken in position order and (M, L, A) starting at
// (-inf, 0, 0): with M' = max(M, mb), L = L 2^(M - M') + 2^(mb - M') lb and
// A likewise (the first block passes through unchanged).
__device__ __forceinline__ void attn_fold(float mb, float lb, float ab, float &M, float &L, float &A) {
  const float mn = fmaxf(M, mb);
  const float co = M == -INFINITY ? 0.f : exp2_fast(M - mn);
  const float w = exp2_fast(mb - mn);
  L = fmaf(L, co, __fmul_rn(w, lb));
  A = fmaf(A, co, __fmul_rn(w, ab));
  M = mn;
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
