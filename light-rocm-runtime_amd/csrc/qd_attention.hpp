// GQA decode attention shared by the stream-ordered kernels and the resident
// megakernel, so both paths run the same arithmetic in the same order.
//
// Split-KV: the attended positions 0..L-1 are cut into chunks of
// attn_chunk_len(L) positions (a multiple of 64, at most kAttnMaxChunks
// chunks). A workgroup owns one (query head, chunk) unit and produces an
// online-softmax partial (max m, sum l, acc[64]); the heads of a group read
// the same K/V rows, the repeats served by the caches. A merge combines
// the partials of a head: out = sum_c e^(m_c - M) acc_c / sum_c e^(m_c - M) l_c.
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

// Positions of a pass owned by one wave (lane l: position 16*wave + l/4,
// dims [16*(l%4), +16)).
constexpr int kWavePositions = kAttnPass / kWavesPerBlock;

struct AttnLds {
  float qkv[3 * kHeadDim];                  // the unit's query head, then this step's K, V row
  float vs[kAttnPass][kHeadDim];            // V rows of the current pass
  float ps[kAttnPass];                      // probabilities of the current pass
  float wp[kWavesPerBlock][kPartStride];    // per-wave partials (m, l, acc)
};

struct NoProbe {
  __device__ void operator()(int) const {}
};

// One (query head, chunk) unit, 256 threads; g is the head's KV head. The
// chunk is walked in passes of 16 * kWaves positions split over the first
// kWaves waves (any further wave only joins the barriers):
// thread t holds position t/4 of the pass with dims [16*(t%4), +16) of its
// K and V rows in registers (requested one pass ahead) and the matching 16
// query dims. Per pass each wave scores its 16 positions (16-dim partial dot
// per lane, summed over the quad), keeps an online softmax over its own
// positions (running max m, sum l) and accumulates P.V with lane = output
// dim from the pass's V rows staged in LDS. After the last pass wave 0
// merges the kWaves wave partials (out = sum_w e^(m_w - M) acc_w,
// l = sum_w e^(m_w - M) l_w) and emits them.
//
// wait_q(request) (whole workgroup, ends with a workgroup barrier) must
// call request() once -- it asks for the first pass's cached rows -- and
// leave the query head in lds.qkv[0, 64) and knew/vnew readable. kcache/vcache load
// cached K/V rows ([position][kv_heads*64], float4 index); knew/vnew supply
// the row at `new_pos` (the position this step writes, whose values may not
// be in the cache yet) with the same row-relative indexing. Results leave
// through emit(m, l, acc_d, d), called by wave 0 with d = lane. probe(k)
// marks phases for profiling: 3 query arrived, 0 first pass staged and
// scored, 1 passes done, 2 emitted.
template <int kWaves, typename KvSrc, typename NewSrc, typename WaitQ, typename Emit,
          typename Probe = NoProbe>
__device__ void attn_partial_unit(const KvSrc &kcache, const KvSrc &vcache,
                                  const NewSrc &knew, const NewSrc &vnew,
                                  int new_pos, int g, int kv_dim, int begin, int end,
                                  AttnLds &sh, WaitQ wait_q, Emit emit,
                                  Probe probe = Probe()) {
  const int t = threadIdx.x;
  const int quarter = t & 3;
  const int jl = t >> 2;  // position within the pass
  const int w = wave_id();
  const int lane = lane_id();
  // Waves past kWaves (a caller's helper wave) only join the barriers.
  static_assert(kWaves >= 1 && kWaves <= kWavesPerBlock, "unit waves");
  constexpr int kPass = kWaves * kWavePositions;
  const bool active = w < kWaves;
  const float scale = rsqrtf(static_cast<float>(kHeadDim));
  float m = -INFINITY, l = 0.f, acc = 0.f;
  float4 kr[4], vr[4];
  auto request = [&](int base) {
    const int j = base + jl;
    if (active && j < end && j != new_pos) {
      const uint32_t row4 = static_cast<uint32_t>(j * kv_dim + g * kHeadDim + quarter * 16) / 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kr[e] = kcache.ld4(row4 + e);
        vr[e] = vcache.ld4(row4 + e);
      }
    }
  };
  // The first pass's cached rows are requested before the query poll and
  // are in flight while the query (and this step's K/V row) are awaited.
  wait_q([&] { request(begin); });
  probe(3);
  float4 qv[4];
  {
    const float4 *q4 = reinterpret_cast<const float4 *>(sh.qkv);
#pragma unroll
    for (int e = 0; e < 4; ++e) qv[e] = q4[quarter * 4 + e];
  }
  for (int base = begin; base < end; base += kPass) {
    const int j = base + jl;
    const bool in = active && j < end;
    if (active && j == new_pos) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kr[e] = knew.ld4((g * kHeadDim + quarter * 16) / 4 + e);
        vr[e] = vnew.ld4((g * kHeadDim + quarter * 16) / 4 + e);
      }
    }
    float corr = 1.f;
    if (active) {
      const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
      float4 *vdst = reinterpret_cast<float4 *>(&sh.vs[jl][quarter * 16]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float4 b = vr[e];
        if (!in) b = zero;
        vdst[e] = b;
      }
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) s = fma4(kr[e], qv[e], s);
      s = quad_sum(s);
      const float sv = in ? s * scale : -INFINITY;
      const float m_new = fmaxf(m, wave_max(sv));
      // Every position appears in the four lanes of its quad: its first lane
      // contributes it to the sum.
      const float p = m_new == -INFINITY ? 0.f : expf(sv - m_new);
      corr = m_new == -INFINITY ? 1.f : expf(m - m_new);
      l = fmaf(l, corr, wave_sum(quarter == 0 ? p : 0.f));
      m = m_new;
      if (quarter == 0) sh.ps[jl] = p;
    }
    if (base + kPass < end) request(base + kPass);
    __syncthreads();  // vs and ps complete
    if (base == begin) probe(0);
    // P.V over this wave's 16 positions, lane = output dim.
    if (active) {
      const float4 *p4 = reinterpret_cast<const float4 *>(&sh.ps[w * kWavePositions]);
      float a = acc * corr;
#pragma unroll
      for (int i = 0; i < kWavePositions / 4; ++i) {
        const float4 pp = p4[i];
        const int r = w * kWavePositions + 4 * i;
        a = fmaf(pp.x, sh.vs[r][lane], a);
        a = fmaf(pp.y, sh.vs[r + 1][lane], a);
        a = fmaf(pp.z, sh.vs[r + 2][lane], a);
        a = fmaf(pp.w, sh.vs[r + 3][lane], a);
      }
      acc = a;
    }
    __syncthreads();  // the next pass overwrites vs / ps
  }
  probe(1);
  // Merge the four wave partials.
  if (active) {
    sh.wp[w][2 + lane] = acc;
    if (lane == 0) {
      sh.wp[w][0] = m;
      sh.wp[w][1] = l;
    }
  }
  __syncthreads();
  if (w == 0) {
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) mx = fmaxf(mx, sh.wp[v][0]);
    float lsum = 0.f, a = 0.f;
#pragma unroll
    for (int v = 0; v < kWaves; ++v) {
      const float mv = sh.wp[v][0];
      const float f = mv == -INFINITY ? 0.f : expf(mv - mx);
      lsum = fmaf(f, sh.wp[v][1], lsum);
      a = fmaf(f, sh.wp[v][2 + lane], a);
    }
    emit(mx, lsum, a, lane);
  }
  probe(2);
}

// One query head over the positions [0, n) of a chunk, computed by one wave;
// the resident role kernel (K/V staged in LDS) and the stream-ordered kernel
// (K/V read from the cache) both run it, so their partials are bit-identical.
// Blocks of 64 positions: lane = position for the scores (64-dim dot in
// order d = 0..63, scale 1/sqrt(64)), an online softmax (running max m, sum
// l), then P.V with lane = output dim: position u of the block feeds
// accumulator u % 4, the four combine as (a0 + a1) + (a2 + a3) and the block
// sum is added to the rescaled running acc. k4(d4, j) returns float4 d4 of
// position j's K row and v(j, d) element d of its V row; both are called
// only with j < n (the positions of a partial last block read row n - 1,
// with their probabilities masked to 0). q holds the head's 64 query values;
// (m, l, acc) carry the state across calls, so a chunk may be walked in
// windows whose lengths are multiples of 64.
template <typename K4, typename V>
__device__ __forceinline__ void attn_head_window(K4 k4, V v, const float4 (&q)[kHeadDim / 4], int n,
                                                 float &m, float &l, float &acc) {
  const int lane = lane_id();
  const float scale = rsqrtf(static_cast<float>(kHeadDim));
  for (int base = 0; base < n; base += kWave) {
    const int last = n - 1 - base;  // wave-uniform: positions past it are masked
    float4 kr[kHeadDim / 4];
#pragma unroll
    for (int d4 = 0; d4 < kHeadDim / 4; ++d4) kr[d4] = k4(d4, base + min(lane, last));
    float s = 0.f;
#pragma unroll
    for (int d4 = 0; d4 < kHeadDim / 4; ++d4) s = fma4(kr[d4], q[d4], s);
    const float sv = lane <= last ? s * scale : -INFINITY;
    const float m_new = fmaxf(m, wave_max(sv));
    const float p = m_new == -INFINITY ? 0.f : expf(sv - m_new);
    const float corr = m_new == -INFINITY ? 1.f : expf(m - m_new);
    l = fmaf(l, corr, wave_sum(p));
    m = m_new;
    float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kWave; ++u)
      a[u & 3] = fmaf(read_lane(p, u), v(base + min(u, last), lane), a[u & 3]);
    acc = fmaf(acc, corr, (a[0] + a[1]) + (a[2] + a[3]));
  }
}

// Merge of one head's partials for output dim d; part(c, k) returns element
// k of chunk c's record (0: m, 1: l, 2 + d: acc). Records are stored head
// major: record (h, c) at (h * kAttnMaxChunks + c) * kPartStride.
template <typename Part>
__device__ __forceinline__ float attn_merge(const Part &part, int chunks, int d) {
  float mx = -INFINITY;
  for (int c = 0; c < chunks; ++c) mx = fmaxf(mx, part(c, 0));
  float num = 0.f, den = 0.f;
  for (int c = 0; c < chunks; ++c) {
    const float w = expf(part(c, 0) - mx);
    den = fmaf(w, part(c, 1), den);
    num = fmaf(w, part(c, 2 + d), num);
  }
  return num / den;
}

}  // namespace dev
}  // namespace qd
