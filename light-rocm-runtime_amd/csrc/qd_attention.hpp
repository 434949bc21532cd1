// GQA decode attention shared by the stream-ordered kernels and the resident
// megakernel, so both paths run the same arithmetic in the same order.
//
// Split-KV: the attended positions 0..L-1 are cut into chunks of
// attn_chunk_len(L) positions (a multiple of 64, at most kAttnMaxChunks
// chunks). A workgroup owns one (KV head, chunk) unit and produces, for each
// of the group's query heads, an online-softmax partial (max m, sum l,
// acc[64]); the chunk is walked in passes of 64 positions. A merge combines
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

struct AttnLds {
  float qs[kMaxGroup * kHeadDim];      // the group's query heads
  float vs[kAttnPass][kHeadDim];       // V rows of the current pass
  float ps[kMaxGroup][kAttnPass];      // scores, then probabilities
  float m[kMaxGroup];                  // running max per head
  float l[kMaxGroup];                  // running sum per head
  float scale[kMaxGroup];              // e^(m_old - m_new) of the pass
};

// One (KV head g, chunk) unit: 256 threads; thread t scores position t/4 of
// the pass on dims [16*(t%4), +16) and owns outputs o = t and t + 256 of the
// group's heads*64 accumulators. wait_q() (whole workgroup) must leave the
// group's queries in lds.qs and make knew/vnew readable; it runs once, after
// the first pass's cached rows were requested. kcache/vcache
// load cached K/V rows ([position][kv_heads*64], float4 index); knew/vnew
// supply the row at `new_pos` (the position this step writes, whose values
// may not be in the cache yet) with the same row-relative indexing. Results
// leave through emit(h_local, m, l, acc_d, d), called once per output
// (head, d); m and l are the head's softmax max and sum.
template <typename KvSrc, typename NewSrc, typename WaitQ, typename Emit>
__device__ void attn_partial_unit(const KvSrc &kcache, const KvSrc &vcache,
                                  const NewSrc &knew, const NewSrc &vnew,
                                  int new_pos, int g, int group, int kv_dim,
                                  int begin, int end, AttnLds &sh, WaitQ wait_q,
                                  Emit emit) {
  const int t = threadIdx.x;
  const int quarter = t & 3;
  const int jl = t >> 2;
  const int outs = group * kHeadDim;
  float acc0 = 0.f, acc1 = 0.f;
  if (t < kMaxGroup) {
    sh.m[t] = -INFINITY;
    sh.l[t] = 0.f;
  }
  for (int base = begin; base < end; base += kAttnPass) {
    const int j = base + jl;
    const bool valid = j < end;
    float4 kr[4], vr[4];
    const bool is_new = valid && j == new_pos;
    if (!is_new) {
      const uint32_t row4 =
          static_cast<uint32_t>((valid ? j : 0) * kv_dim + g * kHeadDim + quarter * 16) / 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kr[e] = kcache.ld4(row4 + e);
        vr[e] = vcache.ld4(row4 + e);
      }
    }
    // The cached rows of the first pass are in flight while the query (and
    // this step's K/V row) are awaited.
    if (base == begin) wait_q();
    if (is_new) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kr[e] = knew.ld4((g * kHeadDim + quarter * 16) / 4 + e);
        vr[e] = vnew.ld4((g * kHeadDim + quarter * 16) / 4 + e);
      }
    }
    __syncthreads();  // previous pass finished reading vs / ps
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float *dst = &sh.vs[jl][quarter * 16 + 4 * e];
      dst[0] = valid ? vr[e].x : 0.f;
      dst[1] = valid ? vr[e].y : 0.f;
      dst[2] = valid ? vr[e].z : 0.f;
      dst[3] = valid ? vr[e].w : 0.f;
    }
    for (int hl = 0; hl < group; ++hl) {
      const float4 *q4 =
          reinterpret_cast<const float4 *>(sh.qs + hl * kHeadDim + quarter * 16);
      float s = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) s = fma4(kr[e], q4[e], s);
      s += __shfl_xor(s, 1, kWave);
      s += __shfl_xor(s, 2, kWave);
      if (quarter == 0)
        sh.ps[hl][jl] = valid ? s * rsqrtf(static_cast<float>(kHeadDim)) : -INFINITY;
    }
    __syncthreads();
    // Wave w updates heads w, w+4, ...: lane = position of the pass.
    for (int hl = wave_id(); hl < group; hl += kWavesPerBlock) {
      const int lane = lane_id();
      const float s = sh.ps[hl][lane];
      float mx = s;
#pragma unroll
      for (int o = kWave / 2; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
      const float m_old = sh.m[hl];
      const float m_new = fmaxf(m_old, mx);
      const float p = expf(s - m_new);
      float sum = p;
#pragma unroll
      for (int o = kWave / 2; o > 0; o >>= 1) sum += __shfl_xor(sum, o, kWave);
      sh.ps[hl][lane] = p;
      if (lane == 0) {
        const float sc = expf(m_old - m_new);
        sh.scale[hl] = sc;
        sh.l[hl] = sh.l[hl] * sc + sum;
        sh.m[hl] = m_new;
      }
    }
    __syncthreads();
    // P.V for the pass.
    if (t < outs) {
      const int hl = t / kHeadDim, d = t % kHeadDim;
      float a = 0.f;
#pragma unroll 8
      for (int jj = 0; jj < kAttnPass; ++jj) a = fmaf(sh.ps[hl][jj], sh.vs[jj][d], a);
      acc0 = acc0 * sh.scale[hl] + a;
    }
    if (t + kBlock < outs) {
      const int o = t + kBlock;
      const int hl = o / kHeadDim, d = o % kHeadDim;
      float a = 0.f;
#pragma unroll 8
      for (int jj = 0; jj < kAttnPass; ++jj) a = fmaf(sh.ps[hl][jj], sh.vs[jj][d], a);
      acc1 = acc1 * sh.scale[hl] + a;
    }
  }
  __syncthreads();
  if (t < outs) emit(t / kHeadDim, sh.m[t / kHeadDim], sh.l[t / kHeadDim], acc0, t % kHeadDim);
  if (t + kBlock < outs) {
    const int o = t + kBlock;
    emit(o / kHeadDim, sh.m[o / kHeadDim], sh.l[o / kHeadDim], acc1, o % kHeadDim);
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
