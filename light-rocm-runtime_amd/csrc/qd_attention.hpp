// GQA decode attention shared by the stream-ordered kernels and the resident
// megakernel, so both paths run the same arithmetic in the same order.
//
// Split-KV: the attended positions 0..L-1 are cut into chunks of
// attn_chunk_len(L, parts, kAttnGrain) positions (a multiple of 16, at most
// kAttnMaxChunks chunks). A chunk of one KV group is one workgroup's work,
// computed in one of two ways fixed by the chunk length, so every path
// agrees:
//  - one block (up to 64 positions, attn_single_block): one wave per query
//    head forms the block's softmax partial on the vector ALUs
//    (attn_block_valu);
//  - longer: the chunk is cut into tiles of 32 positions, dealt round-robin
//    to kAttnSlots waves; each wave keeps an online-softmax partial of all
//    the group's heads (up to kAttnMaxGroup) over its tiles (scores and P.V
//    on FP32 MFMA in 4x4 blocks, attn_tile), and the wave partials are
//    folded in slot order.
// Either way each head gets one record (max m, sum l, acc[64]) per chunk. A
// merge combines the records of a head:
// out = sum_c 2^(m_c - M) acc_c / sum_c 2^(m_c - M) l_c (scores and maxima
// in base-2 units, see kScoreScaleLog2).
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

// Folds a partial (mb, lb, ab) into a running partial (M, L, A) that starts
// at (-inf, 0, 0): with M' = max(M, mb), L = L 2^(M - M') + 2^(mb - M') lb
// and A likewise (the first partial passes through unchanged).
__device__ __forceinline__ void attn_fold(float mb, float lb, float ab, float &M, float &L, float &A) {
  const float mn = fmaxf(M, mb);
  const float co = M == -INFINITY ? 0.f : exp2_fast(M - mn);
  const float w = exp2_fast(mb - mn);
  L = fmaf(L, co, __fmul_rn(w, lb));
  A = fmaf(A, co, __fmul_rn(w, ab));
  M = mn;
}

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
// for kNH query heads taken by one wave, the block's K/V shared by them, on
// the vector ALUs: the arithmetic of a chunk of one block (attn_single_block),
// which the resident role kernel and the stream-ordered kernel both run, so
// their partials are bit-identical. Per head, with lane =
// position: the score is the 64-dim dot in order d = 0..63 scaled by
// kScoreScaleLog2 (positions past `last` masked to -inf), m = the block max
// (wave_max), p = 2^(s - m), l = wave_sum(p); then P.V with lane = output
// dim: position u feeds accumulator u % 4 and acc = (a0 + a1) + (a2 + a3).
// k4(d4, j): float4 d4 of position j's K row; q4(hh, d4): float4 d4 of head
// slot hh's query; v(j, d): element d of position j's V row (positions of a
// partial block read row base + last, their probabilities being 0); pb
// hands the probabilities between lanes (PLanes or PLds: same values).
template <int kNH, typename K4, typename Q4, typename V, typename PB>
__device__ __forceinline__ void attn_block_valu(K4 k4, Q4 q4, V v, PB &pb, int base, int last, float (&m)[kNH],
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

// A chunk of at most one block (chunk length up to kAttnPass: contexts of
// up to 64 * parts positions) is computed on the vector ALUs, one query head
// per wave (attn_block_valu); longer chunks go through the MFMA tiles below.
// With one block per chunk the tiles' cross-wave merge would be all
// overhead, and a wave per head keeps the K/V reads to one block.
__host__ __device__ inline bool attn_single_block(int chunk_len) { return chunk_len <= kAttnPass; }

typedef float attn_f4v __attribute__((ext_vector_type(4)));

// Tile slots per (chunk, KV group): the waves of one attention workgroup.
// Tile i of a chunk belongs to tile slot i % kAttnSlots.
constexpr int kAttnSlots = 8;

// Component c of a float4.
__device__ __forceinline__ float attn_c(float4 v, int c) { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; }

// ---- Tiles of a longer chunk (groups of up to 8 heads) ---------------------
// One v_mfma_f32_4x4x1f32 is 16 independent 4x4 outer products: block b =
// lane / 4; lane 4 b + i gives row i of A and column i of B; register r of
// lane 4 b + j receives element (r, j) of the block's D. Eight heads are two
// head quads, so the 16 blocks cover 8 heads by 32 positions (or 32 dims),
// and 7 of the 8 rows do work for a group of 7, where a 16x16x4 MFMA would use 7
// of 16. Lane l: head quad hq = l / 32, m = l % 32, x = l % 4.
// Both halves of the wave need the same K and V operands, so each half
// loads one half of them and the MFMA's B broadcast (BLGP 1: lanes 0-31's B
// for all 64 lanes; BLGP 2: lanes 32-63's) hands them to the other: each K
// and V element is read from LDS once per tile.
//   scores: block b has head rows 4 hq + 0..3 and positions 4 (b % 8) +
//           0..3; lanes 0-31 hold K dims 0-31 of position t0 + m, lanes
//           32-63 dims 32-63 of the same position; lane l ends holding
//           position t0 + m of rows 4 hq + r (register r);
//   P.V:    the same blocks with output dims as columns; lane l holds
//           element l of each V row; lane l ends holding rows 4 hq + r of
//           dims m (BLGP 1) and 32 + m (BLGP 2).
constexpr int kAttnTile = 32;
constexpr int kAttnMaxGroup = 8;
// A-operand broadcast of the score MFMAs (CBSZ): block 0 of each group of
// 2^3 blocks (ABID 0) hands its A to the group, i.e. lanes 0-3 to lanes 0-31
// and lanes 32-35 to lanes 32-63; the A operand (a head's query) is the same
// in every block of a half.
constexpr int kAttnCbsz = 3;
// Probability tile of one wave in LDS: [8 rows][32 positions], rows 36 floats
// apart (16-byte aligned, the 8 rows' float4 reads on distinct banks).
constexpr int kAttnTilePsStride = 36;
constexpr int kAttnTilePsFloats = kAttnMaxGroup * kAttnTilePsStride;
// LDS of one wave for its probabilities: a tile's [8][36], or the 64 of a
// one-block chunk's head (PLds at offset 4).
constexpr int kAttnPsFloats = kAttnTilePsFloats;
static_assert(kAttnPsFloats >= 4 + kWave, "one-block probabilities fit the wave's LDS");

// One wave's running softmax partial over its tiles (base-2
// units): m[r], the running max of row 4 hq + r (equal on the half's 32
// lanes); l[r], this lane's share of the row's running sum (the
// probabilities of position m of each tile; the half's 32 shares sum to the
// row's sum); o[s][r], row 4 hq + r of output dim 32 s + m.
struct AttnAcc {
  float m[4], l[4];
  attn_f4v o[2];
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      m[r] = -INFINITY;
      l[r] = 0.f;
    }
    o[0] = o[1] = attn_f4v{0.f, 0.f, 0.f, 0.f};
  }
};

// Query operand of a group of up to 8 heads: q[d4] = float4 d4 of the query
// of head 4 (l / 32) + l % 4 (zero past the group's `heads`), in lanes 0-3
// and 32-35 only (the tiles' MFMAs broadcast those lanes' A operand to
// their half; the other lanes hold zeros). q4(h, d4) returns float4 d4 of
// head h's query.
template <typename Q4>
__device__ __forceinline__ void attn_query(Q4 q4, int heads, float4 (&q)[kHeadDim / 4]) {
  const int row = 4 * (lane_id() >> 5) + (lane_id() & 3);
#pragma unroll
  for (int d4 = 0; d4 < kHeadDim / 4; ++d4) q[d4] = make_float4(0.f, 0.f, 0.f, 0.f);
  if ((lane_id() & 31) < 4 && row < heads) {
#pragma unroll
    for (int d4 = 0; d4 < kHeadDim / 4; ++d4) q[d4] = q4(row, d4);
  }
}

// One tile of 32 positions [t0, t0 + 32) for every head of a KV group of up
// to 8. Positions >= end are masked (score -inf). kl(i): float4 i of this
// lane's half of its position's K row (dims 32 hq + 4 i .. 32 hq + 4 i + 3 of
// position min(t0 + m, end - 1)); vl(k): element `lane` of the V row of
// position min(t0 + k, end - 1) (k = 0..31); ps: this wave's
// kAttnTilePsFloats of LDS.
//   S[h][j] = q_h . k_j: 64 MFMAs in four chains: dims 4 i + c (i < 8,
//             BLGP 1) and 32 + 4 i + c (BLGP 2) at step (i, c), chain
//             2 (i % 2) + half; the chains summed as (s0 + s1) + (s2 + s3);
//             scaled by kScoreScaleLog2;
//   online softmax per row: m' = max(m, half_max of the tile's scores),
//             c = 2^(m - m') (0 for the first tile), p = 2^(s - m'),
//             l = l c + p (per lane), o = o c (rounded products);
//   o += P . V: positions in order, one MFMA per position and dim half.
template <typename KL, typename VL>
__device__ __forceinline__ void attn_tile_ops(const float4 (&q)[kHeadDim / 4], KL kl, VL vl, float *ps, int t0,
                                              int end, AttnAcc &acc) {
  const int lane = lane_id(), hq = lane >> 5, m = lane & 31, x = lane & 3;
  float4 kv[kHeadDim / 8];
#pragma unroll
  for (int i = 0; i < kHeadDim / 8; ++i) kv[i] = kl(i);
  attn_f4v s[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) s[u] = attn_f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < kHeadDim / 8; ++i) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float b = attn_c(kv[i], c);
      s[2 * (i & 1)] = __builtin_amdgcn_mfma_f32_4x4x1f32(attn_c(q[i], c), b, s[2 * (i & 1)], kAttnCbsz, 0, 1);
      s[2 * (i & 1) + 1] = __builtin_amdgcn_mfma_f32_4x4x1f32(attn_c(q[kHeadDim / 8 + i], c), b,
                                                              s[2 * (i & 1) + 1], kAttnCbsz, 0, 2);
    }
  }
  const attn_f4v sc = (s[0] + s[1]) + (s[2] + s[3]);
  const bool valid = t0 + m < end;
  float xs[4], mx[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) xs[r] = valid ? __fmul_rn(sc[r], kScoreScaleLog2) : -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; ++r) mx[r] = fmaxf(xs[r], dpp<kDppXor1>(xs[r]));
#pragma unroll
  for (int r = 0; r < 4; ++r) mx[r] = fmaxf(mx[r], dpp<kDppXor2>(mx[r]));
#pragma unroll
  for (int r = 0; r < 4; ++r) mx[r] = fmaxf(mx[r], dpp<kDppHalfMirror>(mx[r]));
#pragma unroll
  for (int r = 0; r < 4; ++r) mx[r] = fmaxf(mx[r], dpp<kDppMirror>(mx[r]));
#pragma unroll
  for (int r = 0; r < 4; ++r) mx[r] = fmaxf(acc.m[r], row_pair_max(mx[r]));
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float cr = acc.m[r] == -INFINITY ? 0.f : exp2_fast(acc.m[r] - mx[r]);
    const float p = exp2_fast(xs[r] - mx[r]);
    ps[(4 * hq + r) * kAttnTilePsStride + m] = p;
    acc.l[r] = fmaf(acc.l[r], cr, p);
    acc.m[r] = mx[r];
    acc.o[0][r] = __fmul_rn(acc.o[0][r], cr);
    acc.o[1][r] = __fmul_rn(acc.o[1][r], cr);
  }
  // Lanes read each other's probabilities: order the wave's LDS writes.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float4 pa[kAttnTile / 4];
#pragma unroll
  for (int k4 = 0; k4 < kAttnTile / 4; ++k4)
    pa[k4] = reinterpret_cast<const float4 *>(ps + (4 * hq + x) * kAttnTilePsStride)[k4];
  // The next tile rewrites ps only after every lane has read it.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // V operands in groups of 8, each group read before its MFMAs (one LDS
  // wait per group rather than one per position).
#pragma unroll
  for (int k0 = 0; k0 < kAttnTile; k0 += 8) {
    float vv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) vv[j] = vl(k0 + j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float a = attn_c(pa[(k0 + j) / 4], (k0 + j) % 4);
      acc.o[0] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, vv[j], acc.o[0], 0, 0, 1);
      acc.o[1] = __builtin_amdgcn_mfma_f32_4x4x1f32(a, vv[j], acc.o[1], 0, 0, 2);
    }
  }
}

// attn_tile_ops with K and V read through k4(pos, d4) (float4 d4 of position
// pos's K row) and v(pos, d) (element d of its V row).
template <typename K4, typename V>
__device__ __forceinline__ void attn_tile(const float4 (&q)[kHeadDim / 4], K4 k4, V v, float *ps, int t0, int end,
                                          AttnAcc &acc) {
  const int lane = lane_id(), hq = lane >> 5;
  const int pk = min(t0 + (lane & 31), end - 1);
  attn_tile_ops(
      q, [&](int i) { return k4(pk, (kHeadDim / 8) * hq + i); }, [&](int k) { return v(min(t0 + k, end - 1), lane); },
      ps, t0, end, acc);
}

// The tiles of slot `slot` that lie in [wb, we) of a chunk
// starting at `begin` (wb - begin a multiple of kAttnTile), in position
// order: tiles slot, slot + kAttnSlots, ... of the chunk.
template <typename K4, typename V>
__device__ __forceinline__ void attn_slot_tiles(const float4 (&q)[kHeadDim / 4], K4 k4, V v, float *ps,
                                                     int begin, int wb, int we, int end, int slot,
                                                     AttnAcc &acc) {
  const int t_lo = (wb - begin) / kAttnTile, t_hi = (we - begin + kAttnTile - 1) / kAttnTile;
  for (int t = t_lo + slot; t < t_hi; t += kAttnSlots)
    attn_tile(q, k4, v, ps, begin + t * kAttnTile, end, acc);
}

// Wave partials of a chunk staged for the merge: [slot][row] maxima and
// sums, [slot][row][64] outputs, for the group's first `heads` rows.
struct AttnStage {
  float *m, *l, *o;  // m, l: kAttnSlots * kMaxGroup floats; o: kAttnSlots * kMaxGroup * 64
  // Each row's sum is the half_sum of its lanes' shares.
  __device__ __forceinline__ void put(int slot, int heads, const AttnAcc &acc) const {
    const int lane = lane_id(), hq = lane >> 5, mm = lane & 31;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float lsum = half_sum(acc.l[r]);
      const int row = 4 * hq + r;
      if (row < heads) {
        if (mm == 0) {
          m[slot * kMaxGroup + row] = acc.m[r];
          l[slot * kMaxGroup + row] = lsum;
        }
        o[(slot * kMaxGroup + row) * kHeadDim + mm] = acc.o[0][r];
        o[(slot * kMaxGroup + row) * kHeadDim + kHeadDim / 2 + mm] = acc.o[1][r];
      }
    }
  }
};
constexpr int kAttnStageFloats = kAttnSlots * kMaxGroup * (2 + kHeadDim);

// The chunk partial of head row h, output dim d, over the slots that took a
// tile (the first min(tiles, kAttnSlots)): M = max_s m_s, w_s = 2^(m_s - M)
// (zero for a slot without a tile), L = sum_s w_s l_s and A = sum_s w_s a_s,
// each sum over the rounded products (never contracted) as the pairwise tree
// ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7)). The slots' weights are
// independent, so no step waits for the previous slot's fold.
__device__ __forceinline__ void attn_slot_merge(const AttnStage &st, int tiles, int h, int d, float &M, float &L,
                                                float &A) {
  static_assert(kAttnSlots == 8, "three-level tree");
  float sm[kAttnSlots], sl[kAttnSlots], so[kAttnSlots];
#pragma unroll
  for (int w = 0; w < kAttnSlots; ++w) {
    sm[w] = st.m[w * kMaxGroup + h];
    sl[w] = st.l[w * kMaxGroup + h];
    so[w] = st.o[(w * kMaxGroup + h) * kHeadDim + d];
  }
  float mx[kAttnSlots];
#pragma unroll
  for (int w = 0; w < kAttnSlots; ++w) mx[w] = w < tiles ? sm[w] : -INFINITY;
  M = fmaxf(fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3])), fmaxf(fmaxf(mx[4], mx[5]), fmaxf(mx[6], mx[7])));
  float pl[kAttnSlots], pa[kAttnSlots];
#pragma unroll
  for (int w = 0; w < kAttnSlots; ++w) {
    const float wt = w < tiles ? exp2_fast(sm[w] - M) : 0.f;
    pl[w] = w < tiles ? __fmul_rn(wt, sl[w]) : 0.f;
    pa[w] = w < tiles ? __fmul_rn(wt, so[w]) : 0.f;
  }
  L = ((pl[0] + pl[1]) + (pl[2] + pl[3])) + ((pl[4] + pl[5]) + (pl[6] + pl[7]));
  A = ((pa[0] + pa[1]) + (pa[2] + pa[3])) + ((pa[4] + pa[5]) + (pa[6] + pa[7]));
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
