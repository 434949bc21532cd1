// GQA decode attention shared by the stream-ordered kernels and the resident
// megakernel, so both paths run the same arithmetic in the same order.
//
// Split-KV: the attended positions 0..L-1 are cut into chunks of
// attn_chunk_len(L, parts, kAttnGrain) positions (a multiple of the
// 16-position tile, at most kAttnMaxChunks chunks). A chunk of one KV group
// is one workgroup's work, computed in one of two ways fixed by the chunk
// length, so every path agrees:
//  - one block (up to 64 positions, attn_single_block): one wave per query
//    head forms the block's softmax partial on the vector ALUs
//    (attn_block_valu);
//  - longer: the chunk is cut into tiles of 16 positions, dealt round-robin
//    to kAttnSlots waves; each wave keeps an online-softmax partial of all
//    the group's heads over its tiles (scores and P.V on FP32 MFMA,
//    attn_tile), and the wave partials are folded in slot order.
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

// Positions per tile: the N (scores) and K (P.V) extent of one
// v_mfma_f32_16x16x4f32 pass. A chunk's tiles start at the chunk's first
// position; tile i of a chunk belongs to tile slot i % kAttnSlots.
constexpr int kAttnTile = 16;
// Tile slots per (chunk, KV group): the waves of one attention workgroup.
constexpr int kAttnSlots = 8;
// Probability tile of one wave in LDS: [16 heads][16 positions], rows
// padded to 17 floats so the column reads of the P.V operand do not collide.
constexpr int kAttnPsStride = 17;
constexpr int kAttnPsFloats = 16 * kAttnPsStride;

// One wave's running softmax partial over its tiles (base-2 units). Lane l
// holds query rows 4 (l / 16) + r (r = 0..3; rows past the group's heads are
// padding): max m[r], sum l[r], and o[n][r], the row's output dim 16 n + l % 16.
struct AttnAcc {
  float m[4], l[4];
  attn_f4v o[4];
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      m[r] = -INFINITY;
      l[r] = 0.f;
      o[r] = attn_f4v{0.f, 0.f, 0.f, 0.f};
    }
  }
};

// Query operand of a group of up to 16 heads: qa[s] = float4 (4 s + l / 16)
// of head l % 16's query (zero past the group's `heads`). q4(h, d4) returns
// float4 d4 of head h's query.
template <typename Q4>
__device__ __forceinline__ void attn_query(Q4 q4, int heads, float4 (&qa)[4]) {
  const int col = lane_id() & 15, quad = lane_id() >> 4;
#pragma unroll
  for (int s = 0; s < 4; ++s) qa[s] = col < heads ? q4(col, 4 * s + quad) : make_float4(0.f, 0.f, 0.f, 0.f);
}

// Component c of a float4.
__device__ __forceinline__ float attn_c(float4 v, int c) { return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w; }

// One tile of 16 positions [t0, t0 + 16) for every head of a KV group, on
// MFMA (the group's heads are the M rows, padded to 16; K and V are read
// once for all of them). Positions >= end are masked: their score is -inf
// and their K/V reads take position end - 1, so no value read past the
// context reaches the sums. k4(pos, d4): float4 d4 of position pos's K row;
// v(pos, d): element d of its V row; ps: this wave's kAttnPsFloats of LDS.
//   S[h][j] = q_h . k_j over 64 dims: 16 MFMAs in four chains, chain s
//             taking dims 16 s + 4 (l / 16) + c of lane l at its k-step c
//             (c = 0..3), the chains summed as (s0 + s1) + (s2 + s3);
//             scaled into base-2 units by kScoreScaleLog2;
//   online softmax per row: m' = max(m, row16_max of the tile), c =
//             2^(m - m') (0 for the first tile), p = 2^(s - m'),
//             l = l c + row16_sum(p), o = o c (rounded products);
//   o += P . V: k-step s covers positions 4 s .. 4 s + 3, N tile n dims
//             16 n .. 16 n + 15 (16 MFMAs).
// The four rows' reductions go step by step together, so their exchanges
// interleave. The resident kernel and the stream-ordered kernel both run
// it, so their partials are bit-identical.
template <typename K4, typename V>
__device__ __forceinline__ void attn_tile(const float4 (&qa)[4], K4 k4, V v, float *ps, int t0, int end,
                                          AttnAcc &acc) {
  const int lane = lane_id(), col = lane & 15, quad = lane >> 4;
  const int pk = min(t0 + col, end - 1);
  float4 kb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) kb[s] = k4(pk, 4 * s + quad);
  float vb[4][4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int pv = min(t0 + 4 * s + quad, end - 1);
#pragma unroll
    for (int n = 0; n < 4; ++n) vb[s][n] = v(pv, 16 * n + col);
  }
  attn_f4v sp[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) sp[s] = attn_f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int s = 0; s < 4; ++s)
      sp[s] = __builtin_amdgcn_mfma_f32_16x16x4f32(attn_c(qa[s], c), attn_c(kb[s], c), sp[s], 0, 0, 0);
  }
  const attn_f4v sc = (sp[0] + sp[1]) + (sp[2] + sp[3]);
  const bool valid = t0 + col < end;
  float x[4], mx[4], cr[4], p[4], sm[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) x[r] = valid ? __fmul_rn(sc[r], kScoreScaleLog2) : -INFINITY;
  // row16_max of each row, then with the running max.
#pragma unroll
  for (int r = 0; r < 4; ++r) mx[r] = fmaxf(x[r], dpp<kDppXor1>(x[r]));
#pragma unroll
  for (int r = 0; r < 4; ++r) mx[r] = fmaxf(mx[r], dpp<kDppXor2>(mx[r]));
#pragma unroll
  for (int r = 0; r < 4; ++r) mx[r] = fmaxf(mx[r], dpp<kDppHalfMirror>(mx[r]));
#pragma unroll
  for (int r = 0; r < 4; ++r) mx[r] = fmaxf(acc.m[r], fmaxf(mx[r], dpp<kDppMirror>(mx[r])));
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    cr[r] = acc.m[r] == -INFINITY ? 0.f : exp2_fast(acc.m[r] - mx[r]);
    p[r] = exp2_fast(x[r] - mx[r]);
    ps[(4 * quad + r) * kAttnPsStride + col] = p[r];
  }
  // row16_sum of each row's probabilities.
#pragma unroll
  for (int r = 0; r < 4; ++r) sm[r] = p[r] + dpp<kDppXor1>(p[r]);
#pragma unroll
  for (int r = 0; r < 4; ++r) sm[r] += dpp<kDppXor2>(sm[r]);
#pragma unroll
  for (int r = 0; r < 4; ++r) sm[r] += dpp<kDppHalfMirror>(sm[r]);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    sm[r] += dpp<kDppMirror>(sm[r]);
    acc.l[r] = fmaf(acc.l[r], cr[r], sm[r]);
    acc.m[r] = mx[r];
#pragma unroll
    for (int n = 0; n < 4; ++n) acc.o[n][r] = __fmul_rn(acc.o[n][r], cr[r]);
  }
  // Lanes read each other's probabilities: order the wave's LDS writes.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const float a = ps[col * kAttnPsStride + 4 * s + quad];
#pragma unroll
    for (int n = 0; n < 4; ++n) acc.o[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vb[s][n], acc.o[n], 0, 0, 0);
  }
  // The next tile rewrites ps only after every lane has read it.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Two tiles [ta, ta + 16) and [tb, tb + 16) of one wave taken together, as
// one online-softmax step over both (their chains interleave): S of each
// tile as in attn_tile; m' = max(m, max(tile a max, tile b max)); c and p as
// in attn_tile; l = l c + (row16_sum(p_a) + row16_sum(p_b)); o = o c, then
// o += P_a . V_a, then P_b . V_b. ps: one probability tile, as attn_tile's.
template <typename K4, typename V>
__device__ __forceinline__ void attn_tile2(const float4 (&qa)[4], K4 k4, V v, float *ps, int ta, int tb, int end,
                                           AttnAcc &acc) {
  const int lane = lane_id(), col = lane & 15, quad = lane >> 4;
  const int t0[2] = {ta, tb};
  float4 kb[2][4];
  float vb[2][4][4];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int pk = min(t0[u] + col, end - 1);
#pragma unroll
    for (int s = 0; s < 4; ++s) kb[u][s] = k4(pk, 4 * s + quad);
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int pv = min(t0[u] + 4 * s + quad, end - 1);
#pragma unroll
      for (int n = 0; n < 4; ++n) vb[u][s][n] = v(pv, 16 * n + col);
    }
  }
  attn_f4v sp[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int s = 0; s < 4; ++s) sp[u][s] = attn_f4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int u = 0; u < 2; ++u)
        sp[u][s] = __builtin_amdgcn_mfma_f32_16x16x4f32(attn_c(qa[s], c), attn_c(kb[u][s], c), sp[u][s], 0, 0, 0);
    }
  }
  float x[2][4], mx[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const attn_f4v sc = (sp[u][0] + sp[u][1]) + (sp[u][2] + sp[u][3]);
    const bool valid = t0[u] + col < end;
#pragma unroll
    for (int r = 0; r < 4; ++r) x[u][r] = valid ? __fmul_rn(sc[r], kScoreScaleLog2) : -INFINITY;
  }
  // row16_max of each row of both tiles, step by step.
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx[u][r] = fmaxf(x[u][r], dpp<kDppXor1>(x[u][r]));
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx[u][r] = fmaxf(mx[u][r], dpp<kDppXor2>(mx[u][r]));
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx[u][r] = fmaxf(mx[u][r], dpp<kDppHalfMirror>(mx[u][r]));
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) mx[u][r] = fmaxf(mx[u][r], dpp<kDppMirror>(mx[u][r]));
  float mn[4], cr[4], p[2][4], sm[2][4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    mn[r] = fmaxf(acc.m[r], fmaxf(mx[0][r], mx[1][r]));
    cr[r] = acc.m[r] == -INFINITY ? 0.f : exp2_fast(acc.m[r] - mn[r]);
  }
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) p[u][r] = exp2_fast(x[u][r] - mn[r]);
  // The A operands of both tiles through the one probability tile: tile a's
  // written and read, then tile b's.
  float pa[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int r = 0; r < 4; ++r) ps[(4 * quad + r) * kAttnPsStride + col] = p[u][r];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int s = 0; s < 4; ++s) pa[u][s] = ps[col * kAttnPsStride + 4 * s + quad];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // row16_sum of each row's probabilities of both tiles.
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm[u][r] = p[u][r] + dpp<kDppXor1>(p[u][r]);
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm[u][r] += dpp<kDppXor2>(sm[u][r]);
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm[u][r] += dpp<kDppHalfMirror>(sm[u][r]);
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm[u][r] += dpp<kDppMirror>(sm[u][r]);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    acc.l[r] = fmaf(acc.l[r], cr[r], sm[0][r] + sm[1][r]);
    acc.m[r] = mn[r];
#pragma unroll
    for (int n = 0; n < 4; ++n) acc.o[n][r] = __fmul_rn(acc.o[n][r], cr[r]);
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int n = 0; n < 4; ++n)
        acc.o[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[u][s], vb[u][s][n], acc.o[n], 0, 0, 0);
    }
  }
}

// The tiles of slot `slot` that lie in [wb, we) of a chunk starting at
// `begin` (wb - begin a multiple of 2 kAttnSlots tiles), in position order:
// tiles t and t + kAttnSlots together (attn_tile2) while both exist, a last
// single one alone (attn_tile).
template <typename K4, typename V>
__device__ __forceinline__ void attn_slot_tiles(const float4 (&qa)[4], K4 k4, V v, float *ps, int begin,
                                                int wb, int we, int end, int slot, AttnAcc &acc) {
  const int t_lo = (wb - begin) / kAttnTile, t_hi = (we - begin + kAttnTile - 1) / kAttnTile;
  for (int t = t_lo + slot; t < t_hi; t += 2 * kAttnSlots) {
    if (t + kAttnSlots < t_hi)
      attn_tile2(qa, k4, v, ps, begin + t * kAttnTile, begin + (t + kAttnSlots) * kAttnTile, end, acc);
    else
      attn_tile(qa, k4, v, ps, begin + t * kAttnTile, end, acc);
  }
}

// Wave partials of a chunk staged for the merge: [slot][row] maxima and
// sums, [slot][row][64] outputs, for the group's first `heads` rows.
struct AttnStage {
  float *m, *l, *o;  // m, l: kAttnSlots * kMaxGroup floats; o: kAttnSlots * kMaxGroup * 64
  __device__ __forceinline__ void put(int slot, int heads, const AttnAcc &acc) const {
    const int lane = lane_id(), col = lane & 15, quad = lane >> 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * quad + r;
      if (row < heads) {
        if (col == 0) {
          m[slot * kMaxGroup + row] = acc.m[r];
          l[slot * kMaxGroup + row] = acc.l[r];
        }
#pragma unroll
        for (int n = 0; n < 4; ++n) o[(slot * kMaxGroup + row) * kHeadDim + 16 * n + col] = acc.o[n][r];
      }
    }
  }
};
constexpr int kAttnStageFloats = kAttnSlots * kMaxGroup * (2 + kHeadDim);

// The chunk partial of head row h, output dim d: the slots that took a tile
// (the first min(tiles, kAttnSlots)) folded in slot order (attn_fold). All
// slots' values are read before the first fold.
__device__ __forceinline__ void attn_slot_merge(const AttnStage &st, int tiles, int h, int d, float &M, float &L,
                                                float &A) {
  float sm[kAttnSlots], sl[kAttnSlots], so[kAttnSlots];
#pragma unroll
  for (int w = 0; w < kAttnSlots; ++w) {
    sm[w] = st.m[w * kMaxGroup + h];
    sl[w] = st.l[w * kMaxGroup + h];
    so[w] = st.o[(w * kMaxGroup + h) * kHeadDim + d];
  }
  M = -INFINITY;
  L = 0.f;
  A = 0.f;
#pragma unroll
  for (int w = 0; w < kAttnSlots; ++w)
    if (w < tiles) attn_fold(sm[w], sl[w], so[w], M, L, A);
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
