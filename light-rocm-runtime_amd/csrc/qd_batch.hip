// Batched decode step for gfx950: up to 16 independent sequences with
// ragged KV lengths advance one token together.
//
// Projections are skinny GEMMs D[seq][row] = sum_k X[seq][k] W[row][k] on
// v_mfma_f32_16x16x4f32: the (up to) 16 sequences are the M dimension and a
// 16-row tile of the weight matrix is N. Lane l of a wave supplies
// A[l % 16][l / 16] and B[l / 16][l % 16] and result register r holds
// D[(l / 16) * 4 + r][l % 16]; so lane l streams weight row (l % 16) of the
// tile in float4 loads at k offset 4 * (l / 16) of each 16-wide k step and
// multiplies it with the same k offsets of sequence (l % 16)'s operand row.
// Each weight is read from HBM once per step for the whole batch. The waves
// of a workgroup split K; their partial tiles are summed in LDS in a fixed
// order and the 256 tile elements go through the fused epilogue (bias,
// RoPE + KV write, residual add, SiLU gate, logits + top-1).
//
// Semantics per sequence are those of the batch-1 step (qd_kernels.hip):
//   RMSNorm                 benchmarks/qwen_stateful_graph_kernel.cpp:665-701
//   QKV + bias, RoPE, KV    benchmarks/qwen_stateful_graph_kernel.cpp:392-552
//   GQA attention           benchmarks/qwen_stateful_graph_kernel.cpp:554-600
//   O / gate-up / down      benchmarks/qwen_stateful_graph_kernel.cpp:158-223,494-515,602-659
//   LM head + top-1         benchmarks/qwen_stateful_graph_kernel.cpp:225-356
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <mutex>

#include "qd_attention.hpp"
#include "qd_batch.hpp"
#include "qd_device.hpp"
#include "qd_device_math.hpp"

namespace qd {
namespace {

using namespace dev;

typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kH = 896;    // hidden = query width
constexpr int kI = 4864;   // MLP intermediate
constexpr int kStep = 16;  // k values one float4 load per lane covers per wave

__device__ __forceinline__ int tile_col() { return lane_id() & 15; }     // N index (weight row)
__device__ __forceinline__ int k_quad() { return (lane_id() >> 4) * 4; }  // k offset in a step

__device__ __forceinline__ float4 ld4(const float *p) {
  return *reinterpret_cast<const float4 *>(p);
}

__device__ __forceinline__ f4v mfma4(float4 a, float4 b, f4v acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, b.x, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, b.y, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, b.z, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, b.w, acc, 0, 0, 0);
  return acc;
}

// The raw operand slice of this lane for kSteps k-steps from kbase:
// sequence row (lane % 16) of x (K floats per row), zero for rows >= rows.
template <int kSteps, int K>
__device__ __forceinline__ void load_operand(const float *__restrict__ x, int rows, int kbase,
                                             float4 (&xa)[kSteps]) {
  const int b = tile_col();
  const int k0 = kbase + k_quad();
  const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
  if (b >= rows) {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) xa[s] = zero;
    return;
  }
  const float *row = x + static_cast<size_t>(b) * K;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) xa[s] = ld4(row + k0 + kStep * s);
}

// The gain slice matching load_operand's k offsets.
template <int kSteps>
__device__ __forceinline__ void load_gain(int kbase, const float *__restrict__ gain,
                                          float4 (&gv)[kSteps]) {
  const int k0 = kbase + k_quad();
#pragma unroll
  for (int s = 0; s < kSteps; ++s) gv[s] = ld4(gain + k0 + kStep * s);
}

// RMSNorm folded into the GEMM: y = x * inv * g gives W.y = inv * W.(x g),
// so the matrix cores take x * g and the epilogue scales by the row's inv.
// Returns this lane's contribution to the sum of squares of its row and
// scales the slice by the gain in place.
template <int kSteps>
__device__ __forceinline__ float gain_operand(const float4 (&gv)[kSteps], float4 (&xa)[kSteps]) {
  float ss = 0.f;
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const float4 g = gv[s];
    float4 &x = xa[s];
    ss = fmaf(x.x, x.x, ss);
    ss = fmaf(x.y, x.y, ss);
    ss = fmaf(x.z, x.z, ss);
    ss = fmaf(x.w, x.w, ss);
    x = make_float4(x.x * g.x, x.y * g.y, x.z * g.z, x.w * g.w);
  }
  return ss;
}

// Sums each row's squares over the workgroup's waves: lanes b, b + 16,
// b + 32, b + 48 of every wave hold row b's pieces. ss[b] receives the sum.
// Ends with a workgroup barrier.
__device__ __forceinline__ void rows_sum_squares(float part, float (*wss)[16], float *ss) {
  part += __shfl_xor(part, 16, kWave);
  part += __shfl_xor(part, 32, kWave);
  if (lane_id() < 16) wss[wave_id()][lane_id()] = part;
  __syncthreads();
  const int waves = blockDim.x / kWave;
  if (threadIdx.x < 16) {
    float t = 0.f;
    for (int w = 0; w < waves; ++w) t += wss[w][threadIdx.x];
    ss[threadIdx.x] = t;
  }
  __syncthreads();
}

// This lane's weight slice for kSteps k-steps from kbase of row wrow (K
// floats per row): float4 s at k = kbase + 16 s + 4 (lane / 16).
template <int kSteps>
__device__ __forceinline__ void load_weights(const float *__restrict__ wrow, int kbase,
                                             float4 (&wv)[kSteps]) {
  const int k0 = kbase + k_quad();
#pragma unroll
  for (int s = 0; s < kSteps; ++s)
    wv[s] = ld_weight(reinterpret_cast<const float4 *>(wrow + k0 + kStep * s));
}

// acc += X[:, k slice] . W[row, k slice]^T from the loaded slices.
template <int kSteps>
__device__ __forceinline__ f4v tile_mfma(const float4 (&xa)[kSteps], const float4 (&wv)[kSteps],
                                         f4v acc) {
#pragma unroll
  for (int s = 0; s < kSteps; ++s) acc = mfma4(xa[s], wv[s], acc);
  return acc;
}

// Keeps the compiler from moving any instruction across this point: placed
// after a kernel's loads so all of them are in flight before the first wait.
__device__ __forceinline__ void issue_fence() { __builtin_amdgcn_sched_barrier(0); }

// Sums the waves' partial tiles: red is [waves][4][64]; thread t < 256
// returns element (register t / 64, lane t % 64), i.e. sequence
// ((t % 64) / 16) * 4 + t / 64 and tile column t % 16. Starts and ends
// with a workgroup barrier.
template <int kWaves>
__device__ __forceinline__ float tile_reduce(f4v acc, float (*red)[4][kWave]) {
  const int w = wave_id(), l = lane_id();
#pragma unroll
  for (int r = 0; r < 4; ++r) red[w][r][l] = acc[r];
  __syncthreads();
  float v = 0.f;
  const int t = threadIdx.x;
  if (t < 4 * kWave) {
#pragma unroll
    for (int u = 0; u < kWaves; ++u) v += red[u][t >> 6][t & 63];
  }
  __syncthreads();
  return v;
}

__device__ __forceinline__ int tile_seq(int t) { return ((t & 63) >> 4) * 4 + (t >> 6); }

// Waits until this thread's vector memory operations have completed (gfx9
// s_waitcnt encoding: vmcnt 0, expcnt and lgkmcnt not waited on).
__device__ __forceinline__ void wait_vm_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Split-K over workgroups: workgroup blockIdx.y of `splits` deposits its
// partial tile (thread t < 256 holds element t) and, with kSsq, its row
// sums of squares ss[0..16); the last workgroup of the tile to arrive sums
// the deposits in split order (deterministic) into v and ss, resets the
// tile's counter and returns true. Other workgroups return false. Deposits
// use device-scope (sc1) stores and loads, which are coherent across the
// XCDs' L2s without an L2 writeback or invalidate; each depositing thread
// waits for its stores to complete before the workgroup's arrival is counted.
constexpr int kSplitRec = 256 + 16;
template <int kSplits, bool kSsq>
__device__ bool split_gather(float &v, float *ss, float *__restrict__ ws, uint32_t *cnt, int tile) {
  __shared__ uint32_t last;
  constexpr int splits = kSplits;
  const int t = threadIdx.x;
  if (splits == 1) return true;
  const Coherent dep(ws + static_cast<size_t>(tile) * splits * kSplitRec,
                     static_cast<uint32_t>(splits * kSplitRec * sizeof(float)));
  const uint32_t mine = blockIdx.y * kSplitRec;
  if (t < 256) dep.st(mine + t, v);
  if (kSsq && t < 16) dep.st(mine + 256 + t, ss[t]);
  wait_vm_stores();
  __syncthreads();
  if (t == 0) last = atomicAdd(cnt + tile, 1u) == static_cast<uint32_t>(splits - 1);
  __syncthreads();
  if (!last) return false;
  // All deposits are requested before any is summed (one round trip).
  float pv[kSplits], pq[kSplits];
#pragma unroll
  for (int s = 0; s < kSplits; ++s) {
    pv[s] = t < 256 ? dep.ld(s * kSplitRec + t) : 0.f;
    pq[s] = kSsq && t < 16 ? dep.ld(s * kSplitRec + 256 + t) : 0.f;
  }
  float sum = 0.f, sq = 0.f;
#pragma unroll
  for (int s = 0; s < kSplits; ++s) {
    sum += pv[s];
    sq += pq[s];
  }
  v = sum;
  if (kSsq) {
    __syncthreads();
    if (t < 16) ss[t] = sq;
    __syncthreads();
  }
  if (t == 0) cnt[tile] = 0u;
  return true;
}

// Counter regions of BatchLaunch::counters.
constexpr int kCntQkv = 0, kCntO = 128, kCntDown = 256, kCntAttn = 512;

__device__ __forceinline__ float *kv_rows(float *cache, uint32_t slot, int layer, int layers,
                                          int capacity, int kv_dim) {
  return cache + (static_cast<size_t>(slot) * layers + layer) * capacity * kv_dim;
}

// ---- kernels --------------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void batch_embed_kernel(BatchLaunch p,
                                                             const float *__restrict__ emb,
                                                             int vocab) {
  const int b = blockIdx.x;
  const uint32_t tok = p.token[b];
  if (tok >= static_cast<uint32_t>(vocab)) return;
  const float *src = emb + static_cast<size_t>(tok) * kH;
  for (int i = threadIdx.x; i < kH; i += kBlock) p.hidden[b * kH + i] = src[i];
}

// Attention RMSNorm + packed QKV + bias + RoPE + KV-cache write. Tile
// blockIdx.x holds, for head T / 4 and i0 = 8 * (T % 4), the rows
// head*64 + i0 + j and head*64 + 32 + i0 + j (j < 8) as tile columns j and
// j + 8: the rotate-half partners sit in lanes l and l ^ 8. Heads [0, nq)
// are queries, then nkv keys, then nkv values (not rotated). K = 896 is
// split over kQkvSplit workgroups of four waves (two: 144 workgroups instead
// of 72, 9.8 against 10.6 us per layer in a same-box A/B).
#ifndef QD_BATCH_QKV_SPLIT
#define QD_BATCH_QKV_SPLIT 2
#endif
constexpr int kQkvSplit = QD_BATCH_QKV_SPLIT;
__global__ __launch_bounds__(kBlock) void batch_qkv_kernel(BatchLaunch p, const float *__restrict__ gain,
                                                           const float *__restrict__ wqkv,
                                                           const float *__restrict__ bqkv, int layer) {
  constexpr int kSteps = kH / kStep / kWavesPerBlock / kQkvSplit;  // 7
  __shared__ float wss[kWavesPerBlock][16];
  __shared__ float ss[16];
  __shared__ float red[kWavesPerBlock][4][kWave];
  const int tile = blockIdx.x;
  const int head = tile >> 2;
  const int i0 = (tile & 3) * 8;
  const int kbase = (blockIdx.y * kWavesPerBlock + wave_id()) * kSteps * kStep;
  const int j = tile_col();
  const int wrow = head * kHeadDim + (j < 8 ? i0 + j : kRotary + i0 + j - 8);
  // Epilogue element of this thread: its bias and rotation are requested
  // with the weights.
  const int t = threadIdx.x;
  const int seq = tile_seq(t);
  const int jt = t & 15;
  const int i = i0 + (jt & 7);
  const int row = head * kHeadDim + (jt < 8 ? i : kRotary + i);
  const int pos = static_cast<int>(p.pos[min(seq, p.rows - 1)]);
  const float bias = bqkv[row];
  const float c = p.rope_cos[pos * kRotary + i];
  const float s = p.rope_sin[pos * kRotary + i];
  float4 wv[kSteps], xa[kSteps];
  load_weights<kSteps>(wqkv + static_cast<size_t>(wrow) * kH, kbase, wv);
  float4 gv[kSteps];
  load_operand<kSteps, kH>(p.hidden, p.rows, kbase, xa);
  load_gain<kSteps>(kbase, gain, gv);
  issue_fence();
  const float part = gain_operand<kSteps>(gv, xa);
  f4v acc = {0.f, 0.f, 0.f, 0.f};
  acc = tile_mfma<kSteps>(xa, wv, acc);
  rows_sum_squares(part, wss, ss);
  float v = tile_reduce<kWavesPerBlock>(acc, red);
  if (!split_gather<kQkvSplit, true>(v, ss, p.split, p.counters + kCntQkv, tile)) return;
  // Epilogue over the 256 tile elements.
  const float v0 = v;
  v = v0 * rsqrtf(ss[seq] / static_cast<float>(kH) + p.eps) + bias;
  const float other = __shfl_xor(v, 8, kWave);
  if (seq >= p.rows) return;
  const uint32_t slot = p.slot[seq];
  const int kv_dim = p.nkv * kHeadDim;
  const int d = row - head * kHeadDim;
  if (head < p.nq + p.nkv) {
    // (a, b) = (row i, row i + 32): a' = a c - b s, b' = b c + a s.
    const float out = jt < 8 ? v * c - other * s : v * c + other * s;
    if (head < p.nq) {
      p.q[seq * (p.nq * kHeadDim) + row] = out;
    } else {
      float *kc = kv_rows(p.k_cache, slot, layer, p.layers, p.capacity, kv_dim);
      kc[static_cast<size_t>(pos) * kv_dim + (head - p.nq) * kHeadDim + d] = out;
    }
  } else {
    float *vc = kv_rows(p.v_cache, slot, layer, p.layers, p.capacity, kv_dim);
    vc[static_cast<size_t>(pos) * kv_dim + (head - p.nq - p.nkv) * kHeadDim + d] = v;
  }
}

// Sum / max over the 16 lanes of a DPP row (lanes 16q .. 16q+15); every
// lane of the row receives the result.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  return v;
}

// GQA decode attention on the matrix cores: workgroup (chunk, KV group g,
// batch row b) serves all query heads of the group (up to 16), so every K/V
// row of the chunk is read once. Waves take 16-position tiles (wave w: tile
// w of each 64-position pass). Per tile:
//   S[head][pos] = (Q / 8) . K^T    16x16x4 MFMAs, lane l supplies
//                                   Q[head l%16] and K[pos l%16] at dims
//                                   16 s + 4 (l/16) + c (float4 loads)
//   online softmax per head row     (S register r of lane l is head
//                                   4 (l/16) + r, position l%16: row
//                                   reductions over the 16-lane DPP rows)
//   O[head][d] += P . V             P and the V tile go through the wave's
//                                   LDS to become MFMA A / B operands.
// The four wave partials are merged into one record (m, l, acc[64]) per
// head; the last chunk of (b, g) to finish merges all chunks (the same
// merge as attn_merge) into attn[b][h*64 + d]. Q is scaled by
// kScoreScaleLog2 = log2(e) / sqrt(64), so scores and maxima are in base-2
// units and every softmax exponential is one v_exp_f32 (2^x).
struct GqaLds {
  float ps[kWavesPerBlock][16][17];   // P tile [head][pos]
  float vs[kWavesPerBlock][16][68];   // V tile [pos][dim]
  float wm[kWavesPerBlock][16];
  float wl[kWavesPerBlock][16];
  float wo[kWavesPerBlock][16][65];   // wave partial O [head][dim]
};

__global__ __launch_bounds__(kBlock) void batch_attn_kernel(BatchLaunch p, int layer) {
  __shared__ GqaLds sh;
  __shared__ uint32_t last;
  const int b = blockIdx.z, g = blockIdx.y, chunk = blockIdx.x;
  const uint32_t slot = p.slot[b];
  const int position = static_cast<int>(p.pos[b]);
  const int length = position + 1;
  const int chunks = attn_chunks(length);
  if (chunk >= chunks) return;
  const int chunk_len = attn_chunk_len(length);
  const int begin = chunk * chunk_len;
  const int end = min(length, begin + chunk_len);
  const int group = p.nq / p.nkv;
  const int kv_dim = p.nkv * kHeadDim;
  const float *kb = kv_rows(p.k_cache, slot, layer, p.layers, p.capacity, kv_dim) + g * kHeadDim;
  const float *vb = kv_rows(p.v_cache, slot, layer, p.layers, p.capacity, kv_dim) + g * kHeadDim;
  const int w = wave_id(), col = tile_col(), quad = lane_id() >> 4;
  const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);

  float4 qa[4];
  if (col < group) {
    const float *qr = p.q + b * (p.nq * kHeadDim) + (g * group + col) * kHeadDim + 4 * quad;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float4 v = ld4(qr + 16 * s);
      qa[s] = make_float4(v.x * kScoreScaleLog2, v.y * kScoreScaleLog2, v.z * kScoreScaleLog2,
                          v.w * kScoreScaleLog2);
    }
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) qa[s] = zero;
  }
  auto load_tile = [&](int p0, float4 (&kr)[4], float4 (&vr)[4]) {
    const int pos = p0 + col;
    if (pos < end) {
      const size_t off = static_cast<size_t>(pos) * kv_dim + 4 * quad;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        kr[s] = ld4(kb + off + 16 * s);
        vr[s] = ld4(vb + off + 16 * s);
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) kr[s] = vr[s] = zero;
    }
  };

  float m[4], lsum[4];
  f4v o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m[r] = -INFINITY;
    lsum[r] = 0.f;
    o[r] = f4v{0.f, 0.f, 0.f, 0.f};
  }
  float4 kc[4], vc[4];
  load_tile(begin + 16 * w, kc, vc);
  for (int base = begin; base < end; base += kAttnPass) {
    const int p0 = base + 16 * w;
    float4 kn[4], vn[4];
    if (base + kAttnPass < end) load_tile(p0 + kAttnPass, kn, vn);
#pragma unroll
    for (int s = 0; s < 4; ++s)
      *reinterpret_cast<float4 *>(&sh.vs[w][col][16 * s + 4 * quad]) = vc[s];
    f4v sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) sacc = mfma4(qa[s], kc[s], sacc);
    const bool valid = p0 + col < end;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float sv = valid ? sacc[r] : -INFINITY;
      const float mn = fmaxf(m[r], row16_max(sv));
      const float pv = mn == -INFINITY ? 0.f : exp2_fast(sv - mn);
      const float corr = mn == -INFINITY ? 1.f : exp2_fast(m[r] - mn);
      lsum[r] = fmaf(lsum[r], corr, row16_sum(pv));
      m[r] = mn;
#pragma unroll
      for (int n = 0; n < 4; ++n) o[n][r] *= corr;
      sh.ps[w][4 * quad + r][col] = pv;
    }
    // The wave's own LDS tiles: LDS operations of a wave complete in order.
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float a = sh.ps[w][col][4 * s + quad];
#pragma unroll
      for (int n = 0; n < 4; ++n)
        o[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, sh.vs[w][4 * s + quad][16 * n + col], o[n],
                                                     0, 0, 0);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      kc[s] = kn[s];
      vc[s] = vn[s];
    }
  }
  // Wave partials -> one record per head of the group.
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if (col == 0) {
      sh.wm[w][4 * quad + r] = m[r];
      sh.wl[w][4 * quad + r] = lsum[r];
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) sh.wo[w][4 * quad + r][16 * n + col] = o[n][r];
  }
  __syncthreads();
  const Coherent recs(p.part + (static_cast<size_t>(b) * p.nq + g * group) * kAttnMaxChunks * kPartStride,
                      group * kAttnMaxChunks * kPartStride * sizeof(float));
  for (int i = threadIdx.x; i < group * kHeadDim; i += kBlock) {
    const int h = i / kHeadDim, d = i % kHeadDim;
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < kWavesPerBlock; ++v) mx = fmaxf(mx, sh.wm[v][h]);
    float lt = 0.f, a = 0.f;
#pragma unroll
    for (int v = 0; v < kWavesPerBlock; ++v) {
      const float f = sh.wm[v][h] == -INFINITY ? 0.f : exp2_fast(sh.wm[v][h] - mx);
      lt = fmaf(f, sh.wl[v][h], lt);
      a = fmaf(f, sh.wo[v][h][d], a);
    }
    const uint32_t rec = (h * kAttnMaxChunks + chunk) * kPartStride;
    recs.st(rec + 2 + d, a);
    if (d == 0) {
      recs.st(rec, mx);
      recs.st(rec + 1, lt);
    }
  }
  wait_vm_stores();
  __syncthreads();
  uint32_t *cnt = p.counters + kCntAttn + b * p.nkv + g;
  if (threadIdx.x == 0) last = atomicAdd(cnt, 1u) == static_cast<uint32_t>(chunks - 1);
  __syncthreads();
  if (!last) return;
  for (int i = threadIdx.x; i < group * kHeadDim; i += kBlock) {
    const int h = i / kHeadDim, d = i % kHeadDim;
    const uint32_t head_rec = h * kAttnMaxChunks * kPartStride;
    // Every chunk's (m, l, acc_d) is requested before any is used.
    float cm[kAttnMaxChunks], cl[kAttnMaxChunks], ca[kAttnMaxChunks];
#pragma unroll
    for (int c = 0; c < kAttnMaxChunks; ++c) {
      const uint32_t rec = head_rec + c * kPartStride;
      const bool in = c < chunks;
      cm[c] = in ? recs.ld(rec) : -INFINITY;
      cl[c] = in ? recs.ld(rec + 1) : 0.f;
      ca[c] = in ? recs.ld(rec + 2 + d) : 0.f;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int c = 0; c < kAttnMaxChunks; ++c) mx = fmaxf(mx, cm[c]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int c = 0; c < kAttnMaxChunks; ++c) {
      const float f = c < chunks ? exp2_fast(cm[c] - mx) : 0.f;
      den = fmaf(f, cl[c], den);
      num = fmaf(f, ca[c], num);
    }
    p.attn[b * (p.nq * kHeadDim) + (g * group + h) * kHeadDim + d] = num / den;
  }
  if (threadIdx.x == 0) *cnt = 0u;
}

// hidden[b][row] += Wo[row] . attn[b] for the 16 rows of tile blockIdx.x;
// K = 896 split over kOSplit workgroups (two: 112 workgroups instead of 56,
// 8.0 against 8.8 us per layer in a same-box A/B).
#ifndef QD_BATCH_O_SPLIT
#define QD_BATCH_O_SPLIT 2
#endif
constexpr int kOSplit = QD_BATCH_O_SPLIT;
__global__ __launch_bounds__(kBlock) void batch_oproj_kernel(BatchLaunch p,
                                                             const float *__restrict__ wo) {
  constexpr int kSteps = kH / kStep / kWavesPerBlock / kOSplit;  // 7
  __shared__ float red[kWavesPerBlock][4][kWave];
  const int tile = blockIdx.x;
  const int n0 = tile * 16;
  const int kbase = (blockIdx.y * kWavesPerBlock + wave_id()) * kSteps * kStep;
  float4 wv[kSteps], xa[kSteps];
  load_weights<kSteps>(wo + static_cast<size_t>(n0 + tile_col()) * kH, kbase, wv);
  load_operand<kSteps, kH>(p.attn, p.rows, kbase, xa);
  issue_fence();
  f4v acc = {0.f, 0.f, 0.f, 0.f};
  acc = tile_mfma<kSteps>(xa, wv, acc);
  float v = tile_reduce<kWavesPerBlock>(acc, red);
  if (!split_gather<kOSplit, false>(v, nullptr, p.split, p.counters + kCntO, tile)) return;
  const int t = threadIdx.x;
  const int seq = tile_seq(t);
  if (seq < p.rows) p.hidden[seq * kH + n0 + (t & 15)] += v;
}

// MLP RMSNorm + gate/up + SiLU: act[b][row] = silu(g) * u. Tile blockIdx.x
// covers rows n0 .. n0 + 7 of the activation: tile column j < 8 is gate row
// n0 + j and column j + 8 the up row n0 + j, so each lane streams one weight
// row and the 608 tiles (of 57 KB each) spread evenly over the CUs. The up
// sum crosses to its gate lane (column j + 8 -> j) by a lane exchange.
__global__ __launch_bounds__(kBlock) void batch_gateup_kernel(BatchLaunch p,
                                                              const float *__restrict__ gain,
                                                              const float *__restrict__ wg,
                                                              const float *__restrict__ wu) {
  constexpr int kSteps = kH / kStep / kWavesPerBlock;  // 14
  __shared__ float wss[kWavesPerBlock][16];
  __shared__ float ss[16];
  __shared__ float red[kWavesPerBlock][4][kWave];
  const int n0 = blockIdx.x * 8;
  const int kbase = wave_id() * kSteps * kStep;
  const int col = tile_col();
  const float *wrow = (col < 8 ? wg : wu) + static_cast<size_t>(n0 + (col & 7)) * kH;
  float4 wv[kSteps], xa[kSteps];
  load_weights<kSteps>(wrow, kbase, wv);
  float4 gv[kSteps];
  load_operand<kSteps, kH>(p.hidden, p.rows, kbase, xa);
  load_gain<kSteps>(kbase, gain, gv);
  issue_fence();
  const float part = gain_operand<kSteps>(gv, xa);
  f4v acc = {0.f, 0.f, 0.f, 0.f};
  acc = tile_mfma<kSteps>(xa, wv, acc);
  rows_sum_squares(part, wss, ss);
  const float v = tile_reduce<kWavesPerBlock>(acc, red);
  // Thread t < 256 holds (sequence tile_seq(t), column t & 15); its partner
  // column t ^ 8 sits in lane (t ^ 8) of the same wave.
  const float other = __shfl_xor(v, 8, kWave);
  const int t = threadIdx.x;
  const int seq = tile_seq(t);
  if (t < 4 * kWave && (t & 15) < 8 && seq < p.rows) {
    const float inv = rsqrtf(ss[seq] / static_cast<float>(kH) + p.eps);
    const float g = v * inv, u = other * inv;
    p.act[seq * kI + n0 + (t & 7)] = g / (1.f + expf(-g)) * u;
  }
}

// hidden[b][row] += Wd[row] . act[b]; K = 4864 split over kDownSplit
// workgroups of four waves.
constexpr int kDownSplit = 4;
__global__ __launch_bounds__(kBlock) void batch_down_kernel(BatchLaunch p,
                                                            const float *__restrict__ wd) {
  constexpr int kSteps = kI / kStep / kWavesPerBlock / kDownSplit;  // 19
  __shared__ float red[kWavesPerBlock][4][kWave];
  const int tile = blockIdx.x;
  const int n0 = tile * 16;
  const int kbase = (blockIdx.y * kWavesPerBlock + wave_id()) * kSteps * kStep;
  float4 wv[kSteps], xa[kSteps];
  load_weights<kSteps>(wd + static_cast<size_t>(n0 + tile_col()) * kI, kbase, wv);
  load_operand<kSteps, kI>(p.act, p.rows, kbase, xa);
  issue_fence();
  f4v acc = {0.f, 0.f, 0.f, 0.f};
  acc = tile_mfma<kSteps>(xa, wv, acc);
  float v = tile_reduce<kWavesPerBlock>(acc, red);
  if (!split_gather<kDownSplit, false>(v, nullptr, p.split, p.counters + kCntDown, tile)) return;
  const int t = threadIdx.x;
  const int seq = tile_seq(t);
  if (seq < p.rows) p.hidden[seq * kH + n0 + (t & 15)] += v;
}

// Final RMSNorm + tied LM head + per-workgroup top-1 of every batch row.
// Workgroups loop over 16-row vocabulary tiles (grid stride); each wave
// keeps its K quarter of the gain-scaled operand in registers and the next
// tile's weights in flight while the current tile is reduced.
__global__ __launch_bounds__(kBlock) void batch_lmhead_kernel(BatchLaunch p, BatchTail tl) {
  constexpr int kSteps = kH / kStep / kWavesPerBlock;  // 14
  __shared__ float wss[kWavesPerBlock][16];
  __shared__ float ss[16];
  __shared__ float red[2][kWavesPerBlock][4][kWave];
  const int kbase = wave_id() * kSteps * kStep;
  const int k0 = kbase + k_quad();
  const int tiles = (tl.vocab + 15) / 16;
  auto load_tile = [&](int tile, float4 (&wv)[kSteps]) {
    const int r = min(tile * 16 + tile_col(), tl.vocab - 1);
    const float *w = tl.head + static_cast<size_t>(r) * kH + k0;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) wv[s] = ld_weight(reinterpret_cast<const float4 *>(w + kStep * s));
  };
  float4 wcur[kSteps];
  int tile = blockIdx.x;
  if (tile < tiles) load_tile(tile, wcur);
  float4 xa[kSteps], gv[kSteps];
  load_operand<kSteps, kH>(p.hidden, p.rows, kbase, xa);
  load_gain<kSteps>(kbase, tl.final_norm, gv);
  const float part = gain_operand<kSteps>(gv, xa);
  rows_sum_squares(part, wss, ss);
  const int t = threadIdx.x;
  const int seq = tile_seq(t);
  const float inv = rsqrtf(ss[seq] / static_cast<float>(kH) + p.eps);
  float *out = seq < p.rows ? tl.logits + static_cast<size_t>(p.slot[seq]) * tl.vocab : nullptr;
  float best = -INFINITY;
  uint32_t best_i = UINT32_MAX;
  for (int it = 0; tile < tiles; tile += gridDim.x, ++it) {
    float4 wnext[kSteps];
    const int next = tile + gridDim.x;
    if (next < tiles) load_tile(next, wnext);
    f4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kSteps; ++s) acc = mfma4(xa[s], wcur[s], acc);
    float (*rb)[4][kWave] = red[it & 1];
#pragma unroll
    for (int r = 0; r < 4; ++r) rb[wave_id()][r][lane_id()] = acc[r];
    __syncthreads();
    float v = 0.f;
#pragma unroll
    for (int u = 0; u < kWavesPerBlock; ++u) v += rb[u][t >> 6][t & 63];
    v *= inv;
    const int n = tile * 16 + (t & 15);
    if (out && n < tl.vocab) {
      out[n] = v;
      if (better(v, static_cast<uint32_t>(n), best, best_i)) {
        best = v;
        best_i = static_cast<uint32_t>(n);
      }
    }
#pragma unroll
    for (int s = 0; s < kSteps; ++s) wcur[s] = wnext[s];
  }
  // The 16 threads of a sequence are lanes q*16 .. q*16+15 of one wave.
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
    const float ov = __shfl_xor(best, o, kWave);
    const uint32_t oi = __shfl_xor(best_i, o, kWave);
    if (better(ov, oi, best, best_i)) {
      best = ov;
      best_i = oi;
    }
  }
  if ((t & 15) == 0 && seq < p.rows) {
    tl.part_val[seq * kBatchLmParts + blockIdx.x] = best;
    tl.part_idx[seq * kBatchLmParts + blockIdx.x] = best_i;
  }
}

// Per batch row: reduces the top-1 partials and writes the slot's state as
// a step leaves it (token sampled, position advanced), as
// argmax_finalize_kernel does for one sequence.
__global__ __launch_bounds__(kBlock) void batch_argmax_kernel(BatchLaunch p, BatchTail tl) {
  __shared__ float bv[kWavesPerBlock];
  __shared__ uint32_t bi[kWavesPerBlock];
  const int b = blockIdx.x;
  float best = -INFINITY;
  uint32_t best_i = UINT32_MAX;
  for (int i = threadIdx.x; i < kBatchLmParts; i += kBlock) {
    const float v = tl.part_val[b * kBatchLmParts + i];
    const uint32_t x = tl.part_idx[b * kBatchLmParts + i];
    if (better(v, x, best, best_i)) {
      best = v;
      best_i = x;
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
  if (lane_id() == 0) {
    bv[wave_id()] = best;
    bi[wave_id()] = best_i;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int w = 1; w < kWavesPerBlock; ++w) {
    if (better(bv[w], bi[w], best, best_i)) {
      best = bv[w];
      best_i = bi[w];
    }
  }
  SeqState st{};
  st.position = p.pos[b] + 1;
  st.token = best_i;
  st.eos = UINT32_MAX;
  st.top_logit = best;
  st.mode = kModeStep;
  // Every logit NaN: nothing can be fed back (stop reason 0).
  st.stopped = best_i == UINT32_MAX ? 1u : 0u;
  p.states[p.slot[b]] = st;
  tl.out_token[b] = best_i;
  tl.out_top[b] = best;
}

struct Scope {
  Marker *m;
  int id;
  Scope(Marker *marker, int kernel) : m(marker), id(kernel) {
    if (m) m->before(id);
  }
  ~Scope() {
    if (m) m->after(id);
  }
};

__global__ void clear_counters_kernel(uint32_t *__restrict__ counters, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) counters[i] = 0u;
}

// The static batch workspace: one copy per GPU the library runs on. Host
// code never passes this name to a kernel (on the host it is a stand-in,
// not a device address); it uses the per-device address batch_scratch()
// obtains from hipGetSymbolAddress.
__device__ __align__(256) static unsigned char scratch[kBatchScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxScratchDevices] = {};

size_t round256(size_t bytes) { return (bytes + 255) / 256 * 256; }

}  // namespace

size_t batch_workspace_bytes(int nq) {
  const size_t r = kBatchRows, qd = size_t(nq) * kHeadDim;
  return round256(r * kH * 4) + 2 * round256(r * qd * 4) + round256(r * kI * 4) +
         round256(r * nq * kAttnMaxChunks * kPartStride * 4) + round256(size_t(kBatchSplitFloats) * 4) +
         round256(size_t(kBatchCounters) * 4) + 2 * round256(r * kBatchLmParts * 4) + 2 * round256(r * 4);
}

BatchWorkspace carve_batch_workspace(void *base, int nq) {
  unsigned char *p = static_cast<unsigned char *>(base);
  auto take = [&](size_t bytes) {
    void *r = p;
    p += round256(bytes);
    return r;
  };
  const size_t r = kBatchRows, qd = size_t(nq) * kHeadDim;
  BatchWorkspace w{};
  w.hidden = static_cast<float *>(take(r * kH * 4));
  w.q = static_cast<float *>(take(r * qd * 4));
  w.attn = static_cast<float *>(take(r * qd * 4));
  w.act = static_cast<float *>(take(r * kI * 4));
  w.part = static_cast<float *>(take(r * nq * kAttnMaxChunks * kPartStride * 4));
  w.split = static_cast<float *>(take(size_t(kBatchSplitFloats) * 4));
  w.counters = static_cast<uint32_t *>(take(size_t(kBatchCounters) * 4));
  w.part_val = static_cast<float *>(take(r * kBatchLmParts * 4));
  w.part_idx = static_cast<uint32_t *>(take(r * kBatchLmParts * 4));
  w.out_token = static_cast<uint32_t *>(take(r * 4));
  w.out_top = static_cast<float *>(take(r * 4));
  return w;
}

static_assert(kH / kHeadDim == 14, "the batched kernels take 14 query heads");

void *batch_scratch(int device, hipError_t *err) {
  *err = hipSuccess;
  if (device < 0 || device >= kMaxScratchDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  if (batch_workspace_bytes(kH / kHeadDim) > kBatchScratchBytes) {
    *err = hipErrorInvalidValue;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *err = e != hipSuccess ? e : hipErrorInvalidSymbol;
      return nullptr;
    }
    g_scratch_ptr[device] = p;
  }
  return g_scratch_ptr[device];
}

std::mutex &batch_scratch_lock(int device) {
  static std::mutex locks[kMaxScratchDevices];
  return locks[device >= 0 && device < kMaxScratchDevices ? device : 0];
}

hipError_t launch_batch_clear_counters(hipStream_t s, uint32_t *counters) {
  clear_counters_kernel<<<(kBatchCounters + kBlock - 1) / kBlock, kBlock, 0, s>>>(counters, kBatchCounters);
  return hipGetLastError();
}

const char *batch_kernel_name(int id) {
  static const char *const names[kBatchKernelCount] = {
      "batch_embed_kernel",  "batch_qkv_kernel",    "batch_attn_kernel",
      "batch_oproj_kernel",  "batch_gateup_kernel",
      "batch_down_kernel",   "batch_lmhead_kernel", "batch_argmax_kernel"};
  return id >= 0 && id < kBatchKernelCount ? names[id] : "unknown";
}

static bool batch_shape_ok(const BatchLaunch &b) {
  return b.rows >= 1 && b.rows <= kBatchRows && b.nkv > 0 && b.nq % b.nkv == 0 &&
         b.nq * kHeadDim == kH && b.nq / b.nkv <= kMaxGroup && kBatchRows * b.nq <= kBatchCounters - kCntAttn &&
         (b.nq + 2 * b.nkv) * 4 <= kCntO - kCntQkv;
}

hipError_t launch_batch_embed(hipStream_t s, const BatchLaunch &b, const float *embed, int vocab,
                              Marker *m) {
  if (!batch_shape_ok(b)) return hipErrorInvalidValue;
  for (int i = 0; i < b.rows; ++i)
    if (b.pos[i] >= static_cast<uint32_t>(b.capacity) || b.token[i] >= static_cast<uint32_t>(vocab))
      return hipErrorInvalidValue;
  Scope scope(m, kBEmbed);
  batch_embed_kernel<<<b.rows, kBlock, 0, s>>>(b, embed, vocab);
  return hipGetLastError();
}

hipError_t launch_batch_layer(hipStream_t s, const BatchLaunch &b, const LayerPtrs &w, int layer,
                              Marker *m) {
  if (!batch_shape_ok(b)) return hipErrorInvalidValue;
  {
    Scope scope(m, kBQkvRope);
    batch_qkv_kernel<<<dim3((b.nq + 2 * b.nkv) * 4, kQkvSplit), kBlock, 0, s>>>(
        b, w.attn_norm, w.wqkv, w.bqkv, layer);
  }
  {
    Scope scope(m, kBAttn);
    batch_attn_kernel<<<dim3(kAttnMaxChunks, b.nkv, b.rows), kBlock, 0, s>>>(b, layer);
  }
  {
    Scope scope(m, kBOproj);
    batch_oproj_kernel<<<dim3(kH / 16, kOSplit), kBlock, 0, s>>>(b, w.wo);
  }
  {
    Scope scope(m, kBGateUp);
    batch_gateup_kernel<<<kI / 8, kBlock, 0, s>>>(b, w.mlp_norm, w.wg, w.wu);
  }
  {
    Scope scope(m, kBDown);
    batch_down_kernel<<<dim3(kH / 16, kDownSplit), kBlock, 0, s>>>(b, w.wd);
  }
  return hipGetLastError();
}

hipError_t launch_batch_tail(hipStream_t s, const BatchLaunch &b, const BatchTail &t, Marker *m) {
  if (!batch_shape_ok(b) || t.vocab <= 0) return hipErrorInvalidValue;
  {
    Scope scope(m, kBLmHead);
    batch_lmhead_kernel<<<kBatchLmParts, kBlock, 0, s>>>(b, t);
  }
  {
    Scope scope(m, kBArgmax);
    batch_argmax_kernel<<<b.rows, kBlock, 0, s>>>(b, t);
  }
  return hipGetLastError();
}

}  // namespace qd
