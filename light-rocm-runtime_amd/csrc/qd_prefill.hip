// Prompt (prefill) kernels for gfx950: the prompt's positions go through a
// layer together, so its projections are dense FP32 GEMMs on the matrix
// cores (v_mfma_f32_32x32x2f32) and its attention a causal flash attention
// (v_mfma_f32_16x16x4f32), instead of one decode step per position.
//
// Semantics follow the decode step per position (the reference's prompt
// stack, benchmarks/triton_mini_decoder_layer.cpp:811-849, is P sequential
// decode steps): RMSNorm eps, rotate-half RoPE at the absolute position,
// K/V cache rows written post-RoPE / raw, attention over positions
// 0..position inclusive with scale 1/sqrt(64) and query head h reading KV
// head h / (heads / kv_heads).
#include <hip/hip_runtime.h>

#include <cmath>
#include <algorithm>
#include <cstdint>

#include "qd_device.hpp"
#include "qd_device_math.hpp"
#include "qd_prefill.hpp"

namespace qd {
namespace {

using namespace dev;

typedef float f16v __attribute__((ext_vector_type(16)));
typedef float f4v __attribute__((ext_vector_type(4)));

// ---- GEMM: C = A . W^T --------------------------------------------------------
// 64 x 64 output tile per workgroup, four waves of 32 x 32 (one
// v_mfma_f32_32x32x2f32 accumulator each). K is consumed in slices of 32
// through a ring of kStages LDS stages filled by global -> LDS DMA
// (global_load_lds_dwordx4, no register staging): while slice s feeds the
// matrix cores, slices s + 1 .. s + kStages - 1 are in flight, so the
// slices' load latency overlaps the MFMA work of the ones before.
// Operand layout of v_mfma_f32_32x32x2f32: lane l supplies A[l % 32][l / 32]
// and B[l / 32][l % 32]; accumulator register r of lane l holds
// D[(r / 4) * 8 + (l / 32) * 4 + r % 4][l % 32].
// A stage holds the A and W tiles row-major, 32 floats (8 float4 slots) per
// row, float4 slot p of row r holding the row's k-quad p ^ (r % 8): a DMA
// instruction writes 8 whole rows (1 KiB) and each lane picks the source
// quad that lands in its slot; the operand reads (one float4 per lane, rows
// of eight consecutive lanes at one k-quad) then fall on 32 distinct banks.
// Lane l reads k-quad 2 j + l / 32 of its row and feeds it to four MFMAs,
// so MFMA (j, c) takes k = 8 j + 4 (l / 32) + c, in A and in B alike.
constexpr int kTileM = 64, kTileN = 64, kTileK = 32;
// Ring depth of the split-K / stream-K GEMMs (64 KiB of LDS: two workgroups
// per CU) and of the gate/up + SwiGLU GEMM (32 KiB: five per CU, so its 1,216
// tiles at M = 512 run as one round on 256 CUs instead of 2.4 rounds of 512).
#ifndef QD_GEMM_STAGES
#define QD_GEMM_STAGES 4
#endif
#ifndef QD_SWIGLU_STAGES
#define QD_SWIGLU_STAGES 2
#endif
constexpr int kStages = QD_GEMM_STAGES;
constexpr int kStagesSwiGLU = QD_SWIGLU_STAGES;
constexpr int kStageFloats = (kTileM + kTileN) * kTileK;

typedef __attribute__((address_space(3))) void gemm_lds_void;

// One 16-byte global -> LDS DMA per lane (lane l's bytes land at the stage
// offset lds + 16 l). Issued from inline assembly: the compiler would
// otherwise guard every later LDS read with a wait for all DMAs in flight,
// serialising the stages; the kernel waits for each slice itself (vmcnt,
// which counts these loads).
__device__ __forceinline__ void gemm_dma16(const float *src, const float *lds) {
  const uint32_t off = static_cast<uint32_t>(
      __builtin_amdgcn_readfirstlane(static_cast<int>(reinterpret_cast<uintptr_t>((gemm_lds_void *)lds))));
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(off), "v"(src) : "memory", "m0");
}
// Workgroup barrier over LDS only: each wave's own LDS operations complete
// first; its DMAs are waited for explicitly before it.
__device__ __forceinline__ void gemm_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Split-K: slice z = blockIdx.z of gridDim.z covers k range [z k / Z,
// (z + 1) k / Z) and, when Z > 1, writes its plain partial product to
// C + z * m * ldc (the caller's workspace); gemm_reduce_kernel then sums the
// partials in slice order and applies the epilogue.
//
// SwiGLU mode (kGemmSwiGLU): tile x covers outputs [32 x, 32 x + 32) of
// act = silu(A . wg^T) * (A . wu^T); its W tile's first 32 rows are wg's
// rows of that range and its last 32 wu's (W2), so waves (wr, 0) hold the
// gate sums and waves (wr, 1) the up sums of the same elements; the up sums
// cross through LDS and waves (wr, 0) store silu_mul(gate, up).
// Stream-K (sk_groups > 0, a one-dimensional grid of sk_groups workgroups):
// the (tile, slice) iterations, tile-major, are cut into sk_groups equal
// contiguous ranges. Workgroup g takes range [g T / G, (g + 1) T / G) and
// writes one plain partial per tile it touches, to partial slot g -
// sk_owner(first iteration of the tile) (C + slot * m * ldc); the reduction
// sums a tile's slots in slot order. Every CU then gets the same number of
// slices whatever the tile count.
__host__ __device__ inline int sk_owner(long long it, int groups, long long total) {
  return static_cast<int>(((it + 1) * groups - 1) / total);
}

// One tile's product over K slices [s_begin, s_end) into C (plain, bias or
// accumulate per mode; SwiGLU as described above).
template <int kSt>
__device__ __forceinline__ void gemm_tile(float *stage_lds, const float *__restrict__ A, int lda,
                                          const float *__restrict__ W, const float *__restrict__ W2,
                                          int ldw, float *__restrict__ C, int ldc, int m, int n, int mode,
                                          const float *__restrict__ bias, bool add_bias, int tx, int m0,
                                          int n0, int s_begin, int s_end) {
  const int lane = lane_id();
  const int w = wave_id();
  const int wr = w >> 1, wc = w & 1;
  const int slices = s_end - s_begin;
  // DMA of slice s into stage b: instruction i of a tile covers rows
  // 8 i .. 8 i + 7; this wave issues instructions w and w + 4 of the A tile
  // and of the W tile. Lane l fills slot l % 8 of row 8 i + l / 8. Rows past
  // m read row m - 1 (their products are never stored); W has n rows.
  const int drow = lane >> 3, dslot = (lane & 7) ^ drow;
  auto issue = [&](int sl, int b) {
    float *st = stage_lds + b * kStageFloats;
    const int k0 = (s_begin + sl) * kTileK + 4 * dslot;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = w + 4 * h;
      const int ra = min(m0 + 8 * i + drow, m - 1);
      const float *wrow;
      if (mode == kGemmSwiGLU) {
        const int j = tx * (kTileN / 2) + 8 * (i & 3) + drow;
        wrow = (i < 4 ? W : W2) + static_cast<size_t>(j) * ldw;
      } else {
        wrow = W + static_cast<size_t>(min(n0 + 8 * i + drow, n - 1)) * ldw;
      }
      gemm_dma16(A + static_cast<size_t>(ra) * lda + k0, st + 8 * i * kTileK);
      gemm_dma16(wrow + k0, st + kTileM * kTileK + 8 * i * kTileK);
    }
  };
  // This lane's operand rows and their swizzle.
  const int ar = wr * 32 + (lane & 31), br = wc * 32 + (lane & 31);
  const int half = lane >> 5;
  f16v acc = {};
#pragma unroll
  for (int st = 0; st < kSt - 1; ++st)
    if (st < slices) issue(st, st);
  for (int sl = 0; sl < slices; ++sl) {
    // Slice sl's DMA has landed once at most 4 (per later slice in flight)
    // of this wave's loads are outstanding; the barrier makes every wave's
    // part visible and retires every wave's reads of the stage refilled next.
    const int ahead = min(kSt - 2, slices - 1 - sl);
    if (ahead >= 2)
      asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if (ahead == 1)
      asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    gemm_lds_barrier();
    if (sl + kSt - 1 < slices) issue(sl + kSt - 1, (sl + kSt - 1) % kSt);
    const float *st = stage_lds + (sl % kSt) * kStageFloats;
    float4 av[4], bv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = 2 * j + half;
      av[j] = *reinterpret_cast<const float4 *>(st + ar * kTileK + 4 * (q ^ (ar & 7)));
      bv[j] = *reinterpret_cast<const float4 *>(st + kTileM * kTileK + br * kTileK + 4 * (q ^ (br & 7)));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[j].x, bv[j].x, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[j].y, bv[j].y, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[j].z, bv[j].z, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[j].w, bv[j].w, acc, 0, 0, 0);
    }
  }
  if (mode == kGemmSwiGLU) {
    float *ex = stage_lds;  // [wr][r][lane] up sums
    gemm_lds_barrier();     // every wave is done with the last stage
    if (wc == 1) {
#pragma unroll
      for (int r = 0; r < 16; ++r) ex[(wr * 16 + r) * kWave + lane] = acc[r];
    }
    gemm_lds_barrier();
    if (wc == 0) {
      const int col = tx * (kTileN / 2) + (lane & 31);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + wr * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
        if (row < m) C[static_cast<size_t>(row) * ldc + col] = silu_mul(acc[r], ex[(wr * 16 + r) * kWave + lane]);
      }
    }
    return;
  }
  const int col = n0 + wc * 32 + (lane & 31);
  if (col >= n) return;
  const float bv = mode == kGemmBias && add_bias ? bias[col] : 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = m0 + wr * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
    if (row < m) {
      float *c = C + static_cast<size_t>(row) * ldc + col;
      if (mode == kGemmAccumulate)
        *c += acc[r];
      else
        *c = acc[r] + bv;
    }
  }
}

template <int kSt>
__global__ __launch_bounds__(kBlock) void gemm_nt_kernel(const float *__restrict__ A, int lda,
                                                         const float *__restrict__ W,
                                                         const float *__restrict__ W2, int ldw,
                                                         float *__restrict__ C, int ldc, int m,
                                                         int n, int k, int mode,
                                                         const float *__restrict__ bias, int sk_groups) {
  __shared__ __attribute__((aligned(16))) float stage_lds[kSt * kStageFloats];
  const int slices_all = k / kTileK;
  if (sk_groups > 0) {
    const int tiles_n = (n + kTileN - 1) / kTileN;
    const long long total = static_cast<long long>((m + kTileM - 1) / kTileM) * tiles_n * slices_all;
    const int g = blockIdx.x;
    const long long it1 = (g + 1) * total / sk_groups;
    for (long long it = g * total / sk_groups; it < it1;) {
      const int tile = static_cast<int>(it / slices_all);
      const long long first = static_cast<long long>(tile) * slices_all;
      const int s_begin = static_cast<int>(it - first);
      const int s_end = static_cast<int>(min(it1 - first, static_cast<long long>(slices_all)));
      const int slot = g - sk_owner(first, sk_groups, total);
      gemm_lds_barrier();  // the previous tile's last stage reads are done
      gemm_tile<kSt>(stage_lds, A, lda, W, W2, ldw, C + static_cast<size_t>(slot) * m * ldc, ldc, m, n, kGemmStore,
                bias, false, tile % tiles_n, (tile / tiles_n) * kTileM, (tile % tiles_n) * kTileN, s_begin,
                s_end);
      it = first + slices_all;
    }
    return;
  }
  const int split = gridDim.z;
  const int s_begin = static_cast<int>(blockIdx.z) * slices_all / split;
  const int s_end = (static_cast<int>(blockIdx.z) + 1) * slices_all / split;
  if (split > 1) {
    C += static_cast<size_t>(blockIdx.z) * m * ldc;
    mode = kGemmStore;
  }
  gemm_tile<kSt>(stage_lds, A, lda, W, W2, ldw, C, ldc, m, n, mode, bias, split == 1, blockIdx.x,
            blockIdx.y * kTileM, blockIdx.x * kTileN, s_begin, s_end);
}

// Sum of the first `parts` partials of element e (part + z * stride + e), in
// slot order: the first kBatch are requested before any is added (one round
// trip), later ones one batch at a time.
__device__ __forceinline__ float sum_partials(const float *__restrict__ part, size_t stride, size_t e, int parts) {
  constexpr int kBatch = 8;
  float v = 0.f;
  for (int z0 = 0; z0 < parts; z0 += kBatch) {
    float pv[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) pv[j] = z0 + j < parts ? part[static_cast<size_t>(z0 + j) * stride + e] : 0.f;
    if (z0 == 0) v = pv[0];
#pragma unroll
    for (int j = 0; j < kBatch; ++j)
      if ((z0 > 0 || j > 0) && z0 + j < parts) v += pv[j];
  }
  return v;
}

// Partial slots of a tile's product: split (classic split-K), or with
// stream-K (sk_groups > 0) the workgroups whose ranges meet the tile of
// element (r, c).
__device__ __forceinline__ int partial_count(int split, int sk_groups, int r, int c, int m, int n, int k) {
  if (sk_groups <= 0) return split;
  const int slices_all = k / kTileK, tiles_n = (n + kTileN - 1) / kTileN;
  const long long total = static_cast<long long>((m + kTileM - 1) / kTileM) * tiles_n * slices_all;
  const long long first = static_cast<long long>((r / kTileM) * tiles_n + c / kTileN) * slices_all;
  return sk_owner(first + slices_all - 1, sk_groups, total) - sk_owner(first, sk_groups, total) + 1;
}

// C[r][c] (op)= sum_z part[z][r][c] (+ bias[c]) for the split-K partials
// (partial_count of them for the element's tile).
__global__ __launch_bounds__(kBlock) void gemm_reduce_kernel(const float *__restrict__ part,
                                                             int split, int sk_groups, int k,
                                                             float *__restrict__ C, int ldc, int m, int n,
                                                             int mode, const float *__restrict__ bias) {
  const size_t total = static_cast<size_t>(m) * n;
  for (size_t e = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; e < total;
       e += static_cast<size_t>(gridDim.x) * kBlock) {
    const int r = static_cast<int>(e / n), c = static_cast<int>(e % n);
    const int parts = partial_count(split, sk_groups, r, c, m, n, k);
    const float v = sum_partials(part, static_cast<size_t>(m) * ldc, static_cast<size_t>(r) * ldc + c, parts);
    float *dst = C + static_cast<size_t>(r) * ldc + c;
    if (mode == kGemmAccumulate)
      *dst += v;
    else
      *dst = mode == kGemmBias ? v + bias[c] : v;
  }
}

// ---- row-wise kernels ----------------------------------------------------------

__global__ __launch_bounds__(kBlock) void embed_rows_kernel(const float *__restrict__ embed,
                                                            const uint32_t *__restrict__ tokens,
                                                            int hidden, float *__restrict__ out) {
  const int r = blockIdx.x;
  const float4 *src = reinterpret_cast<const float4 *>(embed + static_cast<size_t>(tokens[r]) * hidden);
  float4 *dst = reinterpret_cast<float4 *>(out + static_cast<size_t>(r) * hidden);
  for (int c = threadIdx.x; c < hidden / 4; c += kBlock) dst[c] = src[c];
}

// RMSNorm of one prompt row: x * inv * gain with inv from block_inv_rms
// (the whole workgroup). (The decode kernels fold the norm past their
// GEMVs instead, inv * (W . (x * gain)); the two agree to rounding.)
template <int H>
__device__ __forceinline__ void rmsnorm_row(const float *xr, const float *__restrict__ gain, float eps, float *yr,
                                            float *red) {
  const float inv = block_inv_rms<H>(Plain(xr), eps, red);
  const float4 *x4 = reinterpret_cast<const float4 *>(xr);
  const float4 *g4 = reinterpret_cast<const float4 *>(gain);
  float4 *y4 = reinterpret_cast<float4 *>(yr);
  for (int c = threadIdx.x; c < H / 4; c += kBlock) {
    const float4 v = x4[c], g = g4[c];
    y4[c] = make_float4(v.x * inv * g.x, v.y * inv * g.y, v.z * inv * g.z, v.w * inv * g.w);
  }
}

template <int H>
__global__ __launch_bounds__(kBlock) void rmsnorm_rows_kernel(const float *__restrict__ x,
                                                              const float *__restrict__ gain,
                                                              float eps, float *__restrict__ y) {
  __shared__ float red[kWavesPerBlock];
  const int r = blockIdx.x;
  rmsnorm_row<H>(x + static_cast<size_t>(r) * H, gain, eps, y + static_cast<size_t>(r) * H, red);
}

// RoPE of one packed QKV row at position p (query and key heads rotated in
// place) and its K/V rows written to the cache (the whole workgroup).
__device__ __forceinline__ void rope_kv_row(float *row, int p, int nq, int nkv, const float *__restrict__ rope_cos,
                                            const float *__restrict__ rope_sin, float *__restrict__ k_cache,
                                            float *__restrict__ v_cache) {
  const int qd = nq * kHeadDim, kvd = nkv * kHeadDim;
  const int rotations = (nq + nkv) * kRotary;
  for (int u = threadIdx.x; u < rotations + kvd; u += kBlock) {
    if (u < rotations) {
      const int head = u / kRotary, i = u % kRotary;
      const int a = head * kHeadDim + i, b = a + kRotary;
      const float c = rope_cos[p * kRotary + i], s = rope_sin[p * kRotary + i];
      const float x0 = row[a], x1 = row[b];
      float first, second;
      rope_rotate(x0, x1, c, s, first, second);
      row[a] = first;
      row[b] = second;
      if (head >= nq) {
        const int o = (head - nq) * kHeadDim + i;
        k_cache[static_cast<size_t>(p) * kvd + o] = first;
        k_cache[static_cast<size_t>(p) * kvd + o + kRotary] = second;
      }
    } else {
      const int o = u - rotations;
      v_cache[static_cast<size_t>(p) * kvd + o] = row[qd + kvd + o];
    }
  }
}

__global__ __launch_bounds__(kBlock) void rope_kv_rows_kernel(float *__restrict__ qkv, int pos0, int nq,
                                                              int nkv, const float *__restrict__ rope_cos,
                                                              const float *__restrict__ rope_sin,
                                                              float *__restrict__ k_cache,
                                                              float *__restrict__ v_cache) {
  const int r = blockIdx.x;
  rope_kv_row(qkv + static_cast<size_t>(r) * (nq + 2 * nkv) * kHeadDim, pos0 + r, nq, nkv, rope_cos, rope_sin,
              k_cache, v_cache);
}

// gemm_reduce_kernel's sums and epilogue for one row per workgroup, then the
// row epilogue on the finished row: RMSNorm into epi.y (kRowNorm) or RoPE
// with the K/V cache rows (kRowRope), with the arithmetic of
// rmsnorm_rows_kernel / rope_kv_rows_kernel, so the results are the same
// bits as those kernels after gemm_reduce_kernel.
__global__ __launch_bounds__(kBlock) void gemm_reduce_rows_kernel(const float *__restrict__ part, int split,
                                                                  int sk_groups, int k, float *__restrict__ C,
                                                                  int ldc, int m, int n, int mode,
                                                                  const float *__restrict__ bias, RowEpilogue epi) {
  __shared__ float red[kWavesPerBlock];
  const int r = blockIdx.x;
  float *row = C + static_cast<size_t>(r) * ldc;
  for (int c = threadIdx.x; c < n; c += kBlock) {
    const int parts = partial_count(split, sk_groups, r, c, m, n, k);
    const float v = sum_partials(part, static_cast<size_t>(m) * ldc, static_cast<size_t>(r) * ldc + c, parts);
    if (mode == kGemmAccumulate)
      row[c] += v;
    else
      row[c] = mode == kGemmBias ? v + bias[c] : v;
  }
  __syncthreads();
  if (epi.kind == kRowNorm)
    rmsnorm_row<896>(row, epi.gain, epi.eps, epi.y + static_cast<size_t>(r) * n, red);
  else if (epi.kind == kRowRope)
    rope_kv_row(row, epi.pos0 + r, epi.nq, epi.nkv, epi.rope_cos, epi.rope_sin, epi.k_cache, epi.v_cache);
}

// ---- causal GQA flash attention ---------------------------------------------------
// One query block = (query head h, 16 prompt rows); a workgroup's four waves take
// the key blocks (32 positions) round-robin, each keeping an online softmax
// and an output accumulator for the 16 queries, merged in LDS at the end.
// Per key block a wave computes S = Q . K^T (two 16 x 16 tiles over 64
// dims) and O += P . V (four 16 x 16 tiles over 32 keys) with
// v_mfma_f32_16x16x4f32, whose lane l supplies A[l % 16][l / 16] and
// B[l / 16][l % 16] and holds D[(l / 16) * 4 + r][l % 16] in register r.
constexpr int kQBlock = 16;
constexpr int kKBlock = 32;
constexpr int kKRow = kHeadDim + 4;   // LDS K row stride (conflict-free B reads)
constexpr int kVRow = kHeadDim + 16;  // LDS V row stride
constexpr int kPRow = kKBlock + 4;    // LDS P row stride

struct PrefillAttnLds {
  float k[kWavesPerBlock][kKBlock][kKRow];
  float v[kWavesPerBlock][kKBlock][kVRow];
  float p[kWavesPerBlock][kQBlock][kPRow];
  float ml[kWavesPerBlock][kQBlock][2];
  float o[kWavesPerBlock][kQBlock][kHeadDim + 1];
};

// max / sum over the 16 lanes of a DPP row (lanes 16g .. 16g + 15).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return v;
}

// Query block qb of head h (the causal extent of a block grows with qb).
__device__ __forceinline__ void attention_prefill_block(
    PrefillAttnLds &sh, int qb, const float *__restrict__ qkv, int rows, int pos0, int nq, int nkv,
    const float *__restrict__ k_cache, const float *__restrict__ v_cache, float *__restrict__ out) {
  const int h = blockIdx.y;
  const int r0 = qb * kQBlock;
  const int g = h / (nq / nkv);
  const int qd = nq * kHeadDim, kvd = nkv * kHeadDim;
  const int ld = qd + 2 * kvd;
  const int w = wave_id();
  const int lane = lane_id();
  const int lr = lane & 15, lg = lane >> 4;
  // Scores in base-2 units, s log2(e) / sqrt(64), so each softmax
  // exponential is one v_exp_f32 (2^x): e^(s / 8 - m) = 2^(s log2(e) / 8 - m').
  const float scale = 0.18033688011112042f;  // log2(e) / sqrt(64)
  const int last_row = min(rows, r0 + kQBlock) - 1;
  const int keys = pos0 + last_row + 1;  // causal extent of the block
  const int kblocks = (keys + kKBlock - 1) / kKBlock;

  // Query operand: lane supplies Q[row lr][dim 16 lg + s] at k-step s < 16
  // (the K operand takes the same dims), so each lane's 16 dims are
  // contiguous: four float4 reads.
  float qa[kHeadDim / 4];
  {
    const int qrow = min(r0 + lr, rows - 1);
    const float4 *q4 = reinterpret_cast<const float4 *>(qkv + static_cast<size_t>(qrow) * ld + h * kHeadDim + 16 * lg);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float4 v = q4[j];
      qa[4 * j] = v.x;
      qa[4 * j + 1] = v.y;
      qa[4 * j + 2] = v.z;
      qa[4 * j + 3] = v.w;
    }
  }
  // Running state of the lane's four query rows lg * 4 + r.
  float m[4], l[4];
  f4v o[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.f;
    o[r] = f4v{0.f, 0.f, 0.f, 0.f};
  }
  float (*ks)[kKRow] = sh.k[w];
  float (*vs)[kVRow] = sh.v[w];
  float (*ps)[kPRow] = sh.p[w];
  // The block's K and V rows in registers: lane covers rows lane / 16 +
  // 4 i, float4 column lane % 16 (zeros past the causal extent). The wave's
  // next block is loaded while the current one is computed.
  float4 kr[kKBlock / 4], vr[kKBlock / 4];
  auto load_block = [&](int kb) {
#pragma unroll
    for (int i = 0; i < kKBlock / 4; ++i) {
      const int j = kb * kKBlock + lg + 4 * i;
      kr[i] = vr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (j < keys) {
        kr[i] = *reinterpret_cast<const float4 *>(k_cache + static_cast<size_t>(j) * kvd + g * kHeadDim + 4 * lr);
        vr[i] = *reinterpret_cast<const float4 *>(v_cache + static_cast<size_t>(j) * kvd + g * kHeadDim + 4 * lr);
      }
    }
  };
  if (w < kblocks) load_block(w);
  for (int kb = w; kb < kblocks; kb += kWavesPerBlock) {
    const int k0 = kb * kKBlock;
    // Stage the block's rows in the wave's LDS, then start the next block's
    // loads.
#pragma unroll
    for (int i = 0; i < kKBlock / 4; ++i) {
      const int row = lg + 4 * i;
      const float4 kv = kr[i], vv = vr[i];
      *reinterpret_cast<float4 *>(&ks[row][4 * lr]) = kv;
      *reinterpret_cast<float4 *>(&vs[row][4 * lr]) = vv;
    }
    if (kb + kWavesPerBlock < kblocks) load_block(kb + kWavesPerBlock);
    // S tiles: keys k0 + 16 tt + lr. Every B operand is read from LDS before
    // the first MFMA (one wait instead of one per step), and the two tiles'
    // chains run interleaved; each chain keeps its order over st.
    float kop[2][kHeadDim / 4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const float4 v = *reinterpret_cast<const float4 *>(&ks[16 * tt + lr][16 * lg + 4 * j]);
        kop[tt][4 * j] = v.x;
        kop[tt][4 * j + 1] = v.y;
        kop[tt][4 * j + 2] = v.z;
        kop[tt][4 * j + 3] = v.w;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    f4v s[2] = {f4v{0.f, 0.f, 0.f, 0.f}, f4v{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int st = 0; st < kHeadDim / 4; ++st) {
      s[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[st], kop[0][st], s[0], 0, 0, 0);
      s[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[st], kop[1][st], s[1], 0, 0, 0);
    }
    // Online softmax per query row (row = lg * 4 + r, spread over the 16
    // lanes of DPP row lg and the two tiles).
    float corr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int qpos = pos0 + min(r0 + lg * 4 + r, rows - 1);
      float sv[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const int key = k0 + 16 * tt + lr;
        sv[tt] = key <= qpos ? s[tt][r] * scale : -INFINITY;
      }
      const float m_new = fmaxf(m[r], row16_max(fmaxf(sv[0], sv[1])));
      float p0 = 0.f, p1 = 0.f;
      corr[r] = 1.f;
      if (m_new != -INFINITY) {
        p0 = __builtin_amdgcn_exp2f(sv[0] - m_new);
        p1 = __builtin_amdgcn_exp2f(sv[1] - m_new);
        corr[r] = __builtin_amdgcn_exp2f(m[r] - m_new);
      }
      l[r] = fmaf(l[r], corr[r], row16_sum(p0 + p1));
      m[r] = m_new;
      ps[lg * 4 + r][lr] = p0;
      ps[lg * 4 + r][16 + lr] = p1;
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[dt][r] *= corr[r];
    // O += P . V: A = P[row lr][key 4 st + lg], B = V[key 4 st + lg][dim 16 dt + lr],
    // the operands read from LDS first as for S (this key order keeps the V
    // reads of the four lane groups on different banks).
    float pa[kKBlock / 4], vb[kKBlock / 4][4];
#pragma unroll
    for (int st = 0; st < kKBlock / 4; ++st) {
      pa[st] = ps[lr][4 * st + lg];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) vb[st][dt] = vs[4 * st + lg][16 * dt + lr];
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < kKBlock / 4; ++st)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[st], vb[st][dt], o[dt], 0, 0, 0);
  }
  // Merge the four waves' partials.
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int q = lg * 4 + r;
    if (lr == 0) {
      sh.ml[w][q][0] = m[r];
      sh.ml[w][q][1] = l[r];
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) sh.o[w][q][16 * dt + lr] = o[dt][r];
  }
  __syncthreads();
  {
    const int q = threadIdx.x >> 4;        // 16 queries
    const int d0 = (threadIdx.x & 15) * 4;  // 4 dims each
    const int row = r0 + q;
    if (row < rows) {
      float mx = -INFINITY;
#pragma unroll
      for (int v = 0; v < kWavesPerBlock; ++v) mx = fmaxf(mx, sh.ml[v][q][0]);
      float den = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int v = 0; v < kWavesPerBlock; ++v) {
        const float mv = sh.ml[v][q][0];
        const float f = mv == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mv - mx);
        den = fmaf(f, sh.ml[v][q][1], den);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = fmaf(f, sh.o[v][q][d0 + e], acc[e]);
      }
      float *dst = out + static_cast<size_t>(row) * qd + h * kHeadDim + d0;
#pragma unroll
      for (int e = 0; e < 4; ++e) dst[e] = acc[e] / den;
    }
  }
}

// Workgroup (pair p, head h) takes query blocks p and nqb - 1 - p: the pair's
// key blocks add up to about the same count for every p, so the launch is
// one balanced round of workgroups instead of a long causal tail.
__global__ __launch_bounds__(kBlock) void attention_prefill_kernel(
    const float *__restrict__ qkv, int rows, int pos0, int nq, int nkv,
    const float *__restrict__ k_cache, const float *__restrict__ v_cache, float *__restrict__ out) {
  __shared__ __attribute__((aligned(16))) PrefillAttnLds sh;
  const int nqb = (rows + kQBlock - 1) / kQBlock;
  const int p = blockIdx.x;
  attention_prefill_block(sh, p, qkv, rows, pos0, nq, nkv, k_cache, v_cache, out);
  const int q = nqb - 1 - p;
  if (q <= p) return;
  __syncthreads();  // the first block's merge has read the LDS
  attention_prefill_block(sh, q, qkv, rows, pos0, nq, nkv, k_cache, v_cache, out);
}

}  // namespace

int gemm_streamk_slots(int m, int n, int k, int groups) {
  if (m <= 0 || n <= 0 || k < kTileK || groups <= 0) return 0;
  const int slices_all = k / kTileK, tiles_n = (n + kTileN - 1) / kTileN;
  const int tiles = ((m + kTileM - 1) / kTileM) * tiles_n;
  const long long total = static_cast<long long>(tiles) * slices_all;
  int most = 0;
  for (int t = 0; t < tiles; ++t) {
    const long long first = static_cast<long long>(t) * slices_all;
    most = std::max(most, sk_owner(first + slices_all - 1, groups, total) - sk_owner(first, groups, total) + 1);
  }
  return most;
}

hipError_t launch_gemm_nt(hipStream_t s, const float *A, int lda, const float *W, int ldw,
                          float *C, int ldc, int m, int n, int k, GemmMode mode,
                          const float *bias, int split, float *workspace, const RowEpilogue *epi,
                          int sk_groups, size_t workspace_floats) {
  if (k % kTileK != 0 || m <= 0 || n <= 0 || split < 1 || split > k / kTileK || sk_groups < 0 ||
      ((split > 1 || sk_groups > 0) && !workspace))
    return hipErrorInvalidValue;
  // Stream-K: every tile's partial slots must fit the workspace.
  if (sk_groups > 0 &&
      static_cast<size_t>(gemm_streamk_slots(m, n, k, sk_groups)) * m * ldc > workspace_floats)
    return hipErrorInvalidValue;
  const bool partials = split > 1 || sk_groups > 0;
  // A row epilogue runs in the partials' reduction, one workgroup per row.
  if (epi && (!partials || ldc != n || (epi->kind == kRowNorm && (n != 896 || !epi->y || !epi->gain)) ||
              (epi->kind == kRowRope && n != (epi->nq + 2 * epi->nkv) * kHeadDim)))
    return hipErrorInvalidValue;
  if (mode == kGemmSwiGLU) return hipErrorInvalidValue;
  const dim3 grid = sk_groups > 0 ? dim3(sk_groups, 1, 1)
                                  : dim3((n + kTileN - 1) / kTileN, (m + kTileM - 1) / kTileM, split);
  gemm_nt_kernel<kStages><<<grid, kBlock, 0, s>>>(A, lda, W, nullptr, ldw, partials ? workspace : C, ldc, m, n, k,
                                         mode, bias, sk_groups);
  if (partials && epi) {
    gemm_reduce_rows_kernel<<<m, kBlock, 0, s>>>(workspace, split, sk_groups, k, C, ldc, m, n, mode, bias,
                                                 *epi);
  } else if (partials) {
    const size_t total = static_cast<size_t>(m) * n;
    const int blocks = static_cast<int>(std::min<size_t>((total + kBlock - 1) / kBlock, 4096));
    gemm_reduce_kernel<<<blocks, kBlock, 0, s>>>(workspace, split, sk_groups, k, C, ldc, m, n, mode, bias);
  }
  return hipGetLastError();
}

hipError_t launch_embed_rows(hipStream_t s, const float *embed, const uint32_t *tokens, int rows,
                             int hidden, float *out) {
  embed_rows_kernel<<<rows, kBlock, 0, s>>>(embed, tokens, hidden, out);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_rows(hipStream_t s, const float *x, const float *gain, float eps,
                               int rows, float *y) {
  rmsnorm_rows_kernel<896><<<rows, kBlock, 0, s>>>(x, gain, eps, y);
  return hipGetLastError();
}

hipError_t launch_rope_kv_rows(hipStream_t s, float *qkv, int rows, int pos0, int nq, int nkv,
                               const float *rope_cos, const float *rope_sin, float *k_cache,
                               float *v_cache) {
  rope_kv_rows_kernel<<<rows, kBlock, 0, s>>>(qkv, pos0, nq, nkv, rope_cos, rope_sin, k_cache,
                                              v_cache);
  return hipGetLastError();
}

hipError_t launch_attention_prefill(hipStream_t s, const float *qkv, int rows, int pos0, int nq,
                                    int nkv, const float *k_cache, const float *v_cache,
                                    float *out) {
  const int nqb = (rows + kQBlock - 1) / kQBlock;
  const dim3 grid((nqb + 1) / 2, nq);
  attention_prefill_kernel<<<grid, kBlock, 0, s>>>(qkv, rows, pos0, nq, nkv, k_cache, v_cache, out);
  return hipGetLastError();
}

hipError_t launch_gemm_swiglu(hipStream_t s, const float *A, int lda, const float *wg, const float *wu,
                              int ldw, float *act, int ldc, int m, int inter, int k) {
  if (k % kTileK != 0 || m <= 0 || inter <= 0 || inter % (kTileN / 2) != 0) return hipErrorInvalidValue;
  const dim3 grid(inter / (kTileN / 2), (m + kTileM - 1) / kTileM, 1);
  gemm_nt_kernel<kStagesSwiGLU><<<grid, kBlock, 0, s>>>(A, lda, wg, wu, ldw, act, ldc, m, 2 * inter, k,
                                                        kGemmSwiGLU, nullptr, 0);
  return hipGetLastError();
}

}  // namespace qd
