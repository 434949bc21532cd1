// Qwen2 FP32 decode-step kernels for gfx950 (CDNA4, wave64).
//
// Every kernel is bandwidth-bound: weights stream from HBM once per token in
// 128-bit (float4) coalesced loads, each wave owns whole output rows, and the
// activation operand sits in per-lane registers whose slot layout matches the
// weight slots the lane loads. Reductions are wave64 butterflies.
//
// Reference semantics (file:line under the reference tree):
//   RMSNorm                 benchmarks/qwen_stateful_graph_kernel.cpp:665-701
//   QKV + bias              benchmarks/qwen_stateful_graph_kernel.cpp:392-492
//   RoPE + KV-cache write   benchmarks/qwen_stateful_graph_kernel.cpp:517-552
//   GQA attention           benchmarks/qwen_stateful_graph_kernel.cpp:554-600
//   O projection + residual benchmarks/qwen_stateful_graph_kernel.cpp:602-659
//   gate/up + SiLU          benchmarks/qwen_stateful_graph_kernel.cpp:494-515
//   down + residual         benchmarks/qwen_stateful_graph_kernel.cpp:158-223,749-760
//   LM head + top-1         benchmarks/qwen_stateful_graph_kernel.cpp:225-356
//   embedding feedback      benchmarks/qwen_stateful_graph_kernel.cpp:358-390
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <type_traits>

#include "qd_device.hpp"
#include "qd_attention.hpp"
#include "qd_device_math.hpp"
#include "qd_kernels.hpp"

namespace qd {
namespace {

using namespace dev;

// ---- kernels ----------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void embed_kernel(
    const float *__restrict__ emb, const SeqState *__restrict__ st,
    float *__restrict__ hidden, int H, int vocab) {
  if (st->stopped || st->token >= static_cast<uint32_t>(vocab)) return;
  const size_t base = static_cast<size_t>(st->token) * H;
  for (int i = blockIdx.x * kBlock + threadIdx.x; i < H; i += gridDim.x * kBlock)
    hidden[i] = emb[base + i];
}

// attention RMSNorm + packed QKV + bias + RoPE + KV-cache write.
// Work unit u = (head, i): rows head*64+i and head*64+i+32 of the packed
// matrix, which are exactly the pair a rotate-half rotation mixes. Heads
// [0, nq) are queries, [nq, nq+nkv) keys, then values (not rotated).
template <int H, typename W>
__global__ __launch_bounds__(kBlock) void qkv_rope_kernel(
    const float *__restrict__ hidden, const float *__restrict__ gain,
    const W *__restrict__ wqkv, const float *__restrict__ bqkv,
    const float *__restrict__ rope_cos, const float *__restrict__ rope_sin,
    const SeqState *__restrict__ st, float *__restrict__ q,
    float *__restrict__ k_cache, float *__restrict__ v_cache, int nq, int nkv,
    float eps, int capacity) {
  if (st->stopped || st->position >= static_cast<uint32_t>(capacity)) return;
  float4 gv[PairSlots<H>::NJ];
  load_pair_gain<H>(gain, gv);
  float4 xv[PairSlots<H>::NJ];
  const float inv = norm_scale(load_pair_operand_gain<H>(Plain(hidden), gv, xv), H, eps);
  const int position = static_cast<int>(st->position);
  const int kv_dim = nkv * kHeadDim;
  const int units = (nq + 2 * nkv) * kRotary;
  for (int u = blockIdx.x * kWavesPerBlock + wave_id(); u < units;
       u += gridDim.x * kWavesPerBlock) {
    const int head = u / kRotary;
    const int i = u % kRotary;
    const int ra = head * kHeadDim + i;
    const int rb = ra + kRotary;
    float sa, sb;
    dot_pair<H, W>(wqkv + static_cast<size_t>(ra) * H,
                   wqkv + static_cast<size_t>(rb) * H, xv, sa, sb);
    if (lane_id() == 0) {
      const float a = fmaf(sa, inv, bqkv[ra]);
      const float b = fmaf(sb, inv, bqkv[rb]);
      if (head < nq + nkv) {
        const float c = rope_cos[position * kRotary + i];
        const float s = rope_sin[position * kRotary + i];
        float first, second;
        rope_rotate(a, b, c, s, first, second);
        if (head < nq) {
          q[ra] = first;
          q[rb] = second;
        } else {
          float *dst = k_cache + static_cast<size_t>(position) * kv_dim +
                       (head - nq) * kHeadDim;
          dst[i] = first;
          dst[i + kRotary] = second;
        }
      } else {
        float *dst = v_cache + static_cast<size_t>(position) * kv_dim +
                     (head - nq - nkv) * kHeadDim;
        dst[i] = a;
        dst[i + kRotary] = b;
      }
    }
  }
}

// Split-KV decode attention partials (qd_attention.hpp): one workgroup of
// kAttnSlots waves per (chunk, KV group), K/V read from the cache (this
// step's row was written by qkv_rope_kernel). A one-block chunk takes one
// wave per query head (attn_block_valu); a longer one deals its tiles w,
// w + kAttnSlots, ... to wave w (attn_tile) and folds the wave partials in
// slot order. Each head gets one record (m, l, acc[64]) in
// part[head][chunk][66]: the arithmetic of the resident kernel's attention
// CUs.
constexpr int kAttnThreads = kAttnSlots * kWave;
__global__ __launch_bounds__(kAttnThreads) void attn_partial_kernel(
    const float *__restrict__ q, const float *__restrict__ k_cache,
    const float *__restrict__ v_cache, const SeqState *__restrict__ st,
    int nq, int nkv, float *__restrict__ part, int capacity, int parts) {
  __shared__ float ps[kAttnSlots * kAttnPsFloats];
  __shared__ float stage_lds[kAttnStageFloats];
  if (st->stopped || st->position >= static_cast<uint32_t>(capacity)) return;
  const int position = static_cast<int>(st->position);
  const int length = position + 1;
  const int chunk = blockIdx.x;
  if (chunk >= attn_chunks(length, parts, kAttnGrain)) return;
  const int chunk_len = attn_chunk_len(length, parts, kAttnGrain);
  const int g = blockIdx.y;
  const int group = nq / nkv;
  const int kv_dim = nkv * kHeadDim;
  const int begin = chunk * chunk_len;
  const int end = min(length, begin + chunk_len);
  const float *kb = k_cache + g * kHeadDim;
  const float *vb = v_cache + g * kHeadDim;
  const int w = wave_id();
  if (attn_single_block(chunk_len)) {
    // One block: wave w takes head w of the group.
    if (w < group) {
      const int h = g * group + w;
      const float *kc = kb + static_cast<size_t>(begin) * kv_dim;
      const float *vc = vb + static_cast<size_t>(begin) * kv_dim;
      float4 qv[kHeadDim / 4];
#pragma unroll
      for (int d4 = 0; d4 < kHeadDim / 4; ++d4) qv[d4] = reinterpret_cast<const float4 *>(q + h * kHeadDim)[d4];
      PLds pb{ps + w * kAttnPsFloats + 4, kWave};
      float mb[1], lb[1], ab[1];
      attn_block_valu<1>(
          [&](int d4, int j) { return reinterpret_cast<const float4 *>(kc + static_cast<size_t>(j) * kv_dim)[d4]; },
          [&](int, int d4) { return qv[d4]; }, [&](int j, int d) { return vc[static_cast<size_t>(j) * kv_dim + d]; },
          pb, 0, end - begin - 1, mb, lb, ab);
      float M = -INFINITY, L = 0.f, A = 0.f;
      attn_fold(mb[0], lb[0], ab[0], M, L, A);
      float *rec = part + (h * kAttnMaxChunks + chunk) * kPartStride;
      rec[2 + lane_id()] = A;
      if (lane_id() == 0) {
        rec[0] = M;
        rec[1] = L;
      }
    }
    return;
  }
  float4 qa[kHeadDim / 4];
  attn_query([&](int h, int d4) { return reinterpret_cast<const float4 *>(q + (g * group + h) * kHeadDim)[d4]; },
             group, qa);
  AttnAcc acc;
  acc.init();
  attn_slot_tiles(
      qa, [&](int pos, int d4) { return reinterpret_cast<const float4 *>(kb + static_cast<size_t>(pos) * kv_dim)[d4]; },
      [&](int pos, int d) { return vb[static_cast<size_t>(pos) * kv_dim + d]; }, ps + w * kAttnPsFloats, begin,
      begin, end, end, w, acc);
  const AttnStage stage{stage_lds, stage_lds + kAttnSlots * kMaxGroup, stage_lds + 2 * kAttnSlots * kMaxGroup};
  stage.put(w, group, acc);
  __syncthreads();
  const int tiles = (end - begin + kAttnTile - 1) / kAttnTile;
  for (int i = threadIdx.x; i < group * kHeadDim; i += kAttnThreads) {
    const int h = i / kHeadDim, d = i % kHeadDim;
    float M, L, A;
    attn_slot_merge(stage, tiles, h, d, M, L, A);
    float *rec = part + ((g * group + h) * kAttnMaxChunks + chunk) * kPartStride;
    rec[2 + d] = A;
    if (d == 0) {
      rec[0] = M;
      rec[1] = L;
    }
  }
}

// Merges each head's partials into attn[h*64 + d].
__global__ __launch_bounds__(kHeadDim) void attn_combine_kernel(
    const float *__restrict__ part, const SeqState *__restrict__ st, int nq,
    float *__restrict__ attn, int capacity, int parts) {
  if (st->stopped || st->position >= static_cast<uint32_t>(capacity)) return;
  const int chunks = attn_chunks(static_cast<int>(st->position) + 1, parts, kAttnGrain);
  const int h = blockIdx.x;
  const int d = threadIdx.x;
  attn[h * kHeadDim + d] = attn_merge(
      [&](int c, int k) { return part[(h * kAttnMaxChunks + c) * kPartStride + k]; }, chunks,
      d);
}

// hidden[r] += Wo[r,:] . attn; unit u = rows (2u, 2u+1), contiguous. The
// dot is taken per KV group (columns [g QDG, (g + 1) QDG): the group's
// query heads) and added in group order, hidden + group 0 first: the
// resident role kernel's O CUs each hold one group's columns.
template <int H, int QD, int NKV, typename W>
__global__ __launch_bounds__(kBlock) void oproj_residual_kernel(
    const float *__restrict__ attn, const W *__restrict__ wo,
    const SeqState *__restrict__ st, float *__restrict__ hidden) {
  if (st->stopped) return;
  constexpr int QDG = QD / NKV;
  float4 xv[NKV][PairSlots<QDG>::NJ];
#pragma unroll
  for (int g = 0; g < NKV; ++g) load_pair_operand<QDG>(Plain(attn + g * QDG), xv[g]);
  constexpr int units = H / 2;
  for (int u = blockIdx.x * kWavesPerBlock + wave_id(); u < units;
       u += gridDim.x * kWavesPerBlock) {
    const W *a = wo + static_cast<size_t>(2 * u) * QD;
    float ha = hidden[2 * u], hb = hidden[2 * u + 1];
#pragma unroll
    for (int g = 0; g < NKV; ++g) {
      float sa, sb;
      dot_pair<QDG, W>(a + g * QDG, a + QD + g * QDG, xv[g], sa, sb);
      ha += sa;
      hb += sb;
    }
    if (lane_id() == 0) {
      hidden[2 * u] = ha;
      hidden[2 * u + 1] = hb;
    }
  }
}

// MLP RMSNorm + gate/up + SiLU: unit r = (gate row r, up row r).
template <int H, typename W>
__global__ __launch_bounds__(kBlock) void gateup_silu_kernel(
    const float *__restrict__ hidden, const float *__restrict__ gain,
    const W *__restrict__ wg, const W *__restrict__ wu,
    const SeqState *__restrict__ st, float *__restrict__ act, int inter,
    float eps) {
  if (st->stopped) return;
  float4 gv[PairSlots<H>::NJ];
  load_pair_gain<H>(gain, gv);
  float4 xv[PairSlots<H>::NJ];
  const float inv = norm_scale(load_pair_operand_gain<H>(Plain(hidden), gv, xv), H, eps);
  for (int r = blockIdx.x * kWavesPerBlock + wave_id(); r < inter;
       r += gridDim.x * kWavesPerBlock) {
    float gs, us;
    dot_pair<H, W>(wg + static_cast<size_t>(r) * H,
                   wu + static_cast<size_t>(r) * H, xv, gs, us);
    if (lane_id() == 0) act[r] = silu_mul(gs * inv, us * inv);
  }
}

// hidden[r] += Wd[r,:] . act; one row per wave, summed in the column slices
// of dot_row_sliced (the resident role kernel's arithmetic).
template <int H, int I, typename W>
__global__ __launch_bounds__(kBlock) void down_residual_kernel(
    const float *__restrict__ act, const W *__restrict__ wd,
    const SeqState *__restrict__ st, float *__restrict__ hidden) {
  if (st->stopped) return;
  float4 xv[RowSlots<I>::NJ];
  load_row_operand<I>(Plain(act), xv);
  for (int r = blockIdx.x * kWavesPerBlock + wave_id(); r < H;
       r += gridDim.x * kWavesPerBlock) {
    const float s = dot_row_sliced<I, W>(wd + static_cast<size_t>(r) * I, xv);
    if (lane_id() == 0) hidden[r] += s;
  }
}

// Final RMSNorm + LM head over row pairs + per-workgroup top-1 partial.
// Logits go to logits + (history ? generated * vocab : 0).
template <int H>
__global__ __launch_bounds__(kBlock) void lmhead_kernel(
    const float *__restrict__ hidden, const float *__restrict__ gain,
    const float *__restrict__ head, const SeqState *__restrict__ st,
    float *__restrict__ logits, int history, int vocab, float eps,
    float *__restrict__ part_val, uint32_t *__restrict__ part_idx) {
  __shared__ float bv[kWavesPerBlock];
  __shared__ uint32_t bi[kWavesPerBlock];
  if (st->stopped) return;
  float4 gv[PairSlots<H>::NJ];
  load_pair_gain<H>(gain, gv);
  float4 xv[PairSlots<H>::NJ];
  const float inv = norm_scale(load_pair_operand_gain<H>(Plain(hidden), gv, xv), H, eps);
  float *out = logits + (history ? static_cast<size_t>(st->generated) * vocab : 0);
  float best = -INFINITY;
  uint32_t best_i = UINT32_MAX;
  const int units = (vocab + 1) / 2;
  for (int u = blockIdx.x * kWavesPerBlock + wave_id(); u < units;
       u += gridDim.x * kWavesPerBlock) {
    const int r0 = 2 * u;
    const bool has1 = r0 + 1 < vocab;
    const float *a = head + static_cast<size_t>(r0) * H;
    float sa, sb;
    dot_pair<H>(a, has1 ? a + H : a, xv, sa, sb);
    sa *= inv;
    sb *= inv;
    if (lane_id() == 0) {
      out[r0] = sa;
      if (has1) out[r0 + 1] = sb;
    }
    if (better(sa, r0, best, best_i)) {
      best = sa;
      best_i = r0;
    }
    if (has1 && better(sb, r0 + 1, best, best_i)) {
      best = sb;
      best_i = r0 + 1;
    }
  }
  if (lane_id() == 0) {
    bv[wave_id()] = best;
    bi[wave_id()] = best_i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWavesPerBlock; ++w) {
      if (better(bv[w], bi[w], best, best_i)) {
        best = bv[w];
        best_i = bi[w];
      }
    }
    part_val[blockIdx.x] = best;
    part_idx[blockIdx.x] = best_i;
  }
}

// Reduces the top-1 partials, records the sampled token and advances the
// sequence (step mode), or applies the EOS / limit rule (generate mode).
__global__ __launch_bounds__(kBlock) void argmax_finalize_kernel(
    const float *__restrict__ part_val, const uint32_t *__restrict__ part_idx,
    int parts, SeqState *__restrict__ st, uint32_t *__restrict__ out_tokens) {
  __shared__ float bv[kWavesPerBlock];
  __shared__ uint32_t bi[kWavesPerBlock];
  if (st->stopped) return;
  float best = -INFINITY;
  uint32_t best_i = UINT32_MAX;
  for (int p = threadIdx.x; p < parts; p += kBlock) {
    if (better(part_val[p], part_idx[p], best, best_i)) {
      best = part_val[p];
      best_i = part_idx[p];
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
  st->token = best_i;
  st->top_logit = best;
  st->position += 1;
  if (best_i == UINT32_MAX) {
    // Every logit was NaN: nothing can be fed back.
    st->stop_reason = 0u;
    st->stopped = 1u;
    return;
  }
  if (st->mode == kModeGenerate) {
    if (out_tokens) out_tokens[st->generated] = best_i;
    st->generated += 1;
    const bool eos = best_i == st->eos;
    if (eos || st->generated >= st->max_tokens) {
      st->stop_reason = eos ? 2u : 1u;
      st->stopped = 1u;
    }
  }
}

// Writes a slot's decode state for a step-mode token at `position` from
// kernel arguments (no host buffer stays referenced after the launch).
__global__ void set_state_kernel(SeqState *__restrict__ st, uint32_t position, uint32_t token) {
  if (threadIdx.x != 0) return;
  SeqState s{};
  s.position = position;
  s.token = token;
  s.eos = UINT32_MAX;
  s.mode = kModeStep;
  *st = s;
}

// Every NaN of x[0, n) becomes the canonical quiet NaN 0x7FC00000, so no
// loaded value (nor any result derived from it: arithmetic propagates a NaN
// operand's payload) can equal the resident kernel's empty-slot pattern.
// A grid-stride loop over float4s plus the tail.
__global__ void canonical_nan_kernel(float *__restrict__ x, size_t n) {
  const size_t n4 = n / 4;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  float4 *x4 = reinterpret_cast<float4 *>(x);
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4; i += stride) {
    float4 v = x4[i];
    const bool any = __builtin_isnan(v.x) || __builtin_isnan(v.y) || __builtin_isnan(v.z) ||
                     __builtin_isnan(v.w);
    if (any) {
      const float q = __builtin_bit_cast(float, 0x7FC00000u);
      v.x = __builtin_isnan(v.x) ? q : v.x;
      v.y = __builtin_isnan(v.y) ? q : v.y;
      v.z = __builtin_isnan(v.z) ? q : v.z;
      v.w = __builtin_isnan(v.w) ? q : v.w;
      x4[i] = v;
    }
  }
  const size_t tail = n4 * 4 + static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (tail < n && __builtin_isnan(x[tail])) x[tail] = __builtin_bit_cast(float, 0x7FC00000u);
}

// HBM bandwidth probe: workgroups stream chunks of kProbeDepth * 256
// float4s (chunk c by workgroup c mod grid), every lane keeping kProbeDepth
// non-temporal 16-byte loads in flight; the copy variant stores each float4
// to `dst`, the read variant folds them into one value per workgroup.
constexpr int kProbeDepth = 16;
template <bool kCopy>
__global__ __launch_bounds__(kBlock) void hbm_probe_kernel(const float4 *__restrict__ src,
                                                           float4 *__restrict__ dst, size_t n4,
                                                           float *__restrict__ sink) {
  typedef float gf4 __attribute__((ext_vector_type(4)));
  typedef const __attribute__((address_space(1))) gf4 cg4;
  typedef __attribute__((address_space(1))) gf4 g4;
  const size_t chunk = static_cast<size_t>(kProbeDepth) * kBlock;
  float acc = 0.f;
  for (size_t base = static_cast<size_t>(blockIdx.x) * chunk; base < n4;
       base += static_cast<size_t>(gridDim.x) * chunk) {
    gf4 v[kProbeDepth];
#pragma unroll
    for (int d = 0; d < kProbeDepth; ++d) {
      const size_t i = base + static_cast<size_t>(d) * kBlock + threadIdx.x;
      v[d] = i < n4 ? __builtin_nontemporal_load((cg4 *)(src + i)) : gf4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int d = 0; d < kProbeDepth; ++d) {
      const size_t i = base + static_cast<size_t>(d) * kBlock + threadIdx.x;
      if (kCopy) {
        if (i < n4) __builtin_nontemporal_store(v[d], (g4 *)(dst + i));
      } else {
        acc += (v[d].x + v[d].y) + (v[d].z + v[d].w);
      }
    }
  }
  if (!kCopy && acc == 1.2345e30f) sink[blockIdx.x] = acc;  // keeps the loads
}

}  // namespace

// ---- host launchers -----------------------------------------------------------

hipError_t probe_hbm(int device, size_t bytes, uint32_t iters, double *read_gbs, double *copy_gbs) {
  *read_gbs = *copy_gbs = 0.0;
  int cus = 0;
  hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
  if (e != hipSuccess) return e;
  const size_t n4 = bytes / 16;
  float4 *a = nullptr, *b = nullptr;
  float *sink = nullptr;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  hipStream_t s = nullptr;
  auto cleanup = [&] {
    if (s) (void)hipStreamSynchronize(s);
    if (t0) (void)hipEventDestroy(t0);
    if (t1) (void)hipEventDestroy(t1);
    if (s) (void)hipStreamDestroy(s);
    if (a) (void)hipFree(a);
    if (b) (void)hipFree(b);
    if (sink) (void)hipFree(sink);
  };
  const unsigned grid = static_cast<unsigned>(std::max(cus, 1) * 8);
  if ((e = hipMalloc(&a, n4 * 16)) != hipSuccess || (e = hipMalloc(&b, n4 * 16)) != hipSuccess ||
      (e = hipMalloc(&sink, grid * sizeof(float))) != hipSuccess ||
      (e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking)) != hipSuccess ||
      (e = hipEventCreate(&t0)) != hipSuccess || (e = hipEventCreate(&t1)) != hipSuccess ||
      (e = hipMemsetAsync(a, 0, n4 * 16, s)) != hipSuccess) {
    cleanup();
    return e;
  }
  for (int copy = 0; copy < 2; ++copy) {
    double best = 0.0;
    for (uint32_t it = 0; it < iters + 1; ++it) {  // the first run warms up
      (void)hipEventRecord(t0, s);
      if (copy)
        hbm_probe_kernel<true><<<grid, kBlock, 0, s>>>(a, b, n4, sink);
      else
        hbm_probe_kernel<false><<<grid, kBlock, 0, s>>>(a, b, n4, sink);
      (void)hipEventRecord(t1, s);
      if ((e = hipStreamSynchronize(s)) != hipSuccess) {
        cleanup();
        return e;
      }
      float ms = 0.f;
      (void)hipEventElapsedTime(&ms, t0, t1);
      const double gbs = double(n4) * 16.0 * (copy ? 2.0 : 1.0) / (ms * 1e-3) / 1e9;
      if (it > 0) best = std::max(best, gbs);
    }
    (copy ? *copy_gbs : *read_gbs) = best;
  }
  cleanup();
  return hipGetLastError();
}

hipError_t launch_set_state(hipStream_t s, SeqState *st, uint32_t position, uint32_t token) {
  set_state_kernel<<<1, kWave, 0, s>>>(st, position, token);
  return hipGetLastError();
}

hipError_t launch_canonical_nan(hipStream_t s, float *x, size_t n) {
  if (n == 0) return hipSuccess;
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return hipErrorInvalidValue;
  const size_t blocks = std::min<size_t>((n / 4 + kBlock - 1) / kBlock + 1, 4096);
  canonical_nan_kernel<<<static_cast<unsigned>(blocks), kBlock, 0, s>>>(x, n);
  return hipGetLastError();
}

const char *kernel_name(int id) {
  static const char *const names[kKernelCount] = {
      "embed_kernel",         "qkv_rope_kernel",   "attn_partial_kernel",
      "attn_combine_kernel",  "oproj_residual_kernel", "gateup_silu_kernel",
      "down_residual_kernel", "lmhead_kernel",     "argmax_finalize_kernel"};
  return id >= 0 && id < kKernelCount ? names[id] : "unknown";
}

bool shape_supported(int hidden, int intermediate, int heads, int kv_heads,
                     int head_dim) {
  // The Qwen2.5-0.5B layer, the one shape whose parity the kernels are
  // tested at: 14 query heads over 2 KV heads of 64.
  return hidden == 896 && intermediate == 4864 && head_dim == kHeadDim && heads == 14 &&
         kv_heads == 2;
}

namespace {
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
}  // namespace

hipError_t launch_embed(hipStream_t s, const float *emb, const SeqState *st,
                        float *hidden, int hidden_size, int vocab, Marker *m) {
  Scope scope(m, kKEmbed);
  embed_kernel<<<(hidden_size + kBlock - 1) / kBlock, kBlock, 0, s>>>(
      emb, st, hidden, hidden_size, vocab);
  return hipGetLastError();
}

namespace {

// One layer's launches with the decoder matrices read as W (float, Bf16 or F16).
template <typename W>
hipError_t launch_layer_as(hipStream_t s, const LayerLaunch &p, Marker *m) {
  const W *wqkv = reinterpret_cast<const W *>(p.w.wqkv);
  const W *wo = reinterpret_cast<const W *>(p.w.wo);
  const W *wg = reinterpret_cast<const W *>(p.w.wg);
  const W *wu = reinterpret_cast<const W *>(p.w.wu);
  const W *wd = reinterpret_cast<const W *>(p.w.wd);
  constexpr int H = 896, I = 4864, QD = 896;
  const int qkv_units = (p.nq + 2 * p.nkv) * kRotary;
  {
    Scope scope(m, kKQkvRope);
    qkv_rope_kernel<H, W><<<(qkv_units + kWavesPerBlock - 1) / kWavesPerBlock,
                            kBlock, 0, s>>>(
        p.hidden, p.w.attn_norm, wqkv, p.w.bqkv, p.rope_cos, p.rope_sin,
        p.st, p.q, p.k_cache, p.v_cache, p.nq, p.nkv, p.eps, p.capacity);
  }
  {
    Scope scope(m, kKAttnPartial);
    if (p.attn_parts < 1 || p.attn_parts > kAttnMaxChunks) return hipErrorInvalidValue;
    if (p.nq / p.nkv > kAttnMaxGroup) return hipErrorInvalidValue;
    attn_partial_kernel<<<dim3(p.attn_parts, p.nkv), kAttnThreads, 0, s>>>(
        p.q, p.k_cache, p.v_cache, p.st, p.nq, p.nkv, p.part, p.capacity, p.attn_parts);
  }
  {
    Scope scope(m, kKAttnCombine);
    attn_combine_kernel<<<p.nq, kHeadDim, 0, s>>>(p.part, p.st, p.nq, p.attn,
                                                  p.capacity, p.attn_parts);
  }
  {
    Scope scope(m, kKOproj);
    const dim3 grid((H / 2 + kWavesPerBlock - 1) / kWavesPerBlock);
    // Two KV groups (shape_supported).
    if (p.nkv != 2) return hipErrorInvalidValue;
    oproj_residual_kernel<H, QD, 2, W><<<grid, kBlock, 0, s>>>(p.attn, wo, p.st, p.hidden);
  }
  {
    Scope scope(m, kKGateUp);
    gateup_silu_kernel<H, W><<<(I + kWavesPerBlock - 1) / kWavesPerBlock, kBlock,
                               0, s>>>(p.hidden, p.w.mlp_norm, wg, wu, p.st, p.act, I, p.eps);
  }
  {
    Scope scope(m, kKDown);
    down_residual_kernel<H, I, W><<<(H + kWavesPerBlock - 1) / kWavesPerBlock,
                                    kBlock, 0, s>>>(p.act, wd, p.st, p.hidden);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_layer(hipStream_t s, const LayerLaunch &p, Marker *m) {
  switch (p.weights_dtype) {
    case kWeightsF32: return launch_layer_as<float>(s, p, m);
    case kWeightsBf16: return launch_layer_as<Bf16>(s, p, m);
    case kWeightsF16: return launch_layer_as<F16>(s, p, m);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_tail(hipStream_t s, const TailLaunch &p, Marker *m) {
  constexpr int H = 896;
  {
    Scope scope(m, kKLmHead);
    lmhead_kernel<H><<<p.parts, kBlock, 0, s>>>(
        p.hidden, p.final_norm, p.head, p.st, p.logits, p.history, p.vocab,
        p.eps, p.part_val, p.part_idx);
  }
  {
    Scope scope(m, kKArgmax);
    argmax_finalize_kernel<<<1, kBlock, 0, s>>>(p.part_val, p.part_idx,
                                                p.parts, p.st, p.out_tokens);
  }
  return hipGetLastError();
}

}  // namespace qd
