// Resident decode megakernel: one cooperative launch runs every token of a
// greedy generation -- all decoder layers, the LM head, the argmax and the
// embedding feedback -- with the grid synchronised by flag barriers instead
// of kernel boundaries. This is the MI355X counterpart of the reference's
// persistent-graph resident loop (include/lrrt/persistent_graph/
// compiled_scheduler.hpp:108-217 driving benchmarks/
// qwen_stateful_graph_kernel.cpp:661-1083), reorganised around what the
// hardware measures: a flag barrier across 256 CUs costs ~1.5 us, so the
// step is cut into five barrier-separated stages per layer and the argmax is
// recomputed by every workgroup instead of paying another barrier.
//
// Stage map per layer (every stage distributes whole output rows over all
// waves of the grid; cross-workgroup data moves through sc1 buffer accesses):
//   A  attention RMSNorm + packed QKV + bias + RoPE + KV-cache write
//   B  split-KV GQA attention partials; the last chunk of each KV group
//      merges the partials (device-scope arrival counter)
//   C  O projection + residual          h1 = h0 + Wo attn
//   D  MLP RMSNorm + gate/up + SiLU     act
//   E  down projection + residual       hidden = h1 + Wd act
// Tail: final RMSNorm + LM head + per-workgroup top-1, then every workgroup
// reduces the partials to the sampled token.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "qd_device.hpp"
#include "qd_device_math.hpp"
#include "qd_resident.hpp"

namespace qd {
namespace {

using namespace dev;

constexpr uint32_t kSpinLimit = 1u << 20;  // polls before a barrier gives up

// Grid barrier: workgroup b publishes its generation in flags[b]; every
// workgroup waits until all flags reached the generation. Each wait is
// bounded; a timeout raises the error word and the kernel winds down.
struct FlagBarrier {
  Coherent flags;
  uint32_t count;
  uint32_t gen = 0;
  uint32_t *error;
  bool failed = false;

  __device__ FlagBarrier(uint32_t *f, uint32_t n, uint32_t *err)
      : flags(f, n * 4u), count(n), error(err) {}

  __device__ bool sync() {
    ++gen;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores are performed
    __syncthreads();
    if (threadIdx.x == 0) flags.stu(blockIdx.x, gen);
    for (uint32_t spins = 0;; ++spins) {
      bool ok = true;
      for (uint32_t i = threadIdx.x; i < count; i += blockDim.x)
        ok &= flags.ldu(i) >= gen;
      if (__syncthreads_and(ok)) return true;
      if (spins > kSpinLimit) {
        if (threadIdx.x == 0) atomicOr(error, 1u);
        failed = true;
        return false;
      }
    }
  }
};

struct EmbedRow {  // read-only embedding row as an activation source
  const float *p;
  __device__ float ld(uint32_t i) const { return p[i]; }
  __device__ float4 ld4(uint32_t i4) const {
    return reinterpret_cast<const float4 *>(p)[i4];
  }
};

template <int H, typename Src>
__device__ void stage_qkv(const ResidentArgs &a, const LayerPtrs &w,
                          const Src &h0, int position, float *kc, float *vc,
                          float *red) {
  const int units = (a.nq + 2 * a.nkv) * kRotary;
  if (static_cast<int>(blockIdx.x) * kWavesPerBlock >= units) return;
  const float inv = block_inv_rms<H>(h0, a.eps, red);
  float4 xv[PairSlots<H>::NJ];
  load_pair_operand<H, true>(h0, inv, w.attn_norm, xv);
  const int kv_dim = a.nkv * kHeadDim;
  const Coherent q(a.q, a.nq * kHeadDim * 4u);
  const Coherent kcache(kc, static_cast<uint32_t>(a.capacity) * kv_dim * 4u);
  const Coherent vcache(vc, static_cast<uint32_t>(a.capacity) * kv_dim * 4u);
  const int nwaves = gridDim.x * kWavesPerBlock;
  for (int u = blockIdx.x * kWavesPerBlock + wave_id(); u < units; u += nwaves) {
    const int head = u / kRotary;
    const int i = u % kRotary;
    const int ra = head * kHeadDim + i;
    const int rb = ra + kRotary;
    float sa, sb;
    dot_pair<H>(w.wqkv + static_cast<size_t>(ra) * H,
                w.wqkv + static_cast<size_t>(rb) * H, xv, sa, sb);
    if (lane_id() == 0) {
      const float x0 = sa + w.bqkv[ra];
      const float x1 = sb + w.bqkv[rb];
      if (head < a.nq + a.nkv) {
        const float c = a.rope_cos[position * kRotary + i];
        const float s = a.rope_sin[position * kRotary + i];
        const float first = x0 * c - x1 * s;
        const float second = x1 * c + x0 * s;
        if (head < a.nq) {
          q.st(ra, first);
          q.st(rb, second);
        } else {
          const uint32_t base = position * kv_dim + (head - a.nq) * kHeadDim + i;
          kcache.st(base, first);
          kcache.st(base + kRotary, second);
        }
      } else {
        const uint32_t base = position * kv_dim + (head - a.nq - a.nkv) * kHeadDim + i;
        vcache.st(base, x0);
        vcache.st(base + kRotary, x1);
      }
    }
  }
}

struct AttnShared {
  float qs[kMaxGroup * kHeadDim];
  float red[kWavesPerBlock];
  float acc_red[kWavesPerBlock][kHeadDim];
  float scale[kMaxGroup][80];  // per-chunk merge weights (chunks <= 80)
  float den[kMaxGroup];
  int last;
};

// Workgroup unit (KV group g, chunk c): online-softmax partial over the
// chunk's positions for every query head of the group. The workgroup that
// completes a group's last chunk merges the group's partials into attn.
__device__ void attention_unit(const ResidentArgs &a, const float *kc,
                               const float *vc, int length, int chunks,
                               uint32_t target, AttnShared &sh, int u) {
  const int g = u / chunks;
  const int chunk = u % chunks;
  const int group = a.nq / a.nkv;
  const int kv_dim = a.nkv * kHeadDim;
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int quarter = t & 3;
  const int j = chunk * kAttnChunk + (t >> 2);
  const bool valid = j < length;
  const Coherent q(a.q, a.nq * kHeadDim * 4u);
  const Coherent kcache(kc, static_cast<uint32_t>(a.capacity) * kv_dim * 4u);
  const Coherent vcache(vc, static_cast<uint32_t>(a.capacity) * kv_dim * 4u);
  const Coherent pm(a.part_m, a.max_chunks * a.nq * 4u);
  const Coherent pl(a.part_l, a.max_chunks * a.nq * 4u);
  const Coherent pacc(a.part_acc, a.max_chunks * a.nq * kHeadDim * 4u);

  for (int e = t; e < group * kHeadDim; e += kBlock)
    sh.qs[e] = q.ld(g * group * kHeadDim + e);
  float4 kr[4], vr[4];
  const uint32_t row4 = ((valid ? j : 0) * kv_dim + g * kHeadDim + quarter * 16) / 4;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    kr[e] = kcache.ld4(row4 + e);
    vr[e] = vcache.ld4(row4 + e);
  }
  __syncthreads();

  for (int hl = 0; hl < group; ++hl) {
    const float4 *q4 =
        reinterpret_cast<const float4 *>(sh.qs + hl * kHeadDim + quarter * 16);
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) s = fma4(kr[e], q4[e], s);
    s += __shfl_xor(s, 1, kWave);
    s += __shfl_xor(s, 2, kWave);
    s = valid ? s * rsqrtf(static_cast<float>(kHeadDim)) : -INFINITY;
    float m = s;
#pragma unroll
    for (int o = 4; o < kWave; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
    if (lane == 0) sh.red[wave_id()] = m;
    __syncthreads();
    m = fmaxf(fmaxf(sh.red[0], sh.red[1]), fmaxf(sh.red[2], sh.red[3]));
    __syncthreads();
    const float p = valid ? expf(s - m) : 0.f;
    float l = p;
#pragma unroll
    for (int o = 4; o < kWave; o <<= 1) l += __shfl_xor(l, o, kWave);
    if (lane == 0) sh.red[wave_id()] = l;
    float acc[16];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[4 * e + 0] = p * vr[e].x;
      acc[4 * e + 1] = p * vr[e].y;
      acc[4 * e + 2] = p * vr[e].z;
      acc[4 * e + 3] = p * vr[e].w;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
#pragma unroll
      for (int o = 4; o < kWave; o <<= 1) acc[e] += __shfl_xor(acc[e], o, kWave);
    }
    if (lane < 4) {
#pragma unroll
      for (int e = 0; e < 16; ++e) sh.acc_red[wave_id()][quarter * 16 + e] = acc[e];
    }
    __syncthreads();
    const int h = g * group + hl;
    if (t < kHeadDim) {
      float sum = 0.f;
#pragma unroll
      for (int w = 0; w < kWavesPerBlock; ++w) sum += sh.acc_red[w][t];
      pacc.st((chunk * a.nq + h) * kHeadDim + t, sum);
    }
    if (t == 0) {
      pm.st(chunk * a.nq + h, m);
      pl.st(chunk * a.nq + h, sh.red[0] + sh.red[1] + sh.red[2] + sh.red[3]);
    }
    __syncthreads();
  }

  // Arrival on the group's counter; the last arriver merges.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    const uint32_t old = __hip_atomic_fetch_add(a.group_count + g * 64, 1u,
                                                __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    sh.last = old + 1u == target;
  }
  __syncthreads();
  if (!sh.last) return;

  // Merge weights per (head, chunk) into LDS, then one output per thread.
  if (t < group) {
    const int h = g * group + t;
    float mx = -INFINITY;
    for (int c = 0; c < chunks; ++c) mx = fmaxf(mx, pm.ld(c * a.nq + h));
    float den = 0.f;
    for (int c = 0; c < chunks; ++c) {
      const float sc = expf(pm.ld(c * a.nq + h) - mx);
      sh.scale[t][c] = sc;
      den = fmaf(sc, pl.ld(c * a.nq + h), den);
    }
    sh.den[t] = den;
  }
  __syncthreads();
  const Coherent attn(a.attn, a.nq * kHeadDim * 4u);
  for (int e = t; e < group * kHeadDim; e += kBlock) {
    const int hl = e / kHeadDim;
    const int d = e % kHeadDim;
    const int h = g * group + hl;
    float num = 0.f;
    for (int c = 0; c < chunks; ++c)
      num = fmaf(sh.scale[hl][c], pacc.ld((c * a.nq + h) * kHeadDim + d), num);
    attn.st(h * kHeadDim + d, num / sh.den[hl]);
  }
}

__device__ void stage_attention(const ResidentArgs &a, const float *kc,
                                const float *vc, int length, int chunks,
                                uint32_t target, AttnShared &sh) {
  const int units = a.nkv * chunks;
  for (int u = blockIdx.x; u < units; u += gridDim.x)
    attention_unit(a, kc, vc, length, chunks, target, sh, u);
}

template <int H, int QD, typename Src>
__device__ void stage_oproj(const ResidentArgs &a, const LayerPtrs &w,
                            const Src &h0) {
  constexpr int units = H / 2;
  if (static_cast<int>(blockIdx.x) * kWavesPerBlock >= units) return;
  float4 xv[PairSlots<QD>::NJ];
  load_pair_operand<QD, false>(Coherent(a.attn, QD * 4u), 1.f, nullptr, xv);
  const Coherent h1(a.h1, H * 4u);
  const int nwaves = gridDim.x * kWavesPerBlock;
  for (int u = blockIdx.x * kWavesPerBlock + wave_id(); u < units; u += nwaves) {
    const float *row = w.wo + static_cast<size_t>(2 * u) * QD;
    float sa, sb;
    dot_pair<QD>(row, row + QD, xv, sa, sb);
    if (lane_id() == 0) {
      h1.st(2 * u, h0.ld(2 * u) + sa);
      h1.st(2 * u + 1, h0.ld(2 * u + 1) + sb);
    }
  }
}

template <int H>
__device__ void stage_gateup(const ResidentArgs &a, const LayerPtrs &w,
                             const int inter, float *red) {
  const Coherent h1(a.h1, H * 4u);
  const float inv = block_inv_rms<H>(h1, a.eps, red);
  float4 xv[PairSlots<H>::NJ];
  load_pair_operand<H, true>(h1, inv, w.mlp_norm, xv);
  const Coherent act(a.act, inter * 4u);
  const int nwaves = gridDim.x * kWavesPerBlock;
  for (int r = blockIdx.x * kWavesPerBlock + wave_id(); r < inter; r += nwaves) {
    float g, up;
    dot_pair<H>(w.wg + static_cast<size_t>(r) * H,
                w.wu + static_cast<size_t>(r) * H, xv, g, up);
    if (lane_id() == 0) act.st(r, g / (1.f + expf(-g)) * up);
  }
}

template <int H, int I>
__device__ void stage_down(const ResidentArgs &a, const LayerPtrs &w) {
  if (static_cast<int>(blockIdx.x) * kWavesPerBlock >= H) return;
  float4 xv[RowSlots<I>::NJ];
  load_row_operand<I>(Coherent(a.act, I * 4u), xv);
  const Coherent h1(a.h1, H * 4u);
  const Coherent hidden(a.hidden, H * 4u);
  const int nwaves = gridDim.x * kWavesPerBlock;
  for (int r = blockIdx.x * kWavesPerBlock + wave_id(); r < H; r += nwaves) {
    const float s = dot_row<I>(w.wd + static_cast<size_t>(r) * I, xv);
    if (lane_id() == 0) hidden.st(r, h1.ld(r) + s);
  }
}

template <int H>
__device__ void stage_lmhead(const ResidentArgs &a, float *logits, float *red,
                             float *bv, uint32_t *bi) {
  const Coherent hidden(a.hidden, H * 4u);
  const float inv = block_inv_rms<H>(hidden, a.eps, red);
  float4 xv[PairSlots<H>::NJ];
  load_pair_operand<H, true>(hidden, inv, a.final_norm, xv);
  float best = -INFINITY;
  uint32_t best_i = UINT32_MAX;
  const int units = (a.vocab + 1) / 2;
  const int nwaves = gridDim.x * kWavesPerBlock;
  for (int u = blockIdx.x * kWavesPerBlock + wave_id(); u < units; u += nwaves) {
    const int r0 = 2 * u;
    const bool has1 = r0 + 1 < a.vocab;
    const float *row = a.head + static_cast<size_t>(r0) * H;
    float sa, sb;
    dot_pair<H>(row, has1 ? row + H : row, xv, sa, sb);
    if (lane_id() == 0) {
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
    Coherent(a.top_val, gridDim.x * 4u).st(blockIdx.x, best);
    Coherent(a.top_idx, gridDim.x * 4u).stu(blockIdx.x, best_i);
  }
}

// Every workgroup reduces the per-workgroup top-1 partials (same order, same
// result everywhere).
__device__ void reduce_top1(const ResidentArgs &a, float *bv, uint32_t *bi,
                            float &best, uint32_t &best_i) {
  const Coherent tv(a.top_val, gridDim.x * 4u);
  const Coherent ti(a.top_idx, gridDim.x * 4u);
  best = -INFINITY;
  best_i = UINT32_MAX;
  for (uint32_t p = threadIdx.x; p < gridDim.x; p += blockDim.x) {
    const float v = tv.ld(p);
    const uint32_t i = ti.ldu(p);
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
  if (lane_id() == 0) {
    bv[wave_id()] = best;
    bi[wave_id()] = best_i;
  }
  __syncthreads();
  best = bv[0];
  best_i = bi[0];
  for (int w = 1; w < kWavesPerBlock; ++w) {
    if (better(bv[w], bi[w], best, best_i)) {
      best = bv[w];
      best_i = bi[w];
    }
  }
  __syncthreads();
}

// Stage clock of the profiled instantiation: workgroup 0 stamps every
// barrier exit with the 100 MHz wall clock, so a stage's time is its
// slowest workgroup's work plus the barrier that ends it.
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

template <int H, int I, int QD, bool kProfile>
__global__ __launch_bounds__(kBlock) void resident_decode_kernel(ResidentArgs a) {
  __shared__ AttnShared attn_sh;
  __shared__ float red[kWavesPerBlock];
  __shared__ float bv[kWavesPerBlock];
  __shared__ uint32_t bi[kWavesPerBlock];
  FlagBarrier bar(a.flags, gridDim.x, a.error);
  const int kv_dim = a.nkv * kHeadDim;
  uint32_t token = a.first_token;
  uint32_t generated = 0;
  uint32_t stop_reason = 0;
  uint32_t group_target = 0;
  float top = 0.f;
  StageClock<kProfile> clock;
  clock.start();

  for (uint32_t t = 0; t < a.max_tokens; ++t) {
    const int position = static_cast<int>(a.start_position + t);
    if (token >= static_cast<uint32_t>(a.vocab) || position >= a.capacity) break;
    const int length = position + 1;
    const int chunks = (length + kAttnChunk - 1) / kAttnChunk;
    const EmbedRow embed_row{a.embed + static_cast<size_t>(token) * H};
    for (int l = 0; l < a.layers; ++l) {
      const LayerPtrs w = a.layer_ptrs[l];
      float *kc = a.k_cache + static_cast<size_t>(l) * a.capacity * kv_dim;
      float *vc = a.v_cache + static_cast<size_t>(l) * a.capacity * kv_dim;
      const Coherent hidden(a.hidden, H * 4u);
      if (l == 0) {
        stage_qkv<H>(a, w, embed_row, position, kc, vc, red);
      } else {
        stage_qkv<H>(a, w, hidden, position, kc, vc, red);
      }
      if (!bar.sync()) return;
      clock.lap(0);
      group_target += static_cast<uint32_t>(chunks);
      stage_attention(a, kc, vc, length, chunks, group_target, attn_sh);
      if (!bar.sync()) return;
      clock.lap(1);
      if (l == 0) {
        stage_oproj<H, QD>(a, w, embed_row);
      } else {
        stage_oproj<H, QD>(a, w, hidden);
      }
      if (!bar.sync()) return;
      clock.lap(2);
      stage_gateup<H>(a, w, I, red);
      if (!bar.sync()) return;
      clock.lap(3);
      stage_down<H, I>(a, w);
      if (!bar.sync()) return;
      clock.lap(4);
    }
    float *logits = a.logits + (a.history ? static_cast<size_t>(t) * a.vocab : 0);
    stage_lmhead<H>(a, logits, red, bv, bi);
    if (!bar.sync()) return;
    clock.lap(5);
    uint32_t next;
    reduce_top1(a, bv, bi, top, next);
    clock.lap(6);
    token = next;
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
