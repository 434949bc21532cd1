// Device helpers shared by the stream-ordered kernels (qd_kernels.hip) and
// the resident megakernel (qd_roles.hip): wave64 reductions, the float4
// slot layout of the row-pair GEMV, and device-coherent buffer access.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qd_device.hpp"

namespace qd {
namespace dev {

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / kWave; }

// Cross-lane moves inside a 16-lane row (DPP), fused by the compiler into
// the consuming VALU op.
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <- lane 7-i of its 8-lane half
constexpr int kDppMirror = 0x140;     // lane i <- lane 15-i of its row

template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}

__device__ __forceinline__ float read_lane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Wave64 sum and max with the result in every lane (a wave-uniform value).
// The whole wave must be active. Rows reduce through DPP (xor 1, xor 2,
// half-row mirror, row mirror), then the four row results are combined in a
// fixed order: (r0 + r1) + (r2 + r3).
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return (read_lane(v, 0) + read_lane(v, 16)) + (read_lane(v, 32) + read_lane(v, 48));
}

// Value of lane l ^ 4 (kX = 4) or l ^ 8 (kX = 8) inside each row of 16: two
// bank-masked row shifts (a bank is a quarter row). The row shifts only
// ever read lanes of the same row.
template <int kX>
__device__ __forceinline__ float dpp_row_xor(float v) {
  static_assert(kX == 4 || kX == 8, "row xor");
  constexpr int kShr = 0x110 + kX, kShl = 0x100 + kX;
  constexpr int kHiBanks = kX == 4 ? 0xA : 0xC, kLoBanks = kX == 4 ? 0x5 : 0x3;
  const int x = __builtin_bit_cast(int, v);
  int t = __builtin_amdgcn_update_dpp(x, x, kShr, 0xf, kHiBanks, false);
  t = __builtin_amdgcn_update_dpp(t, x, kShl, 0xf, kLoBanks, false);
  return __builtin_bit_cast(float, t);
}

// One halving step of wave_sum_multi: pairs of values (2i, 2i + 1); the lane
// whose bit is set keeps the odd one, its partner the even one, and each
// adds the partner's copy of the value it keeps.
template <int N, typename Ex>
__device__ __forceinline__ void wave_sum_halve(float (&v)[16], bool bit, Ex ex) {
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float keep = bit ? v[2 * i + 1] : v[2 * i];
    const float send = bit ? v[2 * i] : v[2 * i + 1];
    v[i] = keep + ex(send);
  }
}

// Wave sums of N values at once (N a power of two, at most 16). The lanes
// are grouped exactly as wave_sum groups them (pairs, quads, octets, rows of
// 16, then (row 0 + row 1) + (row 2 + row 3)) and addition is commutative,
// so each sum is bit-identical to wave_sum of that value; the exchanges are
// shared between the values (about 4 instructions per value instead of
// about 15). Value k ends in lanes k, k + 16, k + 32 and k + 48 (lane l
// holds value l mod N).
template <int N>
__device__ __forceinline__ float wave_sum_multi(const float (&in)[N]) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16, "power of two up to 16");
  const int lane = lane_id();
  float v[16];
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = in[i];
  auto x1 = [](float y) { return dpp<kDppXor1>(y); };
  auto x2 = [](float y) { return dpp<kDppXor2>(y); };
  auto x4 = [](float y) { return dpp_row_xor<4>(y); };
  auto x8 = [](float y) { return dpp_row_xor<8>(y); };
  if constexpr (N >= 2) wave_sum_halve<N>(v, lane & 1, x1); else v[0] += x1(v[0]);
  if constexpr (N >= 4) wave_sum_halve<N / 2>(v, lane & 2, x2); else v[0] += x2(v[0]);
  if constexpr (N >= 8) wave_sum_halve<N / 4>(v, lane & 4, x4); else v[0] += x4(v[0]);
  if constexpr (N >= 16) wave_sum_halve<N / 8>(v, lane & 8, x8); else v[0] += x8(v[0]);
  float r = v[0];
  r += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 16) << 2, __builtin_bit_cast(int, r)));
  r += __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, r)));
  return r;
}

// Rotary rotation of the pair (a, b) by (c, s): (a c - b s, b c + a s), each
// half as one rounded product and one fused multiply-add, so every kernel
// that rotates gets the same bits whatever its compiler would contract.
__device__ __forceinline__ void rope_rotate(float a, float b, float c, float s, float &first,
                                            float &second) {
  first = fmaf(a, c, -__fmul_rn(b, s));
  second = fmaf(b, c, __fmul_rn(a, s));
}

// Max and sum over each row of 16 lanes, the result in every lane of the
// row: wave_max's and wave_sum's first four steps. The sum groups the lanes
// as a pairwise tree ((v0 + v1) + (v2 + v3)) + ((v4 + v5) + (v6 + v7)), and
// likewise for lanes 8..15, then the two halves.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  return fmaxf(v, dpp<kDppMirror>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  return v + dpp<kDppMirror>(v);
}

// Max and sum over each half of the wave (32 lanes: rows 0-1 and rows 2-3),
// the result in every lane of the half: row16_max / row16_sum, then the two
// rows of a half exchanged by v_permlane16_swap_b32 on two copies of the
// value (row 1 of the first <-> row 0 of the second, row 3 <-> row 2). The
// swap is issued from inline assembly: the compiler's intrinsic for it
// folds the second result into the first at -O3. The s_nop gives the two
// wait states the swap needs after a VALU write of its operands.
__device__ __forceinline__ void row_pair_swap(float v, float &a, float &b) {
  unsigned x = __builtin_bit_cast(unsigned, v), y = x;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(x), "+v"(y));
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}
__device__ __forceinline__ float row_pair_max(float v) {
  float a, b;
  row_pair_swap(v, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float row_pair_sum(float v) {
  float a, b;
  row_pair_swap(v, a, b);
  return a + b;
}
__device__ __forceinline__ float half_max(float v) { return row_pair_max(row16_max(v)); }
__device__ __forceinline__ float half_sum(float v) { return row_pair_sum(row16_sum(v)); }

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  return fmaxf(fmaxf(read_lane(v, 0), read_lane(v, 16)), fmaxf(read_lane(v, 32), read_lane(v, 48)));
}

// Sum over the four lanes of a quad (lanes 4k..4k+3), in every lane of it.
__device__ __forceinline__ float quad_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  return v;
}

__device__ __forceinline__ float fma4(float4 w, float4 x, float acc) {
  acc = fmaf(w.x, x.x, acc);
  acc = fmaf(w.y, x.y, acc);
  acc = fmaf(w.z, x.z, acc);
  acc = fmaf(w.w, x.w, acc);
  return acc;
}

// SwiGLU of one intermediate row: silu(g) * u with silu(g) = g / (1 + e^-g)
// (benchmarks/qwen_stateful_graph_kernel.cpp:512).
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.f + expf(-g)) * u; }

// Greater value wins; equal values go to the lower index; NaN never wins
// (benchmarks/qwen_stateful_graph_kernel.cpp:225-229).
__device__ __forceinline__ bool better(float v, uint32_t i, float bv,
                                       uint32_t bi) {
  return v > bv || (v == bv && i < bi);
}

// ---- device-coherent access ------------------------------------------------
// Data one workgroup writes and another reads inside the same resident launch
// goes through buffer instructions with the sc1 (device scope) policy: loads
// are served coherently across the XCDs' private L2s and stores write
// through, so no L2 writeback/invalidate is needed at the grid barriers. The
// descriptor's record count also bounds every access (out-of-range loads
// return 0, out-of-range stores are dropped).
constexpr int kPolicySc1 = 16;
constexpr int kPolicyNt = 2;
constexpr int kRsrcWord3 = 0x00020000;

typedef unsigned int u32x4 __attribute__((vector_size(16)));
typedef float f32x4 __attribute__((vector_size(16)));

struct Coherent {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ Coherent(const void *base, uint32_t bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0,
                                            static_cast<int>(bytes),
                                            kRsrcWord3)) {}
  __device__ __forceinline__ float ld(uint32_t i) const {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(r, i * 4u, 0, kPolicySc1));
  }
  __device__ __forceinline__ uint32_t ldu(uint32_t i) const {
    return __builtin_amdgcn_raw_buffer_load_b32(r, i * 4u, 0, kPolicySc1);
  }
  // The whole vector is bit-cast at once: bit-casting individual elements of
  // the builtin's result folds every lane to element 0 in this compiler.
  __device__ __forceinline__ float4 ld4(uint32_t i4) const {
    const f32x4 v = __builtin_bit_cast(
        f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, i4 * 16u, 0, kPolicySc1));
    return make_float4(v[0], v[1], v[2], v[3]);
  }
  __device__ __forceinline__ void st(uint32_t i, float v) const {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r,
                                          i * 4u, 0, kPolicySc1);
  }
  __device__ __forceinline__ void st4(uint32_t i4, float4 v) const {
    const f32x4 x = {v.x, v.y, v.z, v.w};
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), r, i4 * 16u, 0, kPolicySc1);
  }
  __device__ __forceinline__ void stu(uint32_t i, uint32_t v) const {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, i * 4u, 0, kPolicySc1);
  }
};

// Plain pointer view with the same interface (stream-ordered kernels, where
// kernel boundaries order everything).
struct Plain {
  const float *p;
  __device__ __forceinline__ Plain(const float *base) : p(base) {}
  __device__ __forceinline__ float ld(uint32_t i) const { return p[i]; }
  __device__ __forceinline__ float4 ld4(uint32_t i4) const {
    return reinterpret_cast<const float4 *>(p)[i4];
  }
};

// Streaming weight load: each weight is read once per token, so the load is
// non-temporal (it does not displace cached lines: code, activations). The
// pointer is taken as global memory so the load is a global_load (vmcnt
// only); a flat load would also hold lgkmcnt, making every LDS wait behind
// it wait for the weights in flight too.
typedef float gf32x4 __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) gf32x4 global_f32x4;
__device__ __forceinline__ float4 ld_weight(const float4 *p) {
  const gf32x4 v = __builtin_nontemporal_load((global_f32x4 *)p);
  return make_float4(v.x, v.y, v.z, v.w);
}

// BF16 weights (the decoder's matrices of an engine created with BF16
// decoder weights): four consecutive BF16 values, 8 bytes, loaded as one
// non-temporal load and widened exactly to FP32 (a BF16 value is the top 16
// bits of its FP32 value). Every GEMV helper below takes its weight rows as
// float or as Bf16 and runs the same FP32 arithmetic either way.
struct Bf16 {
  uint16_t bits;
};
struct alignas(8) Bf16x4 {
  uint32_t lo, hi;  // elements (0, 1) and (2, 3), low half first
};
typedef uint32_t gu32x2 __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(1))) gu32x2 global_u32x2;
__device__ __forceinline__ float4 ld_weight(const Bf16x4 *p) {
  const gu32x2 v = __builtin_nontemporal_load((global_u32x2 *)p);
  return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xFFFF0000u),
                     __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xFFFF0000u));
}
// FP16 weights: four consecutive IEEE half values, 8 bytes, widened exactly
// to FP32 (every half is an FP32 value).
struct F16 {
  uint16_t bits;
};
struct alignas(8) F16x4 {
  uint32_t lo, hi;  // elements (0, 1) and (2, 3), low half first
};
__device__ __forceinline__ float half_lo(uint32_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v & 0xFFFFu)));
}
__device__ __forceinline__ float half_hi(uint32_t v) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v >> 16)));
}
__device__ __forceinline__ float4 ld_weight(const F16x4 *p) {
  const gu32x2 v = __builtin_nontemporal_load((global_u32x2 *)p);
  return make_float4(half_lo(v.x), half_hi(v.x), half_lo(v.y), half_hi(v.y));
}
// The four-element slot type of a weight row of W.
template <typename W>
struct WSlot;
template <>
struct WSlot<float> {
  using type = float4;
};
template <>
struct WSlot<Bf16> {
  using type = Bf16x4;
};
template <>
struct WSlot<F16> {
  using type = F16x4;
};

// A weight slot as the resident kernel keeps it in registers and LDS: the
// stored bits (16 bytes of FP32, 8 bytes of BF16 or FP16), widened to the
// FP32 float4 only where it is multiplied.
template <typename W>
struct WReg;
template <>
struct WReg<float> {
  using type = float4;
  __device__ static float4 widen(float4 r) { return r; }
  __device__ static float4 zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
};
template <>
struct WReg<Bf16> {
  using type = uint2;
  __device__ static float4 widen(uint2 r) {
    return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xFFFF0000u),
                       __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xFFFF0000u));
  }
  __device__ static uint2 zero() { return make_uint2(0u, 0u); }
};
template <>
struct WReg<F16> {
  using type = uint2;
  __device__ static float4 widen(uint2 r) {
    return make_float4(half_lo(r.x), half_hi(r.x), half_lo(r.y), half_hi(r.y));
  }
  __device__ static uint2 zero() { return make_uint2(0u, 0u); }
};
// Pins v in registers at this point: the compiler may not move the
// computation that produced it (a widening) into the instructions that use
// it later (where it would become mixed-precision FMAs on the critical path).
__device__ __forceinline__ float4 pin(float4 v) {
  asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
  return v;
}
// Non-temporal load of one stored slot (no widening).
__device__ __forceinline__ float4 ld_slot(const float4 *p) { return ld_weight(p); }
template <typename S>
__device__ __forceinline__ uint2 ld_slot(const S *p) {
  static_assert(sizeof(S) == 8, "a 16-bit slot is 8 bytes");
  const gu32x2 v = __builtin_nontemporal_load((global_u32x2 *)p);
  return make_uint2(v.x, v.y);
}

// ---- RMSNorm ------------------------------------------------------------------

// 1/rms of x[0..N) computed by the whole workgroup (every thread gets it).
template <int N, typename Src>
__device__ float block_inv_rms(const Src &x, float eps, float *red) {
  constexpr int N4 = N / 4;
  float s = 0.f;
  for (int c = threadIdx.x; c < N4; c += blockDim.x) {
    const float4 v = x.ld4(c);
    s = fmaf(v.x, v.x, s);
    s = fmaf(v.y, v.y, s);
    s = fmaf(v.z, v.z, s);
    s = fmaf(v.w, v.w, s);
  }
  s = wave_sum(s);
  if (lane_id() == 0) red[wave_id()] = s;
  __syncthreads();
  float t = 0.f;
  const int waves = blockDim.x / kWave;
  for (int w = 0; w < waves; ++w) t += red[w];
  __syncthreads();
  return rsqrtf(t / static_cast<float>(N) + eps);
}

// ---- row-pair GEMV slot layout --------------------------------------------------
// A wave computes the dot products of two weight rows with one K-vector.
// The two rows are viewed as one run of 2*K/4 float4 slots; lane l loads
// slots f = 64*j + l. The operand register xv[j] holds the x float4 that
// slot f multiplies, so the same registers serve every row pair.
template <int K>
struct PairSlots {
  static_assert(K % 4 == 0, "rows must be float4 aligned");
  static constexpr int K4 = K / 4;
  static constexpr int NJ = (2 * K4 + kWave - 1) / kWave;
};

// xv[j] = x[c] for the column c of slot j.
template <int K, typename Src>
__device__ __forceinline__ void load_pair_operand(const Src &x,
                                                  float4 (&xv)[PairSlots<K>::NJ]) {
  constexpr int K4 = PairSlots<K>::K4;
  const int lane = lane_id();
#pragma unroll
  for (int j = 0; j < PairSlots<K>::NJ; ++j) {
    const int f = j * kWave + lane;
    const int c = f < K4 ? f : f - K4;
    xv[j] = f < 2 * K4 ? x.ld4(c) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
}

// RMSNorm gains in the slot layout (gv[j] = gain[c]); loaded ahead of the
// activation so the normalised operand needs no global load.
template <int K>
__device__ __forceinline__ void load_pair_gain(const float *gain,
                                               float4 (&gv)[PairSlots<K>::NJ]) {
  constexpr int K4 = PairSlots<K>::K4;
  const global_f32x4 *g4 = (const global_f32x4 *)gain;
  const int lane = lane_id();
#pragma unroll
  for (int j = 0; j < PairSlots<K>::NJ; ++j) {
    const int f = j * kWave + lane;
    const int c = f < K4 ? f : f - K4;
    const gf32x4 v = f < 2 * K4 ? g4[c] : gf32x4{0.f, 0.f, 0.f, 0.f};
    gv[j] = make_float4(v.x, v.y, v.z, v.w);
  }
}

// RMSNorm folded past the GEMV: W . (x * inv * g) = inv * (W . (x * g)).
// Loads the operand as xv[j] = x[c] * gain[c] in the slot layout and
// returns the sum of squares of x, taken per lane over the slots of the
// first row (every element of x once) in slot order and then wave-reduced;
// every wave that loads the same x gets the same bits. The dots of the
// operand are scaled by norm_scale(ss, K, eps) afterwards, so no
// workgroup-wide reduction sits between the arrival of x and the dots.
template <int K, typename Src>
__device__ __forceinline__ float load_pair_operand_gain(const Src &x,
                                                        const float4 (&gv)[PairSlots<K>::NJ],
                                                        float4 (&xv)[PairSlots<K>::NJ]) {
  constexpr int K4 = PairSlots<K>::K4;
  load_pair_operand<K>(x, xv);
  const int lane = lane_id();
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < PairSlots<K>::NJ; ++j)
    if (j * kWave < K4 && j * kWave + lane < K4) ss = fma4(xv[j], xv[j], ss);
#pragma unroll
  for (int j = 0; j < PairSlots<K>::NJ; ++j) {
    xv[j].x *= gv[j].x;
    xv[j].y *= gv[j].y;
    xv[j].z *= gv[j].z;
    xv[j].w *= gv[j].w;
  }
  return wave_sum(ss);
}
__device__ __forceinline__ float norm_scale(float ss, int k, float eps) {
  return rsqrtf(ss / static_cast<float>(k) + eps);
}

// Weight slots of a row pair, loaded into registers (separable from the
// arithmetic so a caller can issue them early).
template <int K, typename W = float>
__device__ __forceinline__ void load_pair_weights(
    const W *a, const W *b, float4 (&w)[PairSlots<K>::NJ]) {
  constexpr int K4 = PairSlots<K>::K4;
  constexpr int NJ = PairSlots<K>::NJ;
  using S = typename WSlot<W>::type;
  const S *a4 = reinterpret_cast<const S *>(a);
  const S *b4 = reinterpret_cast<const S *>(b);
  const int lane = lane_id();
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int f = j * kWave + lane;
    if (j * kWave + kWave <= K4) {
      w[j] = ld_weight(a4 + f);
    } else if (j * kWave >= K4) {
      w[j] = f < 2 * K4 ? ld_weight(b4 + (f - K4)) : make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
      w[j] = ld_weight(f < K4 ? a4 + f : b4 + (f - K4));
    }
  }
}

// Per-lane partial dots of a row pair (the terms pair_dot wave-reduces).
template <int K>
__device__ __forceinline__ void pair_partial(const float4 (&w)[PairSlots<K>::NJ],
                                             const float4 (&xv)[PairSlots<K>::NJ],
                                             float &accA, float &accB) {
  constexpr int K4 = PairSlots<K>::K4;
  constexpr int NJ = PairSlots<K>::NJ;
  const int lane = lane_id();
  accA = 0.f;
  accB = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int f = j * kWave + lane;
    if (j * kWave + kWave <= K4) {
      accA = fma4(w[j], xv[j], accA);
    } else if (j * kWave >= K4) {
      // Lanes past the pair's 2 K4 float4s (the last slot's padding, which
      // an LDS-staged unit may hold any finite or non-finite words in) add
      // nothing.
      if (j * kWave + kWave <= 2 * K4) {
        accB = fma4(w[j], xv[j], accB);
      } else {
        accB = f < 2 * K4 ? fma4(w[j], xv[j], accB) : accB;
      }
    } else {
      const float d = fma4(w[j], xv[j], 0.f);
      if (f < K4) {
        accA += d;
      } else if (f < 2 * K4) {
        accB += d;
      }
    }
  }
}

// Wave-reduced dot products (every lane gets both sums).
template <int K>
__device__ __forceinline__ void pair_dot(const float4 (&w)[PairSlots<K>::NJ],
                                         const float4 (&xv)[PairSlots<K>::NJ],
                                         float &sa, float &sb) {
  float accA, accB;
  pair_partial<K>(w, xv, accA, accB);
  sa = wave_sum(accA);
  sb = wave_sum(accB);
}

template <int K, typename W = float>
__device__ __forceinline__ void dot_pair(const W *a, const W *b,
                                         const float4 (&xv)[PairSlots<K>::NJ],
                                         float &sa, float &sb) {
  float4 w[PairSlots<K>::NJ];
  load_pair_weights<K, W>(a, b, w);
  pair_dot<K>(w, xv, sa, sb);
}

// pair_dot with the operand read from LDS (x[0..K)) slot by slot instead of
// held in registers.
template <int K>
__device__ __forceinline__ void pair_dot_lds(const float4 (&w)[PairSlots<K>::NJ],
                                             const float *x, float &sa, float &sb) {
  constexpr int K4 = PairSlots<K>::K4;
  constexpr int NJ = PairSlots<K>::NJ;
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  const int lane = lane_id();
  float accA = 0.f, accB = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int f = j * kWave + lane;
    const int c = f < K4 ? f : f - K4;
    const float4 xv = f < 2 * K4 ? x4[c] : make_float4(0.f, 0.f, 0.f, 0.f);
    if (j * kWave + kWave <= K4) {
      accA = fma4(w[j], xv, accA);
    } else if (j * kWave >= K4) {
      accB = fma4(w[j], xv, accB);
    } else {
      const float d = fma4(w[j], xv, 0.f);
      if (f < K4) {
        accA += d;
      } else {
        accB += d;
      }
    }
  }
  sa = wave_sum(accA);
  sb = wave_sum(accB);
}

// Single-row dot for K a multiple of 256 floats: lane l loads float4 slots
// 64*j + l; xv[j] is the matching operand.
template <int K>
struct RowSlots {
  static_assert(K % (4 * kWave) == 0, "row must be a whole number of wave loads");
  static constexpr int NJ = K / (4 * kWave);
};

template <int K, typename Src>
__device__ __forceinline__ void load_row_operand(
    const Src &x, float4 (&xv)[RowSlots<K>::NJ]) {
  const int lane = lane_id();
#pragma unroll
  for (int j = 0; j < RowSlots<K>::NJ; ++j) xv[j] = x.ld4(j * kWave + lane);
}

template <int K, typename W = float>
__device__ __forceinline__ void load_row_weights(const W *a,
                                                 float4 (&w)[RowSlots<K>::NJ]) {
  const typename WSlot<W>::type *a4 = reinterpret_cast<const typename WSlot<W>::type *>(a);
  const int lane = lane_id();
#pragma unroll
  for (int j = 0; j < RowSlots<K>::NJ; ++j) w[j] = ld_weight(a4 + j * kWave + lane);
}

template <int K>
__device__ __forceinline__ float row_dot(const float4 (&w)[RowSlots<K>::NJ],
                                         const float4 (&xv)[RowSlots<K>::NJ]) {
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < RowSlots<K>::NJ; ++j) acc = fma4(w[j], xv[j], acc);
  return wave_sum(acc);
}

// row_dot with the operand read from LDS.
template <int K>
__device__ __forceinline__ float row_dot_lds(const float4 (&w)[RowSlots<K>::NJ],
                                             const float *x) {
  const float4 *x4 = reinterpret_cast<const float4 *>(x);
  const int lane = lane_id();
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < RowSlots<K>::NJ; ++j) {
    // Bounds the operand reads the scheduler hoists (register pressure).
    if (j % 4 == 0) __builtin_amdgcn_sched_barrier(0);
    acc = fma4(w[j], x4[j * kWave + lane], acc);
  }
  return wave_sum(acc);
}

template <int K>
__device__ __forceinline__ float dot_row(const float *a,
                                         const float4 (&xv)[RowSlots<K>::NJ]) {
  float4 w[RowSlots<K>::NJ];
  load_row_weights<K>(a, w);
  return row_dot<K>(w, xv);
}

// The down projection's row dot, in column slices. Slice s of a row's NJ
// float4 slots is [row_slice_begin(NJ, s), row_slice_begin(NJ, s + 1)); a
// slice's products are summed per lane in slot order from zero, each lane's
// kRowSlices slice sums combine as a fixed tree, and the lanes' results are
// reduced over the wave (wave_sum). The resident role kernel gives each
// slice to its own wave (each waits only for its slice of the activation)
// and combines the lanes' slice sums through LDS; the stream kernel walks
// the slices in one wave, so both produce the same bits.
constexpr int kRowSlices = 8;
__host__ __device__ constexpr int row_slice_begin(int nj, int s) { return nj * s / kRowSlices; }
__device__ __forceinline__ float combine_slices(const float (&p)[kRowSlices]) {
  return ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
}
template <int K, typename W = float>
__device__ __forceinline__ float dot_row_sliced(const W *a,
                                                const float4 (&xv)[RowSlots<K>::NJ]) {
  constexpr int NJ = RowSlots<K>::NJ;
  static_assert(kRowSlices == 8, "combine_slices");
  float4 w[NJ];
  load_row_weights<K, W>(a, w);
  float p[kRowSlices];
#pragma unroll
  for (int s = 0; s < kRowSlices; ++s) {
    float acc = 0.f;
#pragma unroll
    for (int j = row_slice_begin(NJ, s); j < row_slice_begin(NJ, s + 1); ++j) acc = fma4(w[j], xv[j], acc);
    p[s] = acc;
  }
  return wave_sum(combine_slices(p));
}

}  // namespace dev
}  // namespace qd
