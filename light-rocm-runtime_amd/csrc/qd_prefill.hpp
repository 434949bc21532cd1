// Host-side launchers of the prompt (prefill) kernels (qd_prefill.hip): the
// prompt's positions go through each layer together, as dense FP32 GEMMs on
// the matrix cores plus a causal GQA attention.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qd_device.hpp"

namespace qd {

// GEMM epilogues: C = A . W^T (+ bias) or C += A . W^T (residual); and the
// MLP's gate/up GEMM with SwiGLU fused (launch_gemm_swiglu).
enum GemmMode : int { kGemmStore = 0, kGemmBias = 1, kGemmAccumulate = 2, kGemmSwiGLU = 3 };

// Work on each finished row of a split-K GEMM, run by its reduction: the
// RMSNorm of the row into y (rows of 896, gain, eps), or RoPE of a packed
// QKV row at position pos0 + r with its K/V rows written to the cache.
enum RowEpilogueKind : int { kRowNone = 0, kRowNorm = 1, kRowRope = 2 };
struct RowEpilogue {
  int kind = kRowNone;
  const float *gain = nullptr;
  float eps = 0.f;
  float *y = nullptr;
  int pos0 = 0, nq = 0, nkv = 0;
  const float *rope_cos = nullptr, *rope_sin = nullptr;
  float *k_cache = nullptr, *v_cache = nullptr;
};

// C[m][n] (row stride ldc) for A [m][k] (stride lda) and W [n][k] (stride
// ldw), all FP32 row-major. m, n any size (edges masked); k a multiple of 32.
// split > 1 divides k over that many workgroup slices whose partials go to
// workspace (split * m * ldc floats) and are summed in a fixed order.
// sk_groups > 0 (stream-K) instead deals the tiles' 32-wide K slices to
// sk_groups workgroups in equal contiguous ranges; a tile's partials (one per
// workgroup meeting it, at most gemm_streamk_slots(m, n, k, sk_groups)) go
// to workspace (that many times m * ldc floats, within workspace_floats) and
// are summed in a fixed order. epi (partials, ldc == n) runs a row epilogue
// in that reduction.
hipError_t launch_gemm_nt(hipStream_t s, const float *A, int lda, const float *W, int ldw,
                          float *C, int ldc, int m, int n, int k, GemmMode mode,
                          const float *bias, int split = 1, float *workspace = nullptr,
                          const RowEpilogue *epi = nullptr, int sk_groups = 0, size_t workspace_floats = 0);

// Partial slots a stream-K launch of sk_groups workgroups needs (0 for an
// invalid shape).
int gemm_streamk_slots(int m, int n, int k, int sk_groups);

// out[r] = embed[tokens[r]] for r < rows (hidden floats each).
hipError_t launch_embed_rows(hipStream_t s, const float *embed, const uint32_t *tokens, int rows,
                             int hidden, float *out);

// y[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * gain for r < rows (hidden = 896).
hipError_t launch_rmsnorm_rows(hipStream_t s, const float *x, const float *gain, float eps,
                               int rows, float *y);

// Rotates the query and key heads of every row of qkv ([rows][q | k | v],
// rotate-half at position pos0 + r) in place and writes the rotated K and
// the V rows to the cache slots pos0 + r.
hipError_t launch_rope_kv_rows(hipStream_t s, float *qkv, int rows, int pos0, int nq, int nkv,
                               const float *rope_cos, const float *rope_sin, float *k_cache,
                               float *v_cache);

// Causal GQA attention of rows queries at positions pos0.. over cache
// positions 0..pos0 + r: out[r][h*64 + d] from the rotated queries in qkv.
hipError_t launch_attention_prefill(hipStream_t s, const float *qkv, int rows, int pos0, int nq,
                                    int nkv, const float *k_cache, const float *v_cache,
                                    float *out);

// act[r][i] = silu(A[r] . wg[i]) * (A[r] . wu[i]) for r < m, i < inter
// (act row stride ldc; wg and wu [inter][k] with row stride ldw; inter a
// multiple of 32, k of 32): the gate and up GEMMs and SwiGLU in one launch.
hipError_t launch_gemm_swiglu(hipStream_t s, const float *A, int lda, const float *wg, const float *wu,
                              int ldw, float *act, int ldc, int m, int inter, int k);

}  // namespace qd
