// Host engine behind the C ABI in include/qd/qwen_decode.h.
//
// Owns every device allocation: packed FP32 weights, the KV cache
// [slot][layer][capacity][kv_heads*64], RoPE tables, per-slot activations and
// decode state. All work is queued on one HIP stream of the engine's device;
// errors surface as qd_status at the call that observes them (launch errors
// immediately, device faults at the next synchronisation).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <memory>
#include <stdexcept>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

#include "qd/qwen_decode.h"
#include "qd_bundle.hpp"
#include "qd_device.hpp"
#include "qd_kernels.hpp"
#include "qd_batch.hpp"
#include "qd_prefill.hpp"
#include "qd_resident.hpp"
#include "qd_rng.hpp"

// Stream-K workgroups per CU of the prompt's QKV and down GEMMs (0:
// split-K). The O GEMM keeps split-K 2: its 224 workgroups already give
// every CU one equal share.
#ifndef QD_PREFILL_SK_QKV
#define QD_PREFILL_SK_QKV 1
#endif
#ifndef QD_PREFILL_SK_DOWN
#define QD_PREFILL_SK_DOWN 2
#endif

namespace {

constexpr uint32_t kAbiVersion = 4;
constexpr int kLmHeadParts = 1024;  // LM-head workgroups = top-1 partials

thread_local std::string g_error;

struct QdError : std::runtime_error {
  qd_status status;
  QdError(qd_status s, const std::string &m) : std::runtime_error(m), status(s) {}
};

[[noreturn]] void fail(qd_status s, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  throw QdError(s, buf);
}

qd_status hip_status(hipError_t e) {
  switch (e) {
    case hipErrorIllegalAddress:
    case hipErrorLaunchFailure:
    case hipErrorAssert:
    case hipErrorLaunchTimeOut:
      return QD_ERROR_DEVICE_FAULT;
    case hipErrorInvalidValue:
      return QD_ERROR_INVALID_ARGUMENT;
    default:
      return QD_ERROR_RUNTIME;
  }
}

void check(hipError_t e, const char *what) {
  if (e != hipSuccess) fail(hip_status(e), "%s: %s", what, hipGetErrorString(e));
}

int host_threads() {
  const char *env = std::getenv("OMP_NUM_THREADS");
  int n = env ? std::atoi(env) : 0;
  if (n <= 0) n = static_cast<int>(std::thread::hardware_concurrency());
  return std::max(1, std::min(n, 64));
}

// Fills out[0..n) with N(0, std) from the generator, elements [first, first+n)
// of the stream, on all host threads.
void fill_normal(float *out, size_t n, uint64_t first, uint64_t seed,
                 uint64_t stream, float stddev) {
  const qd::rng::Stream s(seed, stream);
  const int t = static_cast<int>(std::min<size_t>(host_threads(), n / 65536 + 1));
  std::vector<std::thread> pool;
  for (int k = 0; k < t; ++k) {
    pool.emplace_back([=, &s] {
      const size_t b = n * k / t, e = n * (k + 1) / t;
      for (size_t i = b; i < e; ++i)
        out[i] = static_cast<float>(static_cast<double>(stddev) * s.normal(first + i));
    });
  }
  for (auto &th : pool) th.join();
}

// FP32 -> BF16, rounded to nearest even; a NaN becomes the canonical quiet
// NaN 0x7FC0 (the BF16 half of 0x7FC00000), so no weight equals the
// resident kernel's empty-slot pattern after widening either.
uint16_t to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0) return 0x7FC0u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

float from_bf16(uint16_t h) {
  const uint32_t u = uint32_t(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// FP32 -> IEEE FP16, rounded to nearest even (values beyond the largest
// half round to infinity); a NaN becomes the canonical quiet NaN 0x7E00,
// which widens to 0x7FC00000.
uint16_t to_f16(float f) {
  if (f != f) return 0x7E00u;
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

float from_f16(uint16_t h) { return static_cast<float>(__builtin_bit_cast(_Float16, h)); }

}  // namespace

struct qd_engine {
  qd_config cfg{};
  size_t H = 0, I = 0, NQ = 0, NKV = 0, QD = 0, KVD = 0, QKV = 0, V = 0, L = 0,
         CAP = 0, B = 0;
  hipStream_t stream = nullptr;
  hipEvent_t ev_begin = nullptr, ev_end = nullptr;
  std::vector<void *> allocs;
  uint64_t device_bytes = 0;

  float *weights = nullptr;  // arena of all layer weights
  size_t weights_floats = 0;
  std::vector<qd::LayerPtrs> layers;
  float *embed = nullptr, *lm_head = nullptr, *final_norm = nullptr;
  float *k_cache = nullptr, *v_cache = nullptr;
  float *rope_cos = nullptr, *rope_sin = nullptr;
  float *hidden = nullptr, *q = nullptr, *attn = nullptr, *act = nullptr,
        *logits = nullptr;
  float *part = nullptr;  // split-KV partials [16][heads][66]
  float *part_val = nullptr;
  uint32_t *part_idx = nullptr;
  uint32_t *tokens_dev = nullptr;  // [capacity]
  qd::SeqState *states = nullptr;  // [max_batch]
  float *history = nullptr;        // generate-mode logits [capacity][vocab]
  size_t history_rows = 0;

  // Resident megakernel state (qd_roles.hip): one workgroup per CU.
  qd::LayerPtrs *layer_ptrs_dev = nullptr;  // [layers]
  uint64_t *top_pairs = nullptr;            // argmax (value, tag) partials [4 * roles_grid]
  float *roles_slots = nullptr;             // hand-off slots
  size_t roles_slot_bytes = 0;
  uint32_t epoch = 0;                       // last launch epoch (1..4095)
  uint32_t *resident_error = nullptr;       // [1 + kXcds]
  uint32_t spin_limit = qd::kResidentSpinLimit;
  int roles_grid = 0;                       // 0: resident path unavailable
  // Attention chunk geometry of both paths, attn_chunks(length, attn_parts, kAttnGrain):
  // the resident plan's attention CUs per KV group at the engine's capacity
  // (fixed at create, so the stream kernels split a context as the resident
  // kernel does whether or not it runs), else kAttnMaxChunks.
  int attn_parts = qd::kAttnMaxChunks;
  std::string resident_off_reason;
  // Prompt workspace (allocated on the first prefill): rows of the hidden
  // states, RMSNorm output, packed QKV, attention output and SwiGLU
  // activation, plus the chunk's token ids.
  static constexpr size_t kPrefillRows = 512;
  float *pf_h = nullptr, *pf_xn = nullptr, *pf_qkv = nullptr, *pf_attn = nullptr,
        *pf_act = nullptr, *pf_split = nullptr;
  // Split-K factors of the narrow GEMMs (QKV, O, down) so they fill the CUs,
  // used when stream-K is off (sk_target 0).
  static constexpr int kSplitQkv = 2, kSplitO = 2, kSplitDown = 4;
  // Stream-K for the QKV and down GEMMs: up to per_cu workgroups per CU
  // (QD_PREFILL_SK_QKV / QD_PREFILL_SK_DOWN), each taking at least
  // kSkMinSlices K slices of 32, so every CU gets an equal share of the
  // (tile, slice) work; pf_split_floats is the partial workspace that any
  // prompt chunk of up to kPrefillRows rows needs.
  static constexpr int kSkMinSlices = 8;
  int cu_count = 0;
  size_t pf_split_floats = 0;
  int sk_groups(int m, int n, int k, int per_cu) const {
    if (per_cu <= 0 || cu_count <= 0) return 0;
    const long long total = static_cast<long long>((m + 63) / 64) * ((n + 63) / 64) * (k / 32);
    return static_cast<int>(
        std::min<long long>(static_cast<long long>(per_cu) * cu_count, std::max<long long>(1, total / kSkMinSlices)));
  }
  uint32_t *pf_tokens = nullptr;
  // Batched-step workspace (allocated on the first batched step): rows of
  // up to kBatchRows sequences, attention and split-K partials, arrival
  // counters, the LM-head top-1 partials and each row's greedy result.
  float *bt_h = nullptr, *bt_q = nullptr, *bt_attn = nullptr, *bt_act = nullptr,
        *bt_part = nullptr, *bt_split = nullptr, *bt_val = nullptr, *bt_top = nullptr;
  uint32_t *bt_idx = nullptr, *bt_counters = nullptr, *bt_token = nullptr;
  uint32_t *h_bt_out = nullptr;  // pinned [max_batch] tokens then [max_batch] top logits
  // The library's static batch workspace on this engine's device
  // (qd_step_batch_noalloc), looked up at creation; null if the lookup failed.
  void *batch_scratch = nullptr;
  std::string batch_scratch_error;

  qd::SeqState *h_states = nullptr;  // pinned [max_batch]
  uint32_t *h_tokens = nullptr;      // pinned [capacity]
  uint32_t *h_error = nullptr;       // pinned [1]: a resident launch's error word
  std::vector<uint32_t> positions;   // host mirror of each slot's position
  bool loaded = false;
  qd_timing timing{};
  // Per slot: qd_step's launch sequence captured as a HIP graph (nullptr
  // until the slot's first qd_step_graph).
  std::vector<hipGraphExec_t> step_graphs;

  // Teardown cannot report errors; a device fault was already reported by
  // the call that observed it.
  ~qd_engine() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (hipGraphExec_t g : step_graphs)
      if (g) (void)hipGraphExecDestroy(g);
    for (void *p : allocs) (void)hipFree(p);
    if (h_states) (void)hipHostFree(h_states);
    if (h_tokens) (void)hipHostFree(h_tokens);
    if (h_error) (void)hipHostFree(h_error);
    if (h_bt_out) (void)hipHostFree(h_bt_out);
    if (ev_begin) (void)hipEventDestroy(ev_begin);
    if (ev_end) (void)hipEventDestroy(ev_end);
    if (stream) (void)hipStreamDestroy(stream);
  }

  template <typename T>
  T *alloc(size_t count) {
    void *p = nullptr;
    const size_t bytes = std::max<size_t>(count * sizeof(T), 256);
    check(hipMalloc(&p, bytes), "hipMalloc");
    allocs.push_back(p);
    device_bytes += bytes;
    return static_cast<T *>(p);
  }

  float *kv_slice(float *base, size_t seq, size_t layer) const {
    return base + ((seq * L + layer) * CAP) * KVD;
  }

  void set_device() const { check(hipSetDevice(cfg.device), "hipSetDevice"); }

  void upload(float *dst, const float *src, size_t n) {
    check(hipMemcpyAsync(dst, src, n * sizeof(float), hipMemcpyHostToDevice, stream),
          "hipMemcpyAsync H2D");
  }

  // The decoder matrices (wqkv, wo, wg, wu, wd) hold BF16 or FP16 on an
  // engine created with QD_DTYPE_BF16 / QD_DTYPE_F16 decoder weights, else
  // FP32. LayerPtrs keeps their addresses as float pointers either way;
  // element offsets into them go through mat_at.
  int wdtype = qd::kWeightsF32;
  bool narrow() const { return wdtype != qd::kWeightsF32; }
  size_t mat_elem() const { return narrow() ? 2 : 4; }
  uint16_t to_narrow(float f) const { return wdtype == qd::kWeightsF16 ? to_f16(f) : to_bf16(f); }
  float from_narrow(uint16_t h) const { return wdtype == qd::kWeightsF16 ? from_f16(h) : from_bf16(h); }
  const char *dtype_name() const {
    return wdtype == qd::kWeightsF16 ? "FP16" : wdtype == qd::kWeightsBf16 ? "BF16" : "FP32";
  }
  char *mat_at(const float *base, size_t off) const {
    return reinterpret_cast<char *>(const_cast<float *>(base)) + off * mat_elem();
  }
  // n FP32 values into a decoder matrix from element `off` (rounded to BF16
  // or FP16 on such an engine; that copy completes before the call returns).
  void upload_mat(const float *base, size_t off, const float *src, size_t n) {
    if (!narrow()) {
      upload(reinterpret_cast<float *>(mat_at(base, off)), src, n);
      return;
    }
    std::vector<uint16_t> h(n);
    for (size_t i = 0; i < n; ++i) h[i] = to_narrow(src[i]);
    check(hipMemcpyAsync(mat_at(base, off), h.data(), n * 2, hipMemcpyHostToDevice, stream), "H2D");
    check(hipStreamSynchronize(stream), "hipStreamSynchronize");
  }

  void build_rope_tables(float theta) {
    // Same FP32 recipe as the Hugging Face rotary embedding: inv_freq =
    // 1 / theta^(2i/d), angle = p * inv_freq, both rounded to FP32.
    std::vector<float> c(CAP * qd::kRotary), s(CAP * qd::kRotary);
    for (int i = 0; i < qd::kRotary; ++i) {
      const float exponent = static_cast<float>(2 * i) / static_cast<float>(qd::kHeadDim);
      const float inv_freq = 1.0f / std::pow(theta, exponent);
      for (size_t p = 0; p < CAP; ++p) {
        const float angle = static_cast<float>(p) * inv_freq;
        c[p * qd::kRotary + i] = static_cast<float>(std::cos(static_cast<double>(angle)));
        s[p * qd::kRotary + i] = static_cast<float>(std::sin(static_cast<double>(angle)));
      }
    }
    upload(rope_cos, c.data(), c.size());
    upload(rope_sin, s.data(), s.size());
    check(hipStreamSynchronize(stream), "rope upload");
    cfg.rope_theta = theta;
  }

  void check_seq(uint32_t seq) const {
    if (seq >= B) fail(QD_ERROR_INVALID_ARGUMENT, "sequence slot %u out of range (max_batch %zu)", seq, B);
  }
  void check_loaded() const {
    if (!loaded) fail(QD_ERROR_NOT_INITIALIZED, "weights are not loaded");
  }

  // Writes the slot's device state from the host mirror.
  void push_state(uint32_t seq, uint32_t token, uint32_t mode, uint32_t eos,
                  uint32_t max_tokens) {
    qd::SeqState &h = h_states[seq];
    std::memset(&h, 0, sizeof(h));
    h.position = positions[seq];
    h.token = token;
    h.eos = eos;
    h.max_tokens = max_tokens;
    h.mode = mode;
    check(hipMemcpyAsync(states + seq, &h, sizeof(h), hipMemcpyHostToDevice, stream),
          "state upload");
  }

  qd::LayerLaunch layer_args(uint32_t seq, size_t layer) {
    qd::LayerLaunch a{};
    a.w = layers[layer];
    a.rope_cos = rope_cos;
    a.rope_sin = rope_sin;
    a.st = states + seq;
    a.hidden = hidden + seq * H;
    a.q = q + seq * QD;
    a.attn = attn + seq * QD;
    a.act = act + seq * I;
    a.k_cache = kv_slice(k_cache, seq, layer);
    a.v_cache = kv_slice(v_cache, seq, layer);
    a.part = part;
    a.attn_parts = attn_parts;
    a.weights_dtype = wdtype;
    a.capacity = static_cast<int>(CAP);
    a.nq = static_cast<int>(NQ);
    a.nkv = static_cast<int>(NKV);
    a.eps = cfg.rms_eps;
    return a;
  }

  qd::TailLaunch tail_args(uint32_t seq, float *out_logits, int hist,
                           uint32_t *out_tokens) {
    qd::TailLaunch t{};
    t.hidden = hidden + seq * H;
    t.final_norm = final_norm;
    t.head = lm_head;
    t.st = states + seq;
    t.logits = out_logits;
    t.history = hist;
    t.vocab = static_cast<int>(V);
    t.eps = cfg.rms_eps;
    t.part_val = part_val;
    t.part_idx = part_idx;
    t.parts = kLmHeadParts;
    t.out_tokens = out_tokens;
    return t;
  }

  // Embedding + every layer + LM head + argmax for one slot (state already
  // on the device).
  void enqueue_step(uint32_t seq, float *out_logits, int hist,
                    uint32_t *out_tokens, qd::Marker *m = nullptr) {
    check(qd::launch_embed(stream, embed, states + seq, hidden + seq * H,
                           static_cast<int>(H), static_cast<int>(V), m),
          "embed launch");
    for (size_t l = 0; l < L; ++l)
      check(qd::launch_layer(stream, layer_args(seq, l), m), "layer launch");
    check(qd::launch_tail(stream, tail_args(seq, out_logits, hist, out_tokens), m),
          "tail launch");
  }
  // The slot's qd_step launch sequence as an instantiated HIP graph,
  // captured on first use. Every kernel of it reads the position and the
  // token from the slot's device state and takes only fixed buffers and a
  // fixed grid as arguments (the attention split is the engine's, fixed at
  // creation), so one capture serves every later step of the slot. The
  // graph holds kernel nodes only (no memset or copy nodes).
  hipGraphExec_t step_graph(uint32_t seq) {
    if (step_graphs.empty()) step_graphs.assign(B, nullptr);
    if (step_graphs[seq]) return step_graphs[seq];
    check(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    hipGraph_t graph = nullptr;
    try {
      enqueue_step(seq, logits + seq * V, 0, nullptr);
    } catch (...) {
      (void)hipStreamEndCapture(stream, &graph);
      if (graph) (void)hipGraphDestroy(graph);
      throw;
    }
    check(hipStreamEndCapture(stream, &graph), "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    const hipError_t err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    check(err, "hipGraphInstantiate");
    step_graphs[seq] = exec;
    return exec;
  }

  // Algorithmic bytes of one launch of `kernel` when the step attends over
  // `length` positions: weights, KV rows and activations each moved once.
  double kernel_bytes(int kernel, double length) const {
    const double f = 4.0;
    const double mf = static_cast<double>(mat_elem());  // bytes per decoder-matrix element
    const double chunks = qd::attn_chunks(static_cast<int>(length), attn_parts, qd::kAttnGrain);
    switch (kernel) {
      case qd::kKEmbed: return 2 * H * f;
      case qd::kKQkvRope:
        return QKV * H * mf + (QKV + 2 * H + 2 * qd::kRotary + QD + 2 * KVD) * f;
      case qd::kKAttnPartial:
        return (2 * length * KVD + QD + chunks * NQ * (qd::kHeadDim + 2)) * f;
      case qd::kKAttnCombine: return (chunks * NQ * (qd::kHeadDim + 2) + QD) * f;
      case qd::kKOproj: return H * QD * mf + (QD + 2 * H) * f;
      case qd::kKGateUp: return 2 * I * H * mf + (2 * H + I) * f;
      case qd::kKDown: return H * I * mf + (I + 2 * H) * f;
      case qd::kKLmHead: return (V * H + 2 * H + V + 2 * 1024) * f;
      case qd::kKArgmax: return 2 * 1024 * f;
    }
    return 0;
  }

  // Arguments of one batched launch over rows sequences: slot ids, tokens
  // and (host-tracked) positions of batch rows first .. first + rows - 1.
  qd::BatchLaunch batch_args(const uint32_t *slots, const uint32_t *tokens, int rows) {
    if (!bt_h) {
      const size_t r = qd::kBatchRows;
      bt_h = alloc<float>(r * H);
      bt_q = alloc<float>(r * QD);
      bt_attn = alloc<float>(r * QD);
      bt_act = alloc<float>(r * I);
      bt_part = alloc<float>(r * NQ * qd::kAttnMaxChunks * qd::kPartStride);
      bt_split = alloc<float>(qd::kBatchSplitFloats);
      bt_counters = alloc<uint32_t>(qd::kBatchCounters);
      bt_val = alloc<float>(r * qd::kBatchLmParts);
      bt_idx = alloc<uint32_t>(r * qd::kBatchLmParts);
      bt_token = alloc<uint32_t>(B);
      bt_top = alloc<float>(B);
      check(hipMemsetAsync(bt_counters, 0, qd::kBatchCounters * sizeof(uint32_t), stream), "memset");
      check(hipHostMalloc(reinterpret_cast<void **>(&h_bt_out), 2 * B * sizeof(uint32_t),
                          hipHostMallocDefault),
            "hipHostMalloc");
    }
    qd::BatchLaunch b{};
    b.rows = rows;
    for (int i = 0; i < rows; ++i) {
      b.slot[i] = slots[i];
      b.pos[i] = positions[slots[i]];
      b.token[i] = tokens[i];
    }
    b.states = states;
    b.hidden = bt_h;
    b.q = bt_q;
    b.attn = bt_attn;
    b.act = bt_act;
    b.part = bt_part;
    b.split = bt_split;
    b.counters = bt_counters;
    b.k_cache = k_cache;
    b.v_cache = v_cache;
    b.rope_cos = rope_cos;
    b.rope_sin = rope_sin;
    b.layers = static_cast<int>(L);
    b.capacity = static_cast<int>(CAP);
    b.nq = static_cast<int>(NQ);
    b.nkv = static_cast<int>(NKV);
    b.eps = cfg.rms_eps;
    return b;
  }

  // Tail arguments of the group whose first batch row is `first`: each
  // row's logits go to its slot's row of the logits buffer (where
  // qd_read_logits finds them), greedy results to bt_token/bt_top.
  qd::BatchTail batch_tail(size_t first) const {
    qd::BatchTail t{};
    t.final_norm = final_norm;
    t.head = lm_head;
    t.logits = logits;
    t.part_val = bt_val;
    t.part_idx = bt_idx;
    t.out_token = bt_token + first;
    t.out_top = bt_top + first;
    t.vocab = static_cast<int>(V);
    return t;
  }

  // Embedding + every layer + LM head + argmax of one batch group (states
  // and slot list already on the device).
  void enqueue_batch(const qd::BatchLaunch &b, size_t first, qd::Marker *m = nullptr) {
    check(qd::launch_batch_embed(stream, b, embed, static_cast<int>(V), m), "batch embed launch");
    for (size_t l = 0; l < L; ++l)
      check(qd::launch_batch_layer(stream, b, layers[l], static_cast<int>(l), m),
            "batch layer launch");
    check(qd::launch_batch_tail(stream, b, batch_tail(first), m), "batch tail launch");
  }

  // Floating-point operations of one launch of `kernel` (multiply-add = 2).
  double kernel_flops(int kernel, double length) const {
    switch (kernel) {
      case qd::kKQkvRope: return 2.0 * QKV * H;
      case qd::kKAttnPartial: return 4.0 * NQ * qd::kHeadDim * length;
      case qd::kKOproj: return 2.0 * H * QD;
      case qd::kKGateUp: return 4.0 * I * H;
      case qd::kKDown: return 2.0 * H * I;
      case qd::kKLmHead: return 2.0 * V * H;
    }
    return 0;
  }

  // Algorithmic bytes and flops of one batched-step launch over `rows`
  // sequences attending over `attended` positions in total.
  std::pair<double, double> batch_cost(int kernel, double rows, double attended) const {
    const double f = 4.0;
    switch (kernel) {
      case qd::kBEmbed: return {2 * rows * H * f, 0};
      case qd::kBQkvRope: return {(QKV * H + QKV + H + rows * (H + QD + 2 * KVD)) * f, 2 * rows * QKV * H};
      case qd::kBAttn:
        return {(2 * attended * KVD + 2 * rows * QD) * f, 4 * NQ * qd::kHeadDim * attended};
      case qd::kBOproj: return {(H * QD + rows * (QD + 2 * H)) * f, 2 * rows * H * QD};
      case qd::kBGateUp: return {(2 * I * H + H + rows * (H + I)) * f, 4 * rows * I * H};
      case qd::kBDown: return {(H * I + rows * (I + 2 * H)) * f, 2 * rows * H * I};
      case qd::kBLmHead: return {(V * H + H + rows * (H + V)) * f, 2 * rows * V * H};
      case qd::kBArgmax: return {rows * 2 * qd::kBatchLmParts * f, 0};
    }
    return {0, 0};
  }

  // Kernels of the prompt path, for per-kernel event timing.
  enum PrefillKernel : int {
    kPEmbed = 0, kPNorm, kPGemmQkv, kPAttn, kPGemmO, kPGemmGateUp, kPGemmDown,
    kPTail, kPrefillKernels
  };
  static const char *prefill_kernel_name(int id) {
    static const char *const names[kPrefillKernels] = {
        "embed_rows_kernel",    "rmsnorm_rows_kernel",      "gemm_nt_kernel:qkv+rope",
        "attention_prefill_kernel", "gemm_nt_kernel:o+norm",
        "gemm_nt_kernel:gateup+swiglu", "gemm_nt_kernel:down+norm",
        "lmhead_kernel+argmax"};
    return id >= 0 && id < kPrefillKernels ? names[id] : "unknown";
  }

  // Algorithmic bytes and flops of one prompt-path launch for a chunk of n
  // rows at positions pos0..: each operand and result moved once; GEMMs
  // that accumulate read and write C.
  std::pair<double, double> prefill_cost(int kernel, double n, double pos0) const {
    const double f = 4.0;
    switch (kernel) {
      case kPEmbed: return {2 * n * H * f, 0};
      case kPNorm: return {(2 * n * H + H) * f, 0};
      case kPGemmQkv: return {(QKV * H + QKV + n * (H + QKV + 2 * QD + 4 * KVD)) * f, 2 * n * QKV * H};
      case kPAttn:
        return {(2 * (pos0 + n) * KVD + 2 * n * QD) * f,
                4 * NQ * qd::kHeadDim * (n * pos0 + n * (n + 1) / 2)};
      case kPGemmO: return {(H * QD + H + n * (QD + 3 * H)) * f, 2 * n * H * QD};
      case kPGemmGateUp: return {(2 * I * H + n * (H + I)) * f, 4 * n * I * H};
      case kPGemmDown: return {(H * I + H + n * (I + 3 * H)) * f, 2 * n * H * I};
      case kPTail: return {(V * H + H + V) * f, 2 * V * H};
    }
    return {0, 0};
  }


  // One chunk of a prompt (n <= kPrefillRows tokens at positions
  // pos0 .. pos0 + n - 1 of slot seq) through every layer with the prompt
  // kernels; leaves the final hidden rows in pf_h.
  void prefill_chunk(uint32_t seq, const uint32_t *tokens, int n, int pos0, qd::Marker *m = nullptr) {
    if (!pf_h) {
      pf_h = alloc<float>(kPrefillRows * H);
      pf_xn = alloc<float>(kPrefillRows * H);
      pf_qkv = alloc<float>(kPrefillRows * QKV);
      pf_attn = alloc<float>(kPrefillRows * QD);
      pf_act = alloc<float>(kPrefillRows * I);
      pf_tokens = alloc<uint32_t>(kPrefillRows);
      pf_split_floats = kPrefillRows * std::max({kSplitQkv * QKV, kSplitO * H, kSplitDown * H});
      const int shapes[2][3] = {{int(QKV), int(H), QD_PREFILL_SK_QKV}, {int(H), int(I), QD_PREFILL_SK_DOWN}};
      for (int rows = 1; rows <= int(kPrefillRows); ++rows)
        for (const auto &sh : shapes) {
          const int g = sk_groups(rows, sh[0], sh[1], sh[2]);
          if (g > 0)
            pf_split_floats = std::max(pf_split_floats, size_t(qd::gemm_streamk_slots(rows, sh[0], sh[1], g)) *
                                                            size_t(rows) * size_t(sh[0]));
        }
      pf_split = alloc<float>(pf_split_floats);
    }
    check(hipMemcpyAsync(pf_tokens, tokens, size_t(n) * 4, hipMemcpyHostToDevice, stream), "H2D");
    const int h = int(H), in = int(I), qkv = int(QKV), qd = int(QD);
    const int nq = int(NQ), nkv = int(NKV);
    auto span = [&](int id, const char *what, auto &&launch) {
      if (m) m->before(id);
      check(launch(), what);
      if (m) m->after(id);
    };
    span(kPEmbed, "embed rows",
         [&] { return qd::launch_embed_rows(stream, embed, pf_tokens, n, h, pf_h); });
    for (size_t l = 0; l < L; ++l) {
      const qd::LayerPtrs &w = layers[l];
      float *kc = kv_slice(k_cache, seq, l), *vc = kv_slice(v_cache, seq, l);
      // The attention norm of layer 0 runs on its own; every other norm and
      // the RoPE run in the reduction of the split-K GEMM before them.
      if (l == 0)
        span(kPNorm, "norm",
             [&] { return qd::launch_rmsnorm_rows(stream, pf_h, w.attn_norm, cfg.rms_eps, n, pf_xn); });
      span(kPGemmQkv, "qkv gemm + rope", [&] {
        qd::RowEpilogue rope;
        rope.kind = qd::kRowRope;
        rope.pos0 = pos0;
        rope.nq = nq;
        rope.nkv = nkv;
        rope.rope_cos = rope_cos;
        rope.rope_sin = rope_sin;
        rope.k_cache = kc;
        rope.v_cache = vc;
        return qd::launch_gemm_nt(stream, pf_xn, h, w.wqkv, h, pf_qkv, qkv, n, qkv, h, qd::kGemmBias,
                                  w.bqkv, kSplitQkv, pf_split, &rope, sk_groups(n, qkv, h, QD_PREFILL_SK_QKV),
                                  pf_split_floats);
      });
      span(kPAttn, "attention", [&] {
        return qd::launch_attention_prefill(stream, pf_qkv, n, pos0, nq, nkv, kc, vc, pf_attn);
      });
      span(kPGemmO, "o gemm + norm", [&] {
        qd::RowEpilogue norm;
        norm.kind = qd::kRowNorm;
        norm.gain = w.mlp_norm;
        norm.eps = cfg.rms_eps;
        norm.y = pf_xn;
        return qd::launch_gemm_nt(stream, pf_attn, qd, w.wo, qd, pf_h, h, n, h, qd,
                                  qd::kGemmAccumulate, nullptr, kSplitO, pf_split, &norm);
      });
      span(kPGemmGateUp, "gate/up gemm + swiglu", [&] {
        return qd::launch_gemm_swiglu(stream, pf_xn, h, w.wg, w.wu, h, pf_act, in, n, in, h);
      });
      span(kPGemmDown, "down gemm", [&] {
        qd::RowEpilogue norm;
        if (l + 1 < L) {
          norm.kind = qd::kRowNorm;
          norm.gain = layers[l + 1].attn_norm;
          norm.eps = cfg.rms_eps;
          norm.y = pf_xn;
        }
        return qd::launch_gemm_nt(stream, pf_act, in, w.wd, in, pf_h, h, n, h, in,
                                  qd::kGemmAccumulate, nullptr, kSplitDown, pf_split,
                                  l + 1 < L ? &norm : nullptr, sk_groups(n, h, in, QD_PREFILL_SK_DOWN),
                                  pf_split_floats);
      });
    }
  }

  // Role plan of a resident launch whose longest context is `reach`; false
  // when the resident path is off or the plan does not fit the grid.
  bool resident_plan(uint32_t reach, qd::RolePlan *plan) const {
    return roles_grid > 0 &&
           qd::plan_roles(roles_grid, int(H), int(I), int(NQ), int(NKV), int(reach), plan);
  }

  // Launches the resident megakernel (stream ordered; no synchronisation)
  // with a plan from resident_plan. Each launch gets a fresh epoch so no
  // argmax tag of an earlier launch matches; when the epoch counter wraps
  // the tag arena is cleared first. Returns the launch status; the caller
  // decides how to handle a refused cooperative launch.
  hipError_t launch_resident(const qd::RolePlan &plan, uint32_t seq, uint32_t first_token,
                             uint32_t max_tokens, uint32_t eos, float *hist, int use_hist,
                             uint64_t *stage_ticks, uint64_t *trace = nullptr,
                             uint32_t trace_token = 0) {
    epoch = epoch % 4095u + 1u;
    qd::ResidentArgs ra{};
    ra.layer_ptrs = layer_ptrs_dev;
    ra.embed = embed;
    ra.head = lm_head;
    ra.final_norm = final_norm;
    ra.rope_cos = rope_cos;
    ra.rope_sin = rope_sin;
    ra.k_cache = kv_slice(k_cache, seq, 0);
    ra.v_cache = kv_slice(v_cache, seq, 0);
    ra.top = top_pairs;
    ra.slots = roles_slots;
    ra.logits = hist;
    ra.out_tokens = tokens_dev;
    ra.st = states + seq;
    ra.error = resident_error;
    ra.stage_ticks = stage_ticks;
    ra.trace = trace;
    ra.trace_token = trace_token;
    ra.history = use_hist;
    ra.capacity = static_cast<int>(CAP);
    ra.vocab = static_cast<int>(V);
    ra.layers = static_cast<int>(L);
    ra.nq = static_cast<int>(NQ);
    ra.nkv = static_cast<int>(NKV);
    ra.eps = cfg.rms_eps;
    ra.first_token = first_token;
    ra.start_position = positions[seq];
    ra.max_tokens = max_tokens;
    ra.eos = eos;
    ra.epoch = epoch << qd::kTagSeqBits;
    ra.spin_limit = spin_limit;
    for (int r = 0; r < qd::kRoleCount; ++r) ra.role_end[r] = plan.end[r];
    for (int r = 0; r < 3; ++r) ra.group_cus[r] = plan.group_cus[r];
    ra.xcd_place = plan.xcd_place;
    ra.attn_parts = attn_parts;
    // The first token attends to the fewest positions and the last to the
    // most; a chunk never shrinks as the context grows.
    {
      const int first = static_cast<int>(positions[seq]) + 1;
      const int last = static_cast<int>(std::min<uint64_t>(uint64_t(positions[seq]) + max_tokens, CAP));
      ra.attn_mode = qd::attn_chunk_len(first, attn_parts, qd::kAttnGrain) > qd::kAttnPass ? 1
                     : qd::attn_chunk_len(last, attn_parts, qd::kAttnGrain) <= qd::kAttnPass ? 2
                                                                                             : 0;
    }
    ra.weights_dtype = wdtype;
    // Error word and tickets zero, token 0's hand-off slots empty (all bits
    // set), the tag arena zero when the epoch counter wrapped.
    check(qd::launch_roles_prepare(stream, resident_error, roles_slots, roles_slot_bytes / (8 * L),
                                   int(L), epoch == 1u ? top_pairs : nullptr, 4 * roles_grid),
          "resident prepare");
    return qd::launch_roles(stream, ra, roles_grid);
  }

  // After a resident launch has completed (stream synchronised): turns the
  // kernel's error word into a status.
  void check_resident_error() {
    enqueue_resident_error();
    sync();
    resident_status(*h_error);
  }
  // The error word's copy to h_error, stream ordered after the launch.
  void enqueue_resident_error() {
    check(hipMemcpyAsync(h_error, resident_error, 4, hipMemcpyDeviceToHost, stream), "D2H");
  }
  // Fails with the status that a nonzero error word names.
  void resident_status(uint32_t err) {
    if (err & qd::kResidentPlanOverfill)
      fail(QD_ERROR_RUNTIME,
           "resident role plan gives a CU more weight units than it holds on chip (error word 0x%x)",
           err);
    if (err & qd::kResidentPlacement)
      fail(QD_ERROR_RUNTIME,
           "resident kernel: an XCD received more than grid / %d workgroups, which the role "
           "placement assumes (error word 0x%x)",
           qd::kXcds, err);
    if (err & qd::kResidentWaitGaveUp)
      fail(QD_ERROR_DEVICE_FAULT,
           "resident kernel: a hand-off wait gave up after %u polls without its producer "
           "(error word 0x%x)",
           spin_limit, err);
    if (err) fail(QD_ERROR_DEVICE_FAULT, "resident kernel error word 0x%x", err);
  }

  // A cooperative launch can be refused while another process holds the
  // device's cooperative-launch resources. The engine then generates with
  // the stream-ordered kernels (same results) from here on, and says why.
  bool resident_refused(hipError_t err) {
    if (err != hipErrorIllegalState && err != hipErrorCooperativeLaunchTooLarge) return false;
    (void)hipGetLastError();
    roles_grid = 0;
    resident_off_reason = std::string("cooperative launch refused: ") + hipGetErrorString(err);
    return true;
  }

  // Resident launches name (token, stage) pairs in kTagSeqBits bits.
  bool resident_fits(uint32_t max_tokens) const {
    return uint64_t(max_tokens) * (5 * L + 1) + 1 < (uint64_t(1) << qd::kTagSeqBits);
  }

  void sync() { check(hipStreamSynchronize(stream), "hipStreamSynchronize"); }
};

namespace {

qd_status guard(const std::function<void()> &fn) {
  try {
    fn();
    return QD_SUCCESS;
  } catch (const QdError &e) {
    g_error = e.what();
    return e.status;
  } catch (const std::bad_alloc &) {
    g_error = "host allocation failed";
    return QD_ERROR_RUNTIME;
  } catch (const std::invalid_argument &e) {
    g_error = e.what();
    return QD_ERROR_INVALID_ARGUMENT;
  } catch (const std::exception &e) {
    g_error = e.what();
    return QD_ERROR_RUNTIME;
  }
}

void layer_shape_matches(const qd_engine &e, const qd::bundle::LayerWeights &w) {
  const auto &s = w.shape;
  if (s.hidden != e.H || s.heads != e.NQ || s.kv_heads != e.NKV ||
      s.head_dim != qd::kHeadDim || s.intermediate != e.I)
    fail(QD_ERROR_INVALID_ARGUMENT,
         "bundle decoder shape (hidden %u heads %u kv_heads %u head_dim %u "
         "intermediate %u) does not match the engine",
         s.hidden, s.heads, s.kv_heads, s.head_dim, s.intermediate);
}

}  // namespace

namespace qd {
qd_status guard_call(void (*fn)(void *), void *ctx) {
  return guard([&] { fn(ctx); });
}
}  // namespace qd

extern "C" {

const char *qd_status_string(qd_status s) {
  switch (s) {
    case QD_SUCCESS: return "success";
    case QD_ERROR_INVALID_ARGUMENT: return "invalid argument";
    case QD_ERROR_NOT_INITIALIZED: return "not initialized";
    case QD_ERROR_ALREADY_INITIALIZED: return "already initialized";
    case QD_ERROR_NOT_SUPPORTED: return "not supported";
    case QD_ERROR_RUNTIME: return "runtime error";
    case QD_ERROR_DEVICE_FAULT: return "device fault";
  }
  return "unknown status";
}

const char *qd_last_error(void) { return g_error.c_str(); }

uint32_t qd_abi_version(void) { return kAbiVersion; }

qd_status qd_device_count(uint32_t *count) {
  return guard([&] {
    if (!count) fail(QD_ERROR_INVALID_ARGUMENT, "count is null");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = static_cast<uint32_t>(std::max(n, 0));
  });
}

qd_status qd_probe_hbm(int32_t device, uint64_t bytes, uint32_t iters, double *read_gbs,
                       double *copy_gbs) {
  return guard([&] {
    if (!read_gbs || !copy_gbs) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    if (bytes < (uint64_t(1) << 20) || iters == 0)
      fail(QD_ERROR_INVALID_ARGUMENT, "probe needs at least 1 MiB and one iteration");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
      fail(QD_ERROR_NOT_SUPPORTED, "no HIP device visible");
    if (device < 0 || device >= ndev) fail(QD_ERROR_INVALID_ARGUMENT, "device %d out of range", device);
    check(hipSetDevice(device), "hipSetDevice");
    check(qd::probe_hbm(device, size_t(bytes), iters, read_gbs, copy_gbs), "HBM probe");
  });
}

qd_status qd_engine_create(const qd_config *config, qd_engine **out) {
  return guard([&] {
    if (!config || !out) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    const qd_config &c = *config;
    if (c.hidden == 0 || c.heads == 0 || c.kv_heads == 0 || c.intermediate == 0 ||
        c.vocab == 0 || c.layers == 0 || c.capacity == 0 || c.max_batch == 0)
      fail(QD_ERROR_INVALID_ARGUMENT, "zero-sized engine dimension");
    if (c.heads % c.kv_heads != 0)
      fail(QD_ERROR_INVALID_ARGUMENT, "heads %u not a multiple of kv_heads %u", c.heads, c.kv_heads);
    if (!(c.rms_eps > 0.0f) || !(c.rope_theta > 0.0f))
      fail(QD_ERROR_INVALID_ARGUMENT, "rms_eps and rope_theta must be positive");
    if (c.decoder_dtype != QD_DTYPE_F32 && c.decoder_dtype != QD_DTYPE_BF16 &&
        c.decoder_dtype != QD_DTYPE_F16)
      fail(QD_ERROR_INVALID_ARGUMENT,
           "decoder_dtype %u is none of QD_DTYPE_F32, QD_DTYPE_BF16 and QD_DTYPE_F16", c.decoder_dtype);
    if (!qd::shape_supported(static_cast<int>(c.hidden), static_cast<int>(c.intermediate),
                             static_cast<int>(c.heads), static_cast<int>(c.kv_heads),
                             static_cast<int>(c.head_dim)))
      fail(QD_ERROR_NOT_SUPPORTED,
           "unsupported shape: kernels are built for hidden 896, intermediate 4864 and "
           "14 query heads over 2 KV heads of head_dim 64");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
      fail(QD_ERROR_NOT_SUPPORTED, "no HIP device visible");
    if (c.device < 0 || c.device >= ndev)
      fail(QD_ERROR_INVALID_ARGUMENT, "device %d out of range (%d visible)", c.device, ndev);

    auto e = std::make_unique<qd_engine>();
    e->cfg = c;
    e->H = c.hidden;
    e->I = c.intermediate;
    e->NQ = c.heads;
    e->NKV = c.kv_heads;
    e->QD = size_t(c.heads) * qd::kHeadDim;
    e->KVD = size_t(c.kv_heads) * qd::kHeadDim;
    e->QKV = e->QD + 2 * e->KVD;
    e->V = c.vocab;
    e->L = c.layers;
    e->CAP = c.capacity;
    e->B = c.max_batch;
    e->wdtype = c.decoder_dtype == QD_DTYPE_BF16 ? qd::kWeightsBf16
                : c.decoder_dtype == QD_DTYPE_F16  ? qd::kWeightsF16
                                                   : qd::kWeightsF32;
    e->set_device();
    check(hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking), "hipStreamCreate");
    check(hipEventCreate(&e->ev_begin), "hipEventCreate");
    check(hipEventCreate(&e->ev_end), "hipEventCreate");

    // Layer weights in one arena: per layer wqkv | bqkv | wo | wg | wu | wd |
    // attn_norm | mlp_norm, each 256-byte aligned; the five matrices in
    // mat_elem() bytes per element, biases and norms in FP32.
    auto round = [](size_t bytes) { return (bytes + 255) / 256 * 256; };
    const size_t me = e->mat_elem();
    const size_t per_layer = round(e->QKV * e->H * me) + round(e->QKV * 4) + round(e->H * e->QD * me) +
                             2 * round(e->I * e->H * me) + round(e->H * e->I * me) + 2 * round(e->H * 4);
    e->weights_floats = per_layer * e->L / 4;
    e->weights = e->alloc<float>(e->weights_floats);
    e->layers.resize(e->L);
    for (size_t l = 0; l < e->L; ++l) {
      char *p = reinterpret_cast<char *>(e->weights) + l * per_layer;
      qd::LayerPtrs &w = e->layers[l];
      auto take = [&](size_t bytes) {
        const float *q = reinterpret_cast<const float *>(p);
        p += round(bytes);
        return q;
      };
      w.wqkv = take(e->QKV * e->H * me);
      w.bqkv = take(e->QKV * 4);
      w.wo = take(e->H * e->QD * me);
      w.wg = take(e->I * e->H * me);
      w.wu = take(e->I * e->H * me);
      w.wd = take(e->H * e->I * me);
      w.attn_norm = take(e->H * 4);
      w.mlp_norm = take(e->H * 4);
    }
    e->embed = e->alloc<float>(e->V * e->H);
    e->lm_head = c.tied_lm_head ? e->embed : e->alloc<float>(e->V * e->H);
    e->final_norm = e->alloc<float>(e->H);
    e->k_cache = e->alloc<float>(e->B * e->L * e->CAP * e->KVD);
    e->v_cache = e->alloc<float>(e->B * e->L * e->CAP * e->KVD);
    e->rope_cos = e->alloc<float>(e->CAP * qd::kRotary);
    e->rope_sin = e->alloc<float>(e->CAP * qd::kRotary);
    e->hidden = e->alloc<float>(e->B * e->H);
    e->q = e->alloc<float>(e->B * e->QD);
    e->attn = e->alloc<float>(e->B * e->QD);
    e->act = e->alloc<float>(e->B * e->I);
    e->logits = e->alloc<float>(e->B * e->V);
    e->part = e->alloc<float>(size_t(qd::kAttnMaxChunks) * e->NQ * qd::kPartStride);
    e->part_val = e->alloc<float>(kLmHeadParts);
    e->part_idx = e->alloc<uint32_t>(kLmHeadParts);
    e->tokens_dev = e->alloc<uint32_t>(e->CAP);
    e->states = e->alloc<qd::SeqState>(e->B);
    check(hipMemsetAsync(e->k_cache, 0, e->B * e->L * e->CAP * e->KVD * 4, e->stream), "memset");
    check(hipMemsetAsync(e->v_cache, 0, e->B * e->L * e->CAP * e->KVD * 4, e->stream), "memset");
    check(hipMemsetAsync(e->states, 0, e->B * sizeof(qd::SeqState), e->stream), "memset");
    check(hipHostMalloc(reinterpret_cast<void **>(&e->h_states), e->B * sizeof(qd::SeqState),
                        hipHostMallocDefault),
          "hipHostMalloc");
    check(hipHostMalloc(reinterpret_cast<void **>(&e->h_tokens), e->CAP * sizeof(uint32_t),
                        hipHostMallocDefault),
          "hipHostMalloc");
    check(hipHostMalloc(reinterpret_cast<void **>(&e->h_error), sizeof(uint32_t), hipHostMallocDefault),
          "hipHostMalloc");
    e->positions.assign(e->B, 0);
    e->build_rope_tables(c.rope_theta);

    // Resident path: the role-split kernel, one 512-thread workgroup on
    // every CU, all co-resident (cooperative launch), for the model shapes
    // it is built for. QD_RESIDENT=0 turns it off (the engine then
    // generates with the stream-ordered kernels); QD_RESIDENT_SPIN_LIMIT
    // lowers the polls a hand-off wait makes before it gives up (tests
    // force the give-up path with it).
    const int cus = qd::device_cu_count(c.device);
    e->cu_count = std::max(cus, 0);
    {
      qd::RolePlan cap_plan{};
      if (cus >= 64 && cus <= qd::kMaxRoleGrid &&
          qd::plan_roles(cus, int(e->H), int(e->I), int(e->NQ), int(e->NKV), int(e->CAP), &cap_plan))
        e->attn_parts = std::min(qd::kAttnMaxChunks, cap_plan.group_cus[1]);
    }
    const char *env = std::getenv("QD_RESIDENT");
    qd::RolePlan plan{};
    if (env && std::strcmp(env, "0") == 0) {
      e->resident_off_reason = "QD_RESIDENT=0";
    } else if (cus < 64 || cus > qd::kMaxRoleGrid || qd::roles_max_grid(c.device, e->wdtype) < cus) {
      e->resident_off_reason = "device cannot co-schedule one role workgroup per CU";
    } else if (!qd::plan_roles(cus, int(e->H), int(e->I), int(e->NQ), int(e->NKV), 1, &plan)) {
      e->resident_off_reason = "no role plan for this model shape";
    } else {
      e->roles_grid = cus;
    }
    if (const char *lim = std::getenv("QD_RESIDENT_SPIN_LIMIT")) {
      const long v = std::atol(lim);
      if (v >= 1 && v <= long(qd::kResidentSpinLimit)) e->spin_limit = uint32_t(v);
    }
    e->layer_ptrs_dev = e->alloc<qd::LayerPtrs>(e->L);
    check(hipMemcpyAsync(e->layer_ptrs_dev, e->layers.data(), e->L * sizeof(qd::LayerPtrs),
                         hipMemcpyHostToDevice, e->stream), "layer table upload");
    if (e->roles_grid) {
      e->top_pairs = e->alloc<uint64_t>(4 * size_t(e->roles_grid));
      check(hipMemsetAsync(e->top_pairs, 0, 4 * size_t(e->roles_grid) * 8, e->stream), "memset");
      e->roles_slot_bytes = 2 * e->L * 4 *
                            qd::roles_slot_floats(int(e->H), int(e->I), int(e->NQ), int(e->NKV));
      e->roles_slots = e->alloc<float>(e->roles_slot_bytes / 4);
    }
    e->resident_error = e->alloc<uint32_t>(1 + qd::kXcds);
    {
      hipError_t err = hipSuccess;
      e->batch_scratch = qd::batch_scratch(c.device, &err);
      if (!e->batch_scratch) e->batch_scratch_error = hipGetErrorString(err);
    }

    e->sync();
    *out = e.release();
  });
}

qd_status qd_engine_destroy(qd_engine *engine) {
  return guard([&] {
    if (!engine) return;
    engine->set_device();
    delete engine;
  });
}

qd_status qd_engine_config(const qd_engine *e, qd_config *config) {
  return guard([&] {
    if (!e || !config) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    *config = e->cfg;
  });
}

qd_status qd_engine_device_bytes(const qd_engine *e, uint64_t *bytes) {
  return guard([&] {
    if (!e || !bytes) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    *bytes = e->device_bytes;
  });
}

qd_status qd_engine_resident_grid(const qd_engine *e, uint32_t *grid) {
  return guard([&] {
    if (!e || !grid) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    *grid = static_cast<uint32_t>(e->roles_grid);
  });
}

qd_status qd_load_synthetic(qd_engine *e, uint64_t seed, const qd_synthetic_init *init) {
  return guard([&] {
    if (!e || !init) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    e->set_device();
    // Two pinned staging buffers, alternating, so host generation of one
    // chunk overlaps the copy of the previous one.
    const size_t chunk = size_t(16) << 20;  // floats
    float *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    auto cleanup = [&] {
      for (int k = 0; k < 2; ++k) {
        if (done[k]) (void)hipEventDestroy(done[k]);
        if (stage[k]) (void)hipHostFree(stage[k]);
      }
    };
    try {
      for (int k = 0; k < 2; ++k) {
        check(hipHostMalloc(reinterpret_cast<void **>(&stage[k]), chunk * 4, hipHostMallocDefault),
              "hipHostMalloc");
        check(hipEventCreateWithFlags(&done[k], hipEventDisableTiming), "hipEventCreate");
      }
      int slot = 0;
      bool pending[2] = {false, false};
      auto emit = [&](float *dst, size_t n, uint64_t stream_id, float stddev, bool constant) {
        for (size_t off = 0; off < n; off += chunk) {
          const size_t m = std::min(chunk, n - off);
          if (pending[slot]) check(hipEventSynchronize(done[slot]), "stage sync");
          if (constant) {
            std::fill(stage[slot], stage[slot] + m, stddev);
          } else {
            fill_normal(stage[slot], m, off, seed, stream_id, stddev);
          }
          e->upload(dst + off, stage[slot], m);
          check(hipEventRecord(done[slot], e->stream), "hipEventRecord");
          pending[slot] = true;
          slot ^= 1;
        }
      };
      // A decoder matrix from element `first`: FP32, or rounded to BF16 or
      // FP16 in the staging buffer itself (element i's two bytes land at or
      // below where its float was read) on such an engine.
      auto emit_mat = [&](const float *base, size_t first, size_t n, uint64_t stream_id, float stddev) {
        if (!e->narrow()) {
          emit(reinterpret_cast<float *>(e->mat_at(base, first)), n, stream_id, stddev, false);
          return;
        }
        for (size_t off = 0; off < n; off += chunk) {
          const size_t m = std::min(chunk, n - off);
          if (pending[slot]) check(hipEventSynchronize(done[slot]), "stage sync");
          fill_normal(stage[slot], m, off, seed, stream_id, stddev);
          uint16_t *h = reinterpret_cast<uint16_t *>(stage[slot]);
          for (size_t i = 0; i < m; ++i) h[i] = e->to_narrow(stage[slot][i]);
          check(hipMemcpyAsync(e->mat_at(base, first + off), h, m * 2, hipMemcpyHostToDevice, e->stream),
                "H2D");
          check(hipEventRecord(done[slot], e->stream), "hipEventRecord");
          pending[slot] = true;
          slot ^= 1;
        }
      };
      namespace b = qd::bundle;
      for (size_t l = 0; l < e->L; ++l) {
        const uint32_t li = static_cast<uint32_t>(l);
        const qd::LayerPtrs &w = e->layers[l];
        float *bq = const_cast<float *>(w.bqkv);
        emit_mat(w.wqkv, 0, e->QD * e->H, qd::rng::layer_stream(li, b::kQW), init->weight_std);
        emit_mat(w.wqkv, e->QD * e->H, e->KVD * e->H, qd::rng::layer_stream(li, b::kKW), init->weight_std);
        emit_mat(w.wqkv, (e->QD + e->KVD) * e->H, e->KVD * e->H, qd::rng::layer_stream(li, b::kVW),
                 init->weight_std);
        emit(bq, e->QD, qd::rng::layer_stream(li, b::kQB), init->bias_std, false);
        emit(bq + e->QD, e->KVD, qd::rng::layer_stream(li, b::kKB), init->bias_std, false);
        emit(bq + e->QD + e->KVD, e->KVD, qd::rng::layer_stream(li, b::kVB), init->bias_std, false);
        emit_mat(w.wo, 0, e->H * e->QD, qd::rng::layer_stream(li, b::kOW), init->weight_std);
        emit_mat(w.wg, 0, e->I * e->H, qd::rng::layer_stream(li, b::kGateW), init->weight_std);
        emit_mat(w.wu, 0, e->I * e->H, qd::rng::layer_stream(li, b::kUpW), init->weight_std);
        emit_mat(w.wd, 0, e->H * e->I, qd::rng::layer_stream(li, b::kDownW), init->weight_std);
        emit(const_cast<float *>(w.attn_norm), e->H, 0, init->norm_gain, true);
        emit(const_cast<float *>(w.mlp_norm), e->H, 0, init->norm_gain, true);
      }
      emit(e->embed, e->V * e->H, qd::rng::tail_stream(0), init->weight_std, false);
      emit(e->final_norm, e->H, 0, init->norm_gain, true);
      if (e->lm_head != e->embed)
        emit(e->lm_head, e->V * e->H, qd::rng::tail_stream(2), init->weight_std, false);
      e->sync();
    } catch (...) {
      (void)hipStreamSynchronize(e->stream);
      cleanup();
      throw;
    }
    cleanup();
    e->loaded = true;
  });
}

qd_status qd_load_bundle(qd_engine *e, const char *directory) {
  return guard([&] {
    if (!e || !directory) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    e->set_device();
    const std::string dir(directory);
    float theta = 0.0f;
    for (size_t l = 0; l < e->L; ++l) {
      const std::string path = dir + "/layer_" + std::to_string(l) + "/weights.json";
      qd::bundle::LayerWeights w = qd::bundle::load_layer(path);
      layer_shape_matches(*e, w);
      if (l == 0) {
        theta = w.rope_theta;
      } else if (w.rope_theta != theta) {
        fail(QD_ERROR_INVALID_ARGUMENT, "decoder layers use different rope_theta");
      }
      namespace b = qd::bundle;
      const qd::LayerPtrs &p = e->layers[l];
      float *bq = const_cast<float *>(p.bqkv);
      e->upload_mat(p.wqkv, 0, w.tensors[b::kQW].data(), e->QD * e->H);
      e->upload_mat(p.wqkv, e->QD * e->H, w.tensors[b::kKW].data(), e->KVD * e->H);
      e->upload_mat(p.wqkv, (e->QD + e->KVD) * e->H, w.tensors[b::kVW].data(), e->KVD * e->H);
      e->upload(bq, w.tensors[b::kQB].data(), e->QD);
      e->upload(bq + e->QD, w.tensors[b::kKB].data(), e->KVD);
      e->upload(bq + e->QD + e->KVD, w.tensors[b::kVB].data(), e->KVD);
      e->upload_mat(p.wo, 0, w.tensors[b::kOW].data(), e->H * e->QD);
      e->upload_mat(p.wg, 0, w.tensors[b::kGateW].data(), e->I * e->H);
      e->upload_mat(p.wu, 0, w.tensors[b::kUpW].data(), e->I * e->H);
      e->upload_mat(p.wd, 0, w.tensors[b::kDownW].data(), e->H * e->I);
      e->upload(const_cast<float *>(p.attn_norm), w.tensors[b::kAttnNorm].data(), e->H);
      e->upload(const_cast<float *>(p.mlp_norm), w.tensors[b::kMlpNorm].data(), e->H);
      e->sync();  // host vectors die at the end of this iteration
    }
    qd::bundle::TailWeights t = qd::bundle::load_tail(dir + "/model_tail/weights.json");
    // The persistent path requires full-vocabulary embeddings in vocabulary
    // order (benchmarks/qwen_stateful_graph.cpp:635-653).
    if (t.hidden != e->H || t.vocab != e->V || t.token_ids.size() != e->V)
      fail(QD_ERROR_INVALID_ARGUMENT, "model tail requires full-vocabulary embeddings");
    for (uint32_t i = 0; i < t.vocab; ++i)
      if (t.token_ids[i] != i)
        fail(QD_ERROR_INVALID_ARGUMENT, "model tail embeddings must use vocabulary order");
    if (e->lm_head == e->embed &&
        std::memcmp(t.lm_head_weight.data(), t.token_embeddings.data(),
                    t.lm_head_weight.size() * sizeof(float)) != 0)
      fail(QD_ERROR_INVALID_ARGUMENT,
           "engine has a tied LM head but the bundle's lm_head_weight differs from "
           "its token_embeddings");
    e->upload(e->embed, t.token_embeddings.data(), e->V * e->H);
    e->upload(e->final_norm, t.final_norm_weight.data(), e->H);
    if (e->lm_head != e->embed) e->upload(e->lm_head, t.lm_head_weight.data(), e->V * e->H);
    // No loaded NaN keeps its payload (see launch_canonical_nan).
    // (BF16 and FP16 matrices were canonicalised by their rounding; their
    // bytes are not FP32 words, so only the FP32 tensors of such an engine
    // are swept.)
    if (!e->narrow()) {
      check(qd::launch_canonical_nan(e->stream, e->weights, e->weights_floats), "canonical NaN");
    } else {
      for (const qd::LayerPtrs &p : e->layers) {
        check(qd::launch_canonical_nan(e->stream, const_cast<float *>(p.bqkv), e->QKV), "canonical NaN");
        check(qd::launch_canonical_nan(e->stream, const_cast<float *>(p.attn_norm), e->H), "canonical NaN");
        check(qd::launch_canonical_nan(e->stream, const_cast<float *>(p.mlp_norm), e->H), "canonical NaN");
      }
    }
    check(qd::launch_canonical_nan(e->stream, e->embed, e->V * e->H), "canonical NaN");
    check(qd::launch_canonical_nan(e->stream, e->final_norm, e->H), "canonical NaN");
    if (e->lm_head != e->embed)
      check(qd::launch_canonical_nan(e->stream, e->lm_head, e->V * e->H), "canonical NaN");
    e->sync();
    if (theta != e->cfg.rope_theta) e->build_rope_tables(theta);
    e->loaded = true;
  });
}

qd_status qd_read_weight(qd_engine *e, uint32_t layer, uint32_t kind, float *out, size_t count) {
  return guard([&] {
    if (!e || !out) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    e->set_device();
    const void *src = nullptr;
    size_t n = 0;
    bool mat = false;  // a decoder matrix: stored in mat_elem() bytes per element
    namespace b = qd::bundle;
    if (kind == 0x100) {
      src = e->embed; n = e->V * e->H;
    } else if (kind == 0x101) {
      src = e->final_norm; n = e->H;
    } else if (kind == 0x102) {
      src = e->lm_head; n = e->V * e->H;
    } else if (kind < b::kLayerTensorCount && layer < e->L) {
      const qd::LayerPtrs &p = e->layers[layer];
      switch (kind) {
        case b::kAttnNorm: src = p.attn_norm; n = e->H; break;
        case b::kMlpNorm: src = p.mlp_norm; n = e->H; break;
        case b::kQW: src = e->mat_at(p.wqkv, 0); n = e->QD * e->H; mat = true; break;
        case b::kKW: src = e->mat_at(p.wqkv, e->QD * e->H); n = e->KVD * e->H; mat = true; break;
        case b::kVW: src = e->mat_at(p.wqkv, (e->QD + e->KVD) * e->H); n = e->KVD * e->H; mat = true; break;
        case b::kQB: src = p.bqkv; n = e->QD; break;
        case b::kKB: src = p.bqkv + e->QD; n = e->KVD; break;
        case b::kVB: src = p.bqkv + e->QD + e->KVD; n = e->KVD; break;
        case b::kOW: src = p.wo; n = e->H * e->QD; mat = true; break;
        case b::kGateW: src = p.wg; n = e->I * e->H; mat = true; break;
        case b::kUpW: src = p.wu; n = e->I * e->H; mat = true; break;
        case b::kDownW: src = p.wd; n = e->H * e->I; mat = true; break;
      }
    }
    if (!src) fail(QD_ERROR_INVALID_ARGUMENT, "unknown tensor layer %u kind %u", layer, kind);
    if (count != n) fail(QD_ERROR_INVALID_ARGUMENT, "tensor has %zu elements, caller asked %zu", n, count);
    if (mat && e->narrow()) {
      // Widened to FP32 exactly, as the kernels read them.
      std::vector<uint16_t> h(n);
      check(hipMemcpyAsync(h.data(), src, n * 2, hipMemcpyDeviceToHost, e->stream), "D2H");
      e->sync();
      for (size_t i = 0; i < n; ++i) out[i] = e->from_narrow(h[i]);
      return;
    }
    check(hipMemcpyAsync(out, src, n * 4, hipMemcpyDeviceToHost, e->stream), "D2H");
    e->sync();
  });
}

qd_status qd_kv_reset(qd_engine *e, uint32_t seq, uint32_t position) {
  return guard([&] {
    if (!e) fail(QD_ERROR_INVALID_ARGUMENT, "null engine");
    e->check_seq(seq);
    if (position > e->CAP) fail(QD_ERROR_INVALID_ARGUMENT, "position %u beyond capacity %zu", position, e->CAP);
    e->set_device();
    e->positions[seq] = position;
    e->push_state(seq, 0, qd::kModeStep, UINT32_MAX, 0);
    e->sync();
  });
}

static void kv_copy(qd_engine *e, uint32_t seq, uint32_t layer, uint32_t start, uint32_t count,
                    float *k, float *v, bool write) {
  if (!e) fail(QD_ERROR_INVALID_ARGUMENT, "null engine");
  e->check_seq(seq);
  if (layer >= e->L) fail(QD_ERROR_INVALID_ARGUMENT, "layer %u out of range", layer);
  if (size_t(start) + count > e->CAP)
    fail(QD_ERROR_INVALID_ARGUMENT, "positions [%u, %u) beyond capacity %zu", start, start + count, e->CAP);
  if (count == 0) return;
  e->set_device();
  const size_t off = size_t(start) * e->KVD;
  const size_t bytes = size_t(count) * e->KVD * 4;
  float *dk = e->kv_slice(e->k_cache, seq, layer) + off;
  float *dv = e->kv_slice(e->v_cache, seq, layer) + off;
  const hipMemcpyKind kind = write ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost;
  if (k) check(hipMemcpyAsync(write ? static_cast<void *>(dk) : k, write ? static_cast<const void *>(k) : dk, bytes, kind, e->stream), "kv copy");
  if (v) check(hipMemcpyAsync(write ? static_cast<void *>(dv) : v, write ? static_cast<const void *>(v) : dv, bytes, kind, e->stream), "kv copy");
  if (write) {
    // Written rows hold no NaN payload but the canonical one.
    if (k) check(qd::launch_canonical_nan(e->stream, dk, size_t(count) * e->KVD), "canonical NaN");
    if (v) check(qd::launch_canonical_nan(e->stream, dv, size_t(count) * e->KVD), "canonical NaN");
  }
  e->sync();
}

qd_status qd_write_kv(qd_engine *e, uint32_t seq, uint32_t layer, uint32_t start, uint32_t count,
                      const float *k, const float *v) {
  return guard([&] { kv_copy(e, seq, layer, start, count, const_cast<float *>(k), const_cast<float *>(v), true); });
}

qd_status qd_read_kv(qd_engine *e, uint32_t seq, uint32_t layer, uint32_t start, uint32_t count,
                     float *k, float *v) {
  return guard([&] { kv_copy(e, seq, layer, start, count, k, v, false); });
}

qd_status qd_read_activation(qd_engine *e, uint32_t seq, uint32_t which, float *out, size_t count) {
  return guard([&] {
    if (!e || !out) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    e->check_seq(seq);
    const float *src = nullptr;
    size_t n = 0;
    switch (which) {
      case 0: src = e->hidden + size_t(seq) * e->H; n = e->H; break;
      case 1: src = e->q + size_t(seq) * e->QD; n = e->QD; break;
      case 2: src = e->attn + size_t(seq) * e->QD; n = e->QD; break;
      case 3: src = e->act + size_t(seq) * e->I; n = e->I; break;
      default: fail(QD_ERROR_INVALID_ARGUMENT, "unknown activation %u", which);
    }
    if (count != n) fail(QD_ERROR_INVALID_ARGUMENT, "activation has %zu elements, caller asked %zu", n, count);
    e->set_device();
    check(hipMemcpyAsync(out, src, n * 4, hipMemcpyDeviceToHost, e->stream), "D2H");
    e->sync();
  });
}

qd_status qd_read_decode_state(qd_engine *e, uint32_t seq, qd_decode_state *out) {
  return guard([&] {
    if (!e || !out) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    e->check_seq(seq);
    e->set_device();
    qd::SeqState s{};
    check(hipMemcpyAsync(&s, e->states + seq, sizeof(s), hipMemcpyDeviceToHost, e->stream), "D2H");
    e->sync();
    out->token_position = s.position;
    out->kv_length = s.position;
    out->sampled_token = s.token;
    out->eos_token = s.eos;
    out->generated_tokens = s.generated;
    out->maximum_tokens = s.max_tokens;
    out->stop_reason = s.stop_reason;
    out->sampled_logit = s.top_logit;
  });
}

qd_status qd_layer_step(qd_engine *e, uint32_t seq, uint32_t layer, float *hidden) {
  return guard([&] {
    if (!e || !hidden) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    e->check_seq(seq);
    e->check_loaded();
    if (layer >= e->L) fail(QD_ERROR_INVALID_ARGUMENT, "layer %u out of range", layer);
    if (e->positions[seq] >= e->CAP)
      fail(QD_ERROR_INVALID_ARGUMENT, "sequence %u is full (capacity %zu)", seq, e->CAP);
    e->set_device();
    e->push_state(seq, 0, qd::kModeStep, UINT32_MAX, 0);
    e->upload(e->hidden + seq * e->H, hidden, e->H);
    check(qd::launch_layer(e->stream, e->layer_args(seq, layer)), "layer launch");
    check(hipMemcpyAsync(hidden, e->hidden + seq * e->H, e->H * 4, hipMemcpyDeviceToHost, e->stream), "D2H");
    e->sync();
  });
}

qd_status qd_load_hidden(qd_engine *e, uint32_t seq, const float *hidden) {
  return guard([&] {
    if (!e || !hidden) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    e->check_seq(seq);
    e->set_device();
    e->upload(e->hidden + size_t(seq) * e->H, hidden, e->H);
    e->sync();
  });
}

qd_status qd_embed_hidden(qd_engine *e, uint32_t seq, uint32_t token) {
  return guard([&] {
    if (!e) fail(QD_ERROR_INVALID_ARGUMENT, "null engine");
    e->check_seq(seq);
    e->check_loaded();
    if (token >= e->V) fail(QD_ERROR_INVALID_ARGUMENT, "token %u >= vocab %zu", token, e->V);
    e->set_device();
    // The embedding kernel reads the token from the slot state.
    check(qd::launch_set_state(e->stream, e->states + seq, e->positions[seq], token), "state launch");
    check(qd::launch_embed(e->stream, e->embed, e->states + seq, e->hidden + size_t(seq) * e->H,
                           static_cast<int>(e->H), static_cast<int>(e->V)),
          "embed launch");
  });
}

qd_status qd_layer_decode(qd_engine *e, uint32_t seq, uint32_t first_layer, uint32_t layer_count,
                          uint32_t valid_keys) {
  return guard([&] {
    if (!e) fail(QD_ERROR_INVALID_ARGUMENT, "null engine");
    e->check_seq(seq);
    e->check_loaded();
    if (layer_count == 0 || first_layer >= e->L || layer_count > e->L - first_layer)
      fail(QD_ERROR_INVALID_ARGUMENT, "layers [%u, %u) outside [0, %zu)", first_layer,
           first_layer + layer_count, e->L);
    if (valid_keys == 0 || valid_keys > e->CAP)
      fail(QD_ERROR_INVALID_ARGUMENT, "valid_keys %u outside [1, capacity %zu]", valid_keys, e->CAP);
    e->set_device();
    // The query sits at position valid_keys - 1: the slot's position while
    // this token is in flight (qd_tail completes it).
    e->positions[seq] = valid_keys - 1;
    check(qd::launch_set_state(e->stream, e->states + seq, valid_keys - 1, 0), "state launch");
    for (uint32_t l = first_layer; l < first_layer + layer_count; ++l)
      check(qd::launch_layer(e->stream, e->layer_args(seq, l)), "layer launch");
  });
}

qd_status qd_tail(qd_engine *e, uint32_t seq, float *logits_out, uint32_t *greedy, float *top_logit) {
  return guard([&] {
    if (!e) fail(QD_ERROR_INVALID_ARGUMENT, "null engine");
    e->check_seq(seq);
    e->check_loaded();
    if (e->positions[seq] >= e->CAP)
      fail(QD_ERROR_INVALID_ARGUMENT, "sequence %u is full (capacity %zu)", seq, e->CAP);
    e->set_device();
    // A fresh step-mode state at the slot's position (a layer_decode call
    // left this; a qd_step or prefill left the position after its token).
    check(qd::launch_set_state(e->stream, e->states + seq, e->positions[seq], 0), "state launch");
    float *dev_logits = e->logits + size_t(seq) * e->V;
    check(qd::launch_tail(e->stream, e->tail_args(seq, dev_logits, 0, nullptr)), "tail launch");
    check(hipMemcpyAsync(&e->h_states[seq], e->states + seq, sizeof(qd::SeqState),
                         hipMemcpyDeviceToHost, e->stream), "D2H");
    if (logits_out)
      check(hipMemcpyAsync(logits_out, dev_logits, e->V * 4, hipMemcpyDeviceToHost, e->stream), "D2H");
    e->sync();
    e->positions[seq] += 1;
    if (greedy) *greedy = e->h_states[seq].token;
    if (top_logit) *top_logit = e->h_states[seq].top_logit;
  });
}

qd_status qd_read_logits(qd_engine *e, uint32_t seq, float *out, size_t count) {
  return guard([&] {
    if (!e || !out) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    e->check_seq(seq);
    if (count != e->V) fail(QD_ERROR_INVALID_ARGUMENT, "logits have %zu elements, caller asked %zu", e->V, count);
    e->set_device();
    check(hipMemcpyAsync(out, e->logits + size_t(seq) * e->V, e->V * 4, hipMemcpyDeviceToHost, e->stream),
          "D2H");
    e->sync();
  });
}

namespace {
// qd_step and qd_step_graph: the slot's state is written (a copy from
// pinned host memory), the step runs as launches or as the slot's graph,
// then the state and (optionally) the logits come back.
qd_status step_common(qd_engine *e, uint32_t seq, uint32_t token, float *logits_out, uint32_t *greedy,
                      float *top_logit, bool graph) {
  return guard([&] {
    if (!e) fail(QD_ERROR_INVALID_ARGUMENT, "null engine");
    e->check_seq(seq);
    e->check_loaded();
    if (token >= e->V) fail(QD_ERROR_INVALID_ARGUMENT, "token %u >= vocab %zu", token, e->V);
    if (e->positions[seq] >= e->CAP)
      fail(QD_ERROR_INVALID_ARGUMENT, "sequence %u is full (capacity %zu)", seq, e->CAP);
    e->set_device();
    float *dev_logits = e->logits + seq * e->V;
    // qd_step runs the resident kernel for one token when the engine has it
    // (one cooperative launch instead of the stream kernels' ~150); the graph
    // replays the stream kernels. Both compute the same values bit for bit.
    qd::RolePlan plan{};
    bool resident = !graph && e->resident_fits(1) && e->resident_plan(e->positions[seq] + 1, &plan);
    if (resident) {
      const hipError_t err = e->launch_resident(plan, seq, token, 1, UINT32_MAX, dev_logits, 0, nullptr);
      if (err != hipSuccess) {
        if (!e->resident_refused(err)) check(err, "resident launch");
        resident = false;
      }
    }
    if (!resident) {
      hipGraphExec_t g = graph ? e->step_graph(seq) : nullptr;
      e->push_state(seq, token, qd::kModeStep, UINT32_MAX, 0);
      if (g)
        check(hipGraphLaunch(g, e->stream), "hipGraphLaunch");
      else
        e->enqueue_step(seq, dev_logits, 0, nullptr);
    }
    check(hipMemcpyAsync(&e->h_states[seq], e->states + seq, sizeof(qd::SeqState),
                         hipMemcpyDeviceToHost, e->stream), "D2H");
    if (resident) e->enqueue_resident_error();
    if (logits_out)
      check(hipMemcpyAsync(logits_out, dev_logits, e->V * 4, hipMemcpyDeviceToHost, e->stream), "D2H");
    e->sync();
    if (resident) {
      e->resident_status(*e->h_error);
      // The slot's state as the stream step leaves it: a step, not a
      // one-token generation (the kernel wrote position, token and logit).
      qd::SeqState &h = e->h_states[seq];
      h.generated = 0;
      h.max_tokens = 0;
      h.stop_reason = 0;
      h.stopped = 0;
      h.eos = UINT32_MAX;
      h.mode = qd::kModeStep;
      check(hipMemcpyAsync(e->states + seq, &h, sizeof(h), hipMemcpyHostToDevice, e->stream),
            "state upload");
    }
    e->positions[seq] += 1;
    if (greedy) *greedy = e->h_states[seq].token;
    if (top_logit) *top_logit = e->h_states[seq].top_logit;
  });
}
}  // namespace

qd_status qd_step(qd_engine *e, uint32_t seq, uint32_t token, float *logits_out, uint32_t *greedy,
                  float *top_logit) {
  return step_common(e, seq, token, logits_out, greedy, top_logit, false);
}

qd_status qd_step_graph(qd_engine *e, uint32_t seq, uint32_t token, float *logits_out, uint32_t *greedy,
                        float *top_logit) {
  return step_common(e, seq, token, logits_out, greedy, top_logit, true);
}

namespace {

// Event pair around every launch; durations are read after one sync.
struct EventMarker : qd::Marker {
  struct Span {
    int kernel;
    size_t begin, end;
    double bytes, flops;
  };
  qd_engine *e;
  std::vector<hipEvent_t> pool;
  std::vector<std::pair<int, size_t>> open;  // (kernel, begin event index)
  std::vector<Span> spans;
  size_t used = 0;
  double ctx_a = 0, ctx_b = 0;  // workload of the launches being recorded
  std::function<std::pair<double, double>(int)> cost;  // (bytes, flops) of one launch
  explicit EventMarker(qd_engine *engine) : e(engine) {}
  ~EventMarker() override {
    for (hipEvent_t ev : pool) (void)hipEventDestroy(ev);
  }
  size_t next() {
    if (used == pool.size()) {
      hipEvent_t ev;
      check(hipEventCreate(&ev), "hipEventCreate");
      pool.push_back(ev);
    }
    check(hipEventRecord(pool[used], e->stream), "hipEventRecord");
    return used++;
  }
  void before(int kernel) override { open.emplace_back(kernel, next()); }
  void after(int kernel) override {
    const size_t b = open.back().second;
    open.pop_back();
    const std::pair<double, double> c = cost ? cost(kernel) : std::pair<double, double>{0, 0};
    spans.push_back({kernel, b, next(), c.first, c.second});
  }
  // Per-kernel totals (after the stream has synchronised), at most capacity.
  void report(const char *(*name)(int), int kernels, qd_kernel_stat *stats, uint32_t capacity,
              uint32_t *count) const {
    std::vector<qd_kernel_stat> agg(kernels);
    for (int k = 0; k < kernels; ++k) {
      std::memset(&agg[k], 0, sizeof(qd_kernel_stat));
      std::snprintf(agg[k].name, sizeof(agg[k].name), "%s", name(k));
    }
    for (const Span &sp : spans) {
      float ms = 0.f;
      check(hipEventElapsedTime(&ms, pool[sp.begin], pool[sp.end]), "hipEventElapsedTime");
      qd_kernel_stat &st = agg[sp.kernel];
      st.launches += 1;
      st.total_us += ms * 1000.0;
      st.bytes += sp.bytes;
      st.flops += sp.flops;
    }
    uint32_t n = 0;
    for (const auto &st : agg) {
      if (st.launches == 0) continue;
      if (n < capacity) stats[n] = st;
      ++n;
    }
    *count = std::min(n, capacity);
  }
};

// Validates a qd_prefill request.
void check_prefill(qd_engine *e, uint32_t seq, const uint32_t *tokens, uint32_t n) {
  if (!e || (!tokens && n)) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
  e->check_seq(seq);
  e->check_loaded();
  if (n == 0) fail(QD_ERROR_INVALID_ARGUMENT, "empty prompt");
  if (size_t(e->positions[seq]) + n > e->CAP)
    fail(QD_ERROR_INVALID_ARGUMENT, "prompt of %u tokens overflows capacity %zu at position %u", n, e->CAP,
         e->positions[seq]);
  for (uint32_t i = 0; i < n; ++i)
    if (tokens[i] >= e->V) fail(QD_ERROR_INVALID_ARGUMENT, "token %u at %u >= vocab", tokens[i], i);
  e->set_device();
}

// The prompt in chunks of up to kPrefillRows positions, each through all
// layers at once (dense GEMMs); then the tail (final norm, LM head, argmax)
// on the last position, which advances the slot to pos0 + n. m (nullable)
// times every launch.
void run_prefill(qd_engine *e, uint32_t seq, const uint32_t *tokens, uint32_t n, EventMarker *m) {
  if (e->narrow()) {
    // BF16 or FP16 decoder weights: the prompt runs position by position through the
    // stream-ordered step kernels (the prompt GEMMs read FP32 matrices),
    // writing every position's K/V row; then the tail on the last position.
    for (uint32_t i = 0; i < n; ++i) {
      check(qd::launch_set_state(e->stream, e->states + seq, e->positions[seq], tokens[i]), "state launch");
      check(qd::launch_embed(e->stream, e->embed, e->states + seq, e->hidden + size_t(seq) * e->H,
                             static_cast<int>(e->H), static_cast<int>(e->V)),
            "embed launch");
      for (size_t l = 0; l < e->L; ++l) check(qd::launch_layer(e->stream, e->layer_args(seq, l)), "layer launch");
      if (i + 1 < n) e->positions[seq] += 1;
    }
    e->push_state(seq, tokens[n - 1], qd::kModeStep, UINT32_MAX, 0);
    check(qd::launch_tail(e->stream, e->tail_args(seq, e->logits + seq * e->V, 0, nullptr), nullptr),
          "tail launch");
    e->positions[seq] += 1;
    return;
  }
  for (uint32_t done = 0; done < n;) {
    const uint32_t rows = std::min<uint32_t>(n - done, uint32_t(qd_engine::kPrefillRows));
    if (m) {
      m->ctx_a = rows;
      m->ctx_b = e->positions[seq] + done;
    }
    e->prefill_chunk(seq, tokens + done, int(rows), int(e->positions[seq] + done), m);
    done += rows;
    if (done == n)
      check(hipMemcpyAsync(e->hidden + size_t(seq) * e->H, e->pf_h + size_t(rows - 1) * e->H, e->H * 4,
                           hipMemcpyDeviceToDevice, e->stream),
            "D2D");
    e->sync();  // the next chunk's token upload reuses pf_tokens
  }
  e->positions[seq] += n - 1;
  e->push_state(seq, tokens[n - 1], qd::kModeStep, UINT32_MAX, 0);
  if (m) m->before(qd_engine::kPTail);
  check(qd::launch_tail(e->stream, e->tail_args(seq, e->logits + seq * e->V, 0, nullptr), nullptr),
        "tail launch");
  if (m) m->after(qd_engine::kPTail);
  e->positions[seq] += 1;
}

// Validates a qd_step_batch request.
void check_batch(qd_engine *e, uint32_t n_seq, const uint32_t *seq_ids, const uint32_t *tokens,
                 uint32_t steps) {
  if (!e || !seq_ids || !tokens) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
  e->check_loaded();
  if (e->narrow()) fail(QD_ERROR_NOT_SUPPORTED, "batched decode needs FP32 decoder weights");
  if (n_seq == 0 || n_seq > e->B) fail(QD_ERROR_INVALID_ARGUMENT, "n_seq %u out of range", n_seq);
  std::vector<bool> seen(e->B, false);
  for (uint32_t i = 0; i < n_seq; ++i) {
    e->check_seq(seq_ids[i]);
    if (seen[seq_ids[i]]) fail(QD_ERROR_INVALID_ARGUMENT, "sequence %u listed twice", seq_ids[i]);
    seen[seq_ids[i]] = true;
    if (tokens[i] >= e->V) fail(QD_ERROR_INVALID_ARGUMENT, "token %u >= vocab", tokens[i]);
    if (size_t(e->positions[seq_ids[i]]) + steps > e->CAP)
      fail(QD_ERROR_INVALID_ARGUMENT, "sequence %u is full", seq_ids[i]);
  }
  e->set_device();
}

// Enqueues one batched step of the listed slots (groups of kBatchRows) and
// leaves every row's greedy token and logit in bt_token / bt_top; m
// (nullable) times every launch.
void enqueue_step_batch(qd_engine *e, uint32_t n_seq, const uint32_t *seq_ids, const uint32_t *tokens,
                        EventMarker *m) {
  for (uint32_t first = 0; first < n_seq; first += qd::kBatchRows) {
    const int rows = static_cast<int>(std::min<uint32_t>(qd::kBatchRows, n_seq - first));
    const qd::BatchLaunch b = e->batch_args(seq_ids + first, tokens + first, rows);
    if (m) {
      m->ctx_a = rows;
      m->ctx_b = 0;
      for (int i = 0; i < rows; ++i) m->ctx_b += b.pos[i] + 1.0;
    }
    e->enqueue_batch(b, first, m);
  }
}

}  // namespace

qd_status qd_prefill(qd_engine *e, uint32_t seq, const uint32_t *tokens, uint32_t n, float *last_logits,
                     uint32_t *greedy, float *top_logit) {
  return guard([&] {
    check_prefill(e, seq, tokens, n);
    run_prefill(e, seq, tokens, n, nullptr);
    check(hipMemcpyAsync(&e->h_states[seq], e->states + seq, sizeof(qd::SeqState),
                         hipMemcpyDeviceToHost, e->stream), "D2H");
    if (last_logits)
      check(hipMemcpyAsync(last_logits, e->logits + seq * e->V, e->V * 4, hipMemcpyDeviceToHost, e->stream), "D2H");
    e->sync();
    if (greedy) *greedy = e->h_states[seq].token;
    if (top_logit) *top_logit = e->h_states[seq].top_logit;
  });
}

qd_status qd_step_batch(qd_engine *e, uint32_t n_seq, const uint32_t *seq_ids, const uint32_t *tokens,
                        float *logits, uint32_t *greedy) {
  return guard([&] {
    check_batch(e, n_seq, seq_ids, tokens, 1);
    // Groups of up to kBatchRows sequences share every weight read; the
    // kernels take each row's slot, token and position as arguments and
    // leave the slot's state as a batch-1 step would.
    enqueue_step_batch(e, n_seq, seq_ids, tokens, nullptr);
    check(hipMemcpyAsync(e->h_bt_out, e->bt_token, n_seq * 4, hipMemcpyDeviceToHost, e->stream), "D2H");
    check(hipMemcpyAsync(e->h_bt_out + e->B, e->bt_top, n_seq * 4, hipMemcpyDeviceToHost, e->stream),
          "D2H");
    if (logits)
      for (uint32_t i = 0; i < n_seq; ++i)
        check(hipMemcpyAsync(logits + size_t(i) * e->V, e->logits + size_t(seq_ids[i]) * e->V, e->V * 4,
                             hipMemcpyDeviceToHost, e->stream),
              "D2H");
    e->sync();
    for (uint32_t i = 0; i < n_seq; ++i) {
      e->positions[seq_ids[i]] += 1;
      if (greedy) greedy[i] = e->h_bt_out[i];
    }
  });
}

qd_status qd_step_batch_noalloc(qd_engine *e, uint32_t n_seq, const uint32_t *seq_ids,
                                const uint32_t *tokens, float *logits, uint32_t *greedy) {
  return guard([&] {
    if (!e || !seq_ids || !tokens) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    e->check_loaded();
    if (e->narrow()) fail(QD_ERROR_NOT_SUPPORTED, "batched decode needs FP32 decoder weights");
    if (n_seq == 0 || n_seq > uint32_t(qd::kBatchRows))
      fail(QD_ERROR_INVALID_ARGUMENT,
           "qd_step_batch_noalloc takes 1..%d sequences (its static workspace holds one group), got %u",
           qd::kBatchRows, n_seq);
    if (n_seq > e->B) fail(QD_ERROR_INVALID_ARGUMENT, "n_seq %u exceeds max_batch %zu", n_seq, e->B);
    for (uint32_t i = 0; i < n_seq; ++i) {
      e->check_seq(seq_ids[i]);
      for (uint32_t j = 0; j < i; ++j)
        if (seq_ids[j] == seq_ids[i]) fail(QD_ERROR_INVALID_ARGUMENT, "sequence %u listed twice", seq_ids[i]);
      if (tokens[i] >= e->V) fail(QD_ERROR_INVALID_ARGUMENT, "token %u >= vocab", tokens[i]);
      if (size_t(e->positions[seq_ids[i]]) + 1 > e->CAP)
        fail(QD_ERROR_INVALID_ARGUMENT, "sequence %u is full", seq_ids[i]);
    }
    if (!e->batch_scratch)
      fail(QD_ERROR_NOT_SUPPORTED, "static batch workspace unavailable: %s", e->batch_scratch_error.c_str());
    e->set_device();
    // One step at a time per GPU on the shared workspace.
    std::lock_guard<std::mutex> lock(qd::batch_scratch_lock(e->cfg.device));
    // Every buffer but the step's inputs and outputs (weights, KV cache,
    // slot states, the logits rows) lives in the static workspace.
    const qd::BatchWorkspace w = qd::carve_batch_workspace(e->batch_scratch, int(e->NQ));
    qd::BatchLaunch b{};
    b.rows = static_cast<int>(n_seq);
    for (uint32_t i = 0; i < n_seq; ++i) {
      b.slot[i] = seq_ids[i];
      b.pos[i] = e->positions[seq_ids[i]];
      b.token[i] = tokens[i];
    }
    b.states = e->states;
    b.hidden = w.hidden;
    b.q = w.q;
    b.attn = w.attn;
    b.act = w.act;
    b.part = w.part;
    b.split = w.split;
    b.counters = w.counters;
    b.k_cache = e->k_cache;
    b.v_cache = e->v_cache;
    b.rope_cos = e->rope_cos;
    b.rope_sin = e->rope_sin;
    b.layers = static_cast<int>(e->L);
    b.capacity = static_cast<int>(e->CAP);
    b.nq = static_cast<int>(e->NQ);
    b.nkv = static_cast<int>(e->NKV);
    b.eps = e->cfg.rms_eps;
    qd::BatchTail t{};
    t.final_norm = e->final_norm;
    t.head = e->lm_head;
    t.logits = e->logits;
    t.part_val = w.part_val;
    t.part_idx = w.part_idx;
    t.out_token = w.out_token;
    t.out_top = w.out_top;
    t.vocab = static_cast<int>(e->V);
    // The workspace keeps the last call's contents: the arrival counters
    // start at zero (a fill kernel, no memset node).
    check(qd::launch_batch_clear_counters(e->stream, w.counters), "counter clear");
    check(qd::launch_batch_embed(e->stream, b, e->embed, static_cast<int>(e->V)), "batch embed launch");
    for (size_t l = 0; l < e->L; ++l)
      check(qd::launch_batch_layer(e->stream, b, e->layers[l], static_cast<int>(l)), "batch layer launch");
    check(qd::launch_batch_tail(e->stream, b, t), "batch tail launch");
    if (greedy)
      check(hipMemcpyAsync(greedy, w.out_token, n_seq * 4, hipMemcpyDeviceToHost, e->stream), "D2H");
    if (logits)
      for (uint32_t i = 0; i < n_seq; ++i)
        check(hipMemcpyAsync(logits + size_t(i) * e->V, e->logits + size_t(seq_ids[i]) * e->V, e->V * 4,
                             hipMemcpyDeviceToHost, e->stream),
              "D2H");
    e->sync();
    for (uint32_t i = 0; i < n_seq; ++i) e->positions[seq_ids[i]] += 1;
  });
}

qd_status qd_generate_resident(qd_engine *e, uint32_t seq, uint32_t first_token, uint32_t max_tokens,
                               uint32_t eos, uint32_t *out_tokens, uint32_t *generated,
                               uint32_t *stop_reason, float *all_logits) {
  return guard([&] {
    if (!e || !out_tokens) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    e->check_seq(seq);
    e->check_loaded();
    if (max_tokens == 0) fail(QD_ERROR_INVALID_ARGUMENT, "max_tokens must be positive");
    if (first_token >= e->V) fail(QD_ERROR_INVALID_ARGUMENT, "token %u >= vocab", first_token);
    if (size_t(e->positions[seq]) + max_tokens > e->CAP)
      fail(QD_ERROR_INVALID_ARGUMENT, "generation of %u tokens from position %u overflows capacity %zu",
           max_tokens, e->positions[seq], e->CAP);
    e->set_device();
    float *hist = e->logits + size_t(seq) * e->V;
    int use_hist = 0;
    if (all_logits) {
      if (e->history_rows < max_tokens) {
        if (e->history) {
          check(hipFree(e->history), "hipFree");
          e->allocs.erase(std::find(e->allocs.begin(), e->allocs.end(), static_cast<void *>(e->history)));
          e->device_bytes -= std::max<size_t>(e->history_rows * e->V * 4, 256);
        }
        e->history = e->alloc<float>(size_t(max_tokens) * e->V);
        e->history_rows = max_tokens;
      }
      hist = e->history;
      use_hist = 1;
    }
    qd::RolePlan plan{};
    bool resident = e->resident_fits(max_tokens) && e->resident_plan(e->positions[seq] + max_tokens, &plan);
    check(hipEventRecord(e->ev_begin, e->stream), "hipEventRecord");
    if (resident) {
      // The kernel takes its start from the launch arguments and writes the
      // slot's whole state when it ends.
      const hipError_t err =
          e->launch_resident(plan, seq, first_token, max_tokens, eos, hist, use_hist, nullptr);
      if (err != hipSuccess) {
        if (!e->resident_refused(err)) check(err, "resident launch");
        resident = false;
      }
    }
    if (!resident) {
      e->push_state(seq, first_token, qd::kModeGenerate, eos, max_tokens);
      for (uint32_t t = 0; t < max_tokens; ++t) e->enqueue_step(seq, hist, use_hist, e->tokens_dev);
    }
    check(hipEventRecord(e->ev_end, e->stream), "hipEventRecord");
    // One synchronisation for the state, the error word and the tokens (all
    // max_tokens words); a one-token generation's logits row comes along.
    check(hipMemcpyAsync(&e->h_states[seq], e->states + seq, sizeof(qd::SeqState), hipMemcpyDeviceToHost,
                         e->stream), "D2H");
    if (resident) e->enqueue_resident_error();
    check(hipMemcpyAsync(e->h_tokens, e->tokens_dev, size_t(max_tokens) * 4, hipMemcpyDeviceToHost,
                         e->stream), "D2H");
    const bool row_now = all_logits && max_tokens == 1;
    if (row_now)
      check(hipMemcpyAsync(all_logits, e->history, e->V * 4, hipMemcpyDeviceToHost, e->stream), "D2H");
    e->sync();
    if (resident) e->resident_status(*e->h_error);
    const qd::SeqState &s = e->h_states[seq];
    const uint32_t n = std::min(s.generated, max_tokens);
    std::memcpy(out_tokens, e->h_tokens, size_t(n) * 4);
    if (all_logits && n && !row_now) {
      check(hipMemcpyAsync(all_logits, e->history, size_t(n) * e->V * 4, hipMemcpyDeviceToHost, e->stream), "D2H");
      e->sync();
    }
    float ms = 0.f;
    check(hipEventElapsedTime(&ms, e->ev_begin, e->ev_end), "hipEventElapsedTime");
    e->timing.total_us = ms * 1000.0;
    e->timing.tokens = n;
    e->timing.per_token_us = n ? e->timing.total_us / n : 0.0;
    e->positions[seq] = s.position;
    if (generated) *generated = n;
    if (stop_reason) *stop_reason = s.stop_reason;
  });
}


qd_status qd_profile_kernels(qd_engine *e, uint32_t seq, uint32_t first_token, uint32_t tokens,
                             qd_kernel_stat *stats, uint32_t capacity, uint32_t *count) {
  return guard([&] {
    if (!e || !stats || !count) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    e->check_seq(seq);
    e->check_loaded();
    if (tokens == 0) fail(QD_ERROR_INVALID_ARGUMENT, "tokens must be positive");
    if (first_token >= e->V) fail(QD_ERROR_INVALID_ARGUMENT, "token %u >= vocab", first_token);
    if (size_t(e->positions[seq]) + tokens > e->CAP)
      fail(QD_ERROR_INVALID_ARGUMENT, "profiling %u tokens overflows capacity", tokens);
    e->set_device();
    EventMarker marker(e);
    marker.cost = [&](int k) {
      return std::pair<double, double>{e->kernel_bytes(k, marker.ctx_a), e->kernel_flops(k, marker.ctx_a)};
    };
    e->push_state(seq, first_token, qd::kModeGenerate, UINT32_MAX, tokens);
    for (uint32_t t = 0; t < tokens; ++t) {
      marker.ctx_a = double(e->positions[seq]) + t + 1;
      e->enqueue_step(seq, e->logits + size_t(seq) * e->V, 0, e->tokens_dev, &marker);
    }
    e->sync();
    e->positions[seq] += tokens;
    marker.report(qd::kernel_name, qd::kKernelCount, stats, capacity, count);
  });
}

qd_status qd_profile_batch(qd_engine *e, uint32_t n_seq, const uint32_t *seq_ids, const uint32_t *tokens,
                           uint32_t steps, qd_kernel_stat *stats, uint32_t capacity, uint32_t *count) {
  return guard([&] {
    if (!stats || !count) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    if (steps == 0) fail(QD_ERROR_INVALID_ARGUMENT, "steps must be positive");
    check_batch(e, n_seq, seq_ids, tokens, steps);
    EventMarker marker(e);
    marker.cost = [&](int k) { return e->batch_cost(k, marker.ctx_a, marker.ctx_b); };
    std::vector<uint32_t> feed(tokens, tokens + n_seq);
    for (uint32_t step = 0; step < steps; ++step) {
      enqueue_step_batch(e, n_seq, seq_ids, feed.data(), &marker);
      check(hipMemcpyAsync(e->h_bt_out, e->bt_token, n_seq * 4, hipMemcpyDeviceToHost, e->stream), "D2H");
      e->sync();
      for (uint32_t i = 0; i < n_seq; ++i) {
        e->positions[seq_ids[i]] += 1;
        // A NaN row has no token to feed back: it repeats its input.
        if (e->h_bt_out[i] < e->V) feed[i] = e->h_bt_out[i];
      }
    }
    marker.report(qd::batch_kernel_name, qd::kBatchKernelCount, stats, capacity, count);
  });
}

qd_status qd_profile_prefill(qd_engine *e, uint32_t seq, const uint32_t *tokens, uint32_t n,
                             qd_kernel_stat *stats, uint32_t capacity, uint32_t *count) {
  return guard([&] {
    if (!stats || !count) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    check_prefill(e, seq, tokens, n);
    EventMarker marker(e);
    marker.cost = [&](int k) { return e->prefill_cost(k, marker.ctx_a, marker.ctx_b); };
    run_prefill(e, seq, tokens, n, &marker);
    e->sync();
    marker.report(qd_engine::prefill_kernel_name, qd_engine::kPrefillKernels, stats, capacity, count);
  });
}

namespace {

// One profiled resident launch of `tokens` tokens: stage totals of
// workgroup 0 into ticks_out[kResidentStages] and, when trace_out is set,
// every workgroup's timeline of token trace_token.
void profiled_resident_launch(qd_engine *e, uint32_t seq, uint32_t first_token, uint32_t tokens,
                              uint64_t *ticks_out, uint64_t *trace_out, uint32_t trace_token) {
  e->check_seq(seq);
  e->check_loaded();
  if (e->roles_grid == 0)
    fail(QD_ERROR_NOT_SUPPORTED, "resident path disabled: %s", e->resident_off_reason.c_str());
  if (tokens == 0) fail(QD_ERROR_INVALID_ARGUMENT, "tokens must be positive");
  if (first_token >= e->V) fail(QD_ERROR_INVALID_ARGUMENT, "token %u >= vocab", first_token);
  if (size_t(e->positions[seq]) + tokens > e->CAP)
    fail(QD_ERROR_INVALID_ARGUMENT, "profiling %u tokens overflows capacity", tokens);
  if (!e->resident_fits(tokens)) fail(QD_ERROR_INVALID_ARGUMENT, "too many tokens for one resident launch");
  qd::RolePlan plan{};
  if (!e->resident_plan(e->positions[seq] + tokens, &plan))
    fail(QD_ERROR_NOT_SUPPORTED, "no resident role plan reaches context %zu", size_t(e->positions[seq]) + tokens);
  e->set_device();
  const size_t trace_elems =
      trace_out ? size_t(e->roles_grid) * (e->L + 1) * qd::kResidentStages : 0;
  // Temporary buffers of a diagnostic call, released before returning.
  uint64_t *ticks = nullptr, *trace = nullptr;
  check(hipMalloc(&ticks, qd::kResidentStages * sizeof(uint64_t)), "hipMalloc");
  if (trace_elems && hipMalloc(&trace, trace_elems * sizeof(uint64_t)) != hipSuccess) {
    (void)hipFree(ticks);
    fail(QD_ERROR_RUNTIME, "hipMalloc of the trace buffer failed");
  }
  auto release = [&] {
    (void)hipFree(ticks);
    if (trace) (void)hipFree(trace);
  };
  try {
    check(hipMemsetAsync(ticks, 0, qd::kResidentStages * sizeof(uint64_t), e->stream), "memset");
    if (trace) check(hipMemsetAsync(trace, 0, trace_elems * sizeof(uint64_t), e->stream), "memset");
    const hipError_t launched = e->launch_resident(plan, seq, first_token, tokens, UINT32_MAX,
                                                   e->logits + size_t(seq) * e->V, 0, ticks, trace,
                                                   trace_token);
    if (launched != hipSuccess) {
      if (e->resident_refused(launched))
        fail(QD_ERROR_NOT_SUPPORTED, "%s", e->resident_off_reason.c_str());
      check(launched, "resident launch");
    }
    check(hipMemcpyAsync(ticks_out, ticks, qd::kResidentStages * sizeof(uint64_t),
                         hipMemcpyDeviceToHost, e->stream), "D2H");
    if (trace)
      check(hipMemcpyAsync(trace_out, trace, trace_elems * sizeof(uint64_t), hipMemcpyDeviceToHost,
                           e->stream), "D2H");
    check(hipMemcpyAsync(&e->h_states[seq], e->states + seq, sizeof(qd::SeqState),
                         hipMemcpyDeviceToHost, e->stream), "D2H");
    e->sync();
    e->check_resident_error();
    e->positions[seq] = e->h_states[seq].position;
  } catch (...) {
    release();
    throw;
  }
  release();
}

}  // namespace

qd_status qd_profile_resident(qd_engine *e, uint32_t seq, uint32_t first_token, uint32_t tokens,
                              double *stage_us, uint32_t capacity, uint32_t *count) {
  return guard([&] {
    if (!e || !stage_us || !count) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    uint64_t h[qd::kResidentStages] = {};
    profiled_resident_launch(e, seq, first_token, tokens, h, nullptr, 0);
    const uint32_t n = std::min<uint32_t>(capacity, qd::kResidentStages);
    for (uint32_t s = 0; s < n; ++s) stage_us[s] = double(h[s]) / 100.0;  // 100 MHz
    *count = n;
  });
}

qd_status qd_trace_resident(qd_engine *e, uint32_t seq, uint32_t first_token, uint32_t tokens,
                            uint32_t trace_token, uint64_t *timeline, size_t capacity,
                            uint32_t *workgroups, uint32_t *rows, uint32_t *stages) {
  return guard([&] {
    if (!e || !timeline || !workgroups || !rows || !stages)
      fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    if (trace_token >= tokens) fail(QD_ERROR_INVALID_ARGUMENT, "trace_token must be below tokens");
    e->check_seq(seq);
    const int grid = e->roles_grid;
    const size_t need = size_t(grid) * (e->L + 1) * qd::kResidentStages;
    *workgroups = uint32_t(grid);
    *rows = uint32_t(e->L + 1);
    *stages = qd::kResidentStages;
    if (e->roles_grid == 0)
      fail(QD_ERROR_NOT_SUPPORTED, "resident path disabled: %s", e->resident_off_reason.c_str());
    if (capacity < need) fail(QD_ERROR_INVALID_ARGUMENT, "timeline needs %zu entries", need);
    uint64_t h[qd::kResidentStages] = {};
    profiled_resident_launch(e, seq, first_token, tokens, h, timeline, trace_token);
  });
}

qd_status qd_last_timing(const qd_engine *e, qd_timing *timing) {
  return guard([&] {
    if (!e || !timing) fail(QD_ERROR_INVALID_ARGUMENT, "null argument");
    *timing = e->timing;
  });
}

qd_status qd_sync(qd_engine *e) {
  return guard([&] {
    if (!e) fail(QD_ERROR_INVALID_ARGUMENT, "null engine");
    e->set_device();
    e->sync();
  });
}

}  // extern "C"
