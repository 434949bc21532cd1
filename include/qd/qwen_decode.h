/*
 * qwen_decode.h -- C ABI of the MI355X-native Qwen2 FP32 decode engine.
 *
 * The engine keeps FP32 weights, the KV cache and the decode state resident
 * in HBM and runs the decode step as hand-written gfx950 HIP kernels. Plain
 * pointers and sizes only: every host buffer below is ordinary host memory,
 * every size is in elements unless it says bytes.
 *
 * Conventions (mirroring the reference runtime's C ABI, include/lrrt/lrrt.h):
 *   - every call returns qd_status with the numeric values of lr_status_t
 *     (include/lrrt/lrrt.h:17-25); no exception crosses the ABI;
 *   - qd_last_error() returns the calling thread's last diagnostic text;
 *   - the engine owns all device memory; qd_engine_destroy waits for pending
 *     work (include/lrrt/lrrt.h:92-93);
 *   - one engine is driven by one host thread at a time;
 *   - the KV cache never travels through the host between steps
 *     (docs/iree-qwen-kv-cache-abi.md:283-290).
 *
 * Position convention: every sequence slot has a position = number of tokens
 * whose K/V are in its cache = the slot the next consumed token writes.
 */
#ifndef QD_QWEN_DECODE_H_
#define QD_QWEN_DECODE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QD_API __attribute__((visibility("default")))

/* Same numeric values as lr_status_t (include/lrrt/lrrt.h:17-25). */
typedef enum qd_status {
  QD_SUCCESS = 0,
  QD_ERROR_INVALID_ARGUMENT = 1,
  QD_ERROR_NOT_INITIALIZED = 2,
  QD_ERROR_ALREADY_INITIALIZED = 3,
  QD_ERROR_NOT_SUPPORTED = 4,
  QD_ERROR_RUNTIME = 5,
  QD_ERROR_DEVICE_FAULT = 6
} qd_status;

/* Mirrors the reference's StopReason (executor/qwen/stateful_graph_context.hpp:87-91). */
typedef enum qd_stop_reason {
  QD_STOP_NONE = 0,
  QD_STOP_MAXIMUM_TOKENS = 1,
  QD_STOP_EOS_TOKEN = 2
} qd_stop_reason;

/* Model shape and engine capacity. The shape fields carry the meaning of the
 * reference's DecoderLayerShape / ModelTailWeights
 * (executor/qwen/weight_bundle.hpp:21-58) plus the eps and theta the
 * persistent path hard-codes (benchmarks/qwen_stateful_graph.cpp:379,818). */
typedef struct qd_config {
  uint32_t hidden;       /* 896 */
  uint32_t heads;        /* 14 query heads (the only supported value) */
  uint32_t kv_heads;     /* 2 (the only supported value with 14 heads) */
  uint32_t head_dim;     /* 64 (the only supported value) */
  uint32_t intermediate; /* 4864 */
  uint32_t vocab;        /* 151936 */
  uint32_t layers;       /* 24 */
  uint32_t capacity;     /* KV positions per sequence slot */
  uint32_t max_batch;    /* sequence slots */
  uint32_t tied_lm_head; /* nonzero: LM head aliases the token embeddings */
  float rms_eps;         /* 1e-6 */
  float rope_theta;      /* 1e6 */
  int32_t device;        /* HIP device ordinal */
  uint32_t decoder_dtype; /* qd_dtype of the decoder layers' matrices (wqkv, wo,
                           * gate, up, down): QD_DTYPE_F32 (0), QD_DTYPE_BF16 or
                           * QD_DTYPE_F16, with biases, norms, embeddings and the
                           * LM head kept in FP32 (the reference's FP16- and
                           * BF16-decoder + FP32-tail modes,
                           * examples/qwen/README.md:291-300). The matrices are
                           * rounded to nearest even when loaded; every kernel
                           * reads them at half the bytes, widens each value
                           * exactly and computes in FP32 in the FP32 order, so
                           * such an engine equals an FP32 engine loaded with the
                           * rounded weights bit for bit. It runs the resident
                           * kernel; it has no batched step (QD_ERROR_NOT_SUPPORTED),
                           * and its prefill runs the prompt position by position. */
} qd_config;

/* Storage types of qd_config.decoder_dtype. */
typedef enum qd_dtype { QD_DTYPE_F32 = 0, QD_DTYPE_BF16 = 1, QD_DTYPE_F16 = 2 } qd_dtype;

/* Distributions for qd_load_synthetic (0.02, 0.01, 1.0). */
typedef struct qd_synthetic_init {
  float weight_std; /* projections and token embeddings: N(0, weight_std) */
  float bias_std;   /* q/k/v biases: N(0, bias_std) */
  float norm_gain;  /* every RMSNorm gain */
  float reserved;
} qd_synthetic_init;

/* Device-resident decode state of one sequence slot; same fields as the
 * reference's DecodeState (executor/qwen/stateful_graph_context.hpp:96-105),
 * except that `token_position` is the next free slot (see above). */
typedef struct qd_decode_state {
  uint32_t token_position;
  uint32_t kv_length;
  uint32_t sampled_token;
  uint32_t eos_token;
  uint32_t generated_tokens;
  uint32_t maximum_tokens;
  uint32_t stop_reason;
  float sampled_logit;
} qd_decode_state;

/* Per-engine timing of the last qd_generate_resident call (HIP events on the
 * engine stream), in microseconds. */
typedef struct qd_timing {
  double total_us;
  double per_token_us;
  uint32_t tokens;
  uint32_t reserved;
} qd_timing;

/* Per-kernel totals from the qd_profile_* calls: summed HIP-event durations,
 * summed algorithmic bytes (bytes the kernel must move at minimum) and
 * summed floating-point operations (a multiply-add counts 2) of its
 * launches. */
typedef struct qd_kernel_stat {
  char name[48];
  uint32_t launches;
  uint32_t reserved;
  double total_us;
  double bytes;
  double flops;
} qd_kernel_stat;

typedef struct qd_engine qd_engine;

QD_API const char *qd_status_string(qd_status status);
QD_API const char *qd_last_error(void);
QD_API uint32_t qd_abi_version(void);
/* Number of visible HIP devices (0 on a host without a GPU). */
QD_API qd_status qd_device_count(uint32_t *count);

/* Creates an engine: allocates weights, KV cache [max_batch][layers]
 * [capacity][kv_heads*head_dim] and scratch on `config->device`. Replaces
 * the reference's DecoderLayer / ModelTail constructors
 * (examples/triton/mini_decoder_layer.hpp:205-254,770-800) and the device
 * buffers of benchmarks/qwen_stateful_graph.cpp:935-1010. */
QD_API qd_status qd_engine_create(const qd_config *config, qd_engine **engine);
/* Waits for pending work, then frees everything. */
QD_API qd_status qd_engine_destroy(qd_engine *engine);
QD_API qd_status qd_engine_config(const qd_engine *engine, qd_config *config);
/* Total device bytes held by the engine. */
QD_API qd_status qd_engine_device_bytes(const qd_engine *engine, uint64_t *bytes);

/* Workgroups of the resident decode megakernel qd_generate_resident uses
 * (one per CU), or 0 when the engine generates with stream-ordered kernels
 * (QD_RESIDENT=0 in the environment at create time, a device that cannot
 * co-schedule one workgroup per CU, or a refused cooperative launch). A
 * resident hand-off wait that gives up (a producer never published within
 * its spin limit) fails the call with QD_ERROR_DEVICE_FAULT; every
 * workgroup still exits. */
QD_API qd_status qd_engine_resident_grid(const qd_engine *engine,
                                         uint32_t *grid);

/* Loads a reference weight bundle directory: layer_<i>/weights.json for each
 * layer plus model_tail/weights.json. Replaces load_decoder_layer_weights and
 * load_model_tail_weights (executor/qwen/weight_bundle.hpp:460-602) feeding
 * the device copies of benchmarks/qwen_stateful_graph.cpp:858-910. */
QD_API qd_status qd_load_bundle(qd_engine *engine, const char *directory);
/* Fills every weight from the counter-based generator (seeded, identical to
 * the oracle's). Replaces the synthetic fill of
 * benchmarks/qwen_stateful_graph.cpp:615-621,794-832. */
QD_API qd_status qd_load_synthetic(qd_engine *engine, uint64_t seed,
                                   const qd_synthetic_init *init);
/* Copies one tensor of the resident weights back to the host (tests).
 * kind: 0..11 layer tensors in bundle order, 0x100 embeddings, 0x101 final
 * norm, 0x102 LM head. `count` must equal the tensor's element count. */
QD_API qd_status qd_read_weight(qd_engine *engine, uint32_t layer,
                                uint32_t kind, float *out, size_t count);

/* Sets a sequence slot's position (KV length) without touching cache
 * contents; resets its decode state. Mirrors ResidentExecutor::initialize and
 * initialize_decode_state (include/lrrt/persistent_graph/resident_executor.hpp:329-356,
 * benchmarks/qwen_stateful_graph.cpp:1256-1270). */
QD_API qd_status qd_kv_reset(qd_engine *engine, uint32_t seq,
                             uint32_t position);
/* Writes / reads `count` positions of one layer's K and V starting at
 * `start`, token-major [count][kv_heads*head_dim]. Writing mirrors the KV
 * half of DecoderLayer::copy_inputs (examples/triton/mini_decoder_layer.hpp:256-276);
 * every written NaN is stored as the canonical quiet NaN 0x7FC00000, as are
 * NaNs in weights loaded by qd_load_bundle. */
QD_API qd_status qd_write_kv(qd_engine *engine, uint32_t seq, uint32_t layer,
                             uint32_t start, uint32_t count, const float *k,
                             const float *v);
QD_API qd_status qd_read_kv(qd_engine *engine, uint32_t seq, uint32_t layer,
                            uint32_t start, uint32_t count, float *k,
                            float *v);
/* Diagnostics: copies the slot's current activation vector `which`
 * (0 hidden [hidden], 1 query [heads*64], 2 attention output [heads*64],
 * 3 SwiGLU activation [intermediate]) to the host. */
QD_API qd_status qd_read_activation(qd_engine *engine, uint32_t seq,
                                    uint32_t which, float *out, size_t count);
QD_API qd_status qd_read_decode_state(qd_engine *engine, uint32_t seq,
                                      qd_decode_state *state);

/* One decoder layer on a host hidden vector at the slot's current position
 * (writes K/V at that position, attends over 0..position), in place. Does
 * not advance the position. The host round trip of copy_inputs + run +
 * copy_output of one reference DecoderLayer (single-layer checks such as
 * BASELINE config 1); the device-resident hand-off is qd_layer_decode. */
QD_API qd_status qd_layer_step(qd_engine *engine, uint32_t seq,
                               uint32_t layer, float *hidden);

/* ---- layer-by-layer decode (the reference executor surface) ----------------
 * The slot's device hidden vector is the hand-off between these calls: it
 * never travels through the host. A driver of the reference stack
 * (benchmarks/triton_mini_decoder_layer.cpp:1051-1068) maps to
 *   qd_embed_hidden (or qd_load_hidden), qd_layer_decode per layer (or one
 *   call for the whole stack), qd_tail, qd_read_logits,
 * and produces exactly qd_step's logits, token and K/V rows. */

/* Host row -> the slot's device hidden vector (the next layer's input).
 * Replaces DecoderLayer::copy_hidden_state
 * (examples/triton/mini_decoder_layer.hpp:286-303). Synchronous. */
QD_API qd_status qd_load_hidden(qd_engine *engine, uint32_t seq,
                                const float *hidden);
/* hidden = embeddings[token] on the device: the lookup the reference
 * driver does on the host before copy_hidden_state
 * (benchmarks/triton_mini_decoder_layer.cpp:1052-1054). Asynchronous. */
QD_API qd_status qd_embed_hidden(qd_engine *engine, uint32_t seq,
                                 uint32_t token);
/* Decoder layers [first_layer, first_layer + layer_count) on the slot's
 * device hidden vector for the query at position valid_keys - 1: each layer
 * writes its K/V row there, attends over positions 0..valid_keys - 1 and
 * leaves its output on the device as the next layer's input. Sets the
 * slot's position to valid_keys - 1 (the token in flight; qd_tail
 * completes it). Asynchronous: errors surface at the next synchronising
 * call. Replaces DecoderLayer::decode_to_hidden_state / decode_to_buffer
 * (examples/triton/mini_decoder_layer.hpp:345-372), whose valid_keys it
 * takes. */
QD_API qd_status qd_layer_decode(qd_engine *engine, uint32_t seq,
                                 uint32_t first_layer, uint32_t layer_count,
                                 uint32_t valid_keys);
/* Final RMSNorm + LM head + argmax (lowest index on ties) on the slot's
 * device hidden vector; advances the slot's position by one. logits_out
 * (vocab floats), greedy_out and top_logit may be NULL; the logits also
 * stay on the device for qd_read_logits. Replaces ModelTail::run
 * (examples/triton/mini_decoder_layer.hpp:819-859) plus the host top_logits
 * of benchmarks/triton_mini_decoder_layer.cpp:394-422. Synchronous. */
QD_API qd_status qd_tail(qd_engine *engine, uint32_t seq, float *logits_out,
                         uint32_t *greedy_out, float *top_logit);
/* The slot's logits of its last qd_step / qd_tail / qd_prefill /
 * qd_step_batch / qd_step_batch_noalloc (`count` must equal vocab). Replaces ModelTail::copy_logits
 * (examples/triton/mini_decoder_layer.hpp:866-871). */
QD_API qd_status qd_read_logits(qd_engine *engine, uint32_t seq, float *out,
                                size_t count);

/* One full decode step of `token_in` at the slot's position: embedding, all
 * layers, final norm, LM head, argmax (lowest index on ties); advances the
 * position by one. logits_out (vocab floats) and top_logit may be NULL.
 * Runs as one launch of the resident kernel when the engine has one (else,
 * and with QD_RESIDENT=0, as the stream-ordered kernels); the two compute
 * the same values bit for bit and leave the same decode state. Replaces the
 * per-token loop body of benchmarks/triton_mini_decoder_layer.cpp:1041-1076
 * (stack + ModelTail::run + copy_logits + host top_logits). */
QD_API qd_status qd_step(qd_engine *engine, uint32_t seq, uint32_t token_in,
                         float *logits_out, uint32_t *greedy_out,
                         float *top_logit);

/* The stream-ordered step through a HIP graph: the slot's launch sequence
 * (embedding, every layer, LM head, argmax: 147 kernels at 24 layers) is
 * captured on the
 * slot's first call and replayed by one hipGraphLaunch per token after that;
 * the kernels read the position and token from the slot's device state, so
 * one graph serves every step. Same arguments, semantics and results (bit
 * for bit) as qd_step. Replaces the reference's HIP-Graph step
 * (benchmarks/qwen_hip_graph.hpp:27-199, timed beside the resident path in
 * docs/stateful-graph.md:636-650). */
QD_API qd_status qd_step_graph(qd_engine *engine, uint32_t seq, uint32_t token_in,
                               float *logits_out, uint32_t *greedy_out,
                               float *top_logit);

/* Prefill of n tokens from the slot's position; advances it by n. Writes the
 * last position's logits (nullable) and greedy token. Semantically n
 * sequential qd_step calls (the reference's prompt stack,
 * benchmarks/triton_mini_decoder_layer.cpp:811-849). */
QD_API qd_status qd_prefill(qd_engine *engine, uint32_t seq,
                            const uint32_t *tokens, uint32_t n,
                            float *last_logits, uint32_t *greedy_out,
                            float *top_logit);

/* One decode step for n_seq independent sequences at their own positions.
 * logits [n_seq][vocab] and greedy [n_seq] (both nullable); each sequence's
 * logits also stay on the device in its slot's row, for qd_read_logits.
 * The reference has no batched step (examples/qwen/README.md:431-432): its
 * semantics per sequence are qd_step's. */
QD_API qd_status qd_step_batch(qd_engine *engine, uint32_t n_seq,
                               const uint32_t *seq_ids, const uint32_t *tokens,
                               float *logits, uint32_t *greedy);

/* qd_step_batch for one group of 1..16 sequences that allocates nothing:
 * no hipMalloc, hipFree or other allocating call, on its first call or
 * later. Its scratch (activation rows, attention records, split-K partials,
 * arrival counters, LM-head partials: 2.25 MiB) is a static device array of
 * the library, one per GPU, whose address the engine looks up when it is
 * created. Results equal qd_step_batch's bit for bit. Calls on one GPU (two
 * engines, or two host threads) share that array: the library serialises
 * them per GPU with a host lock, so they cannot interleave on the device.
 * The call synchronises its stream before it returns (it is not capturable
 * into a HIP graph). More than 16 sequences: QD_ERROR_INVALID_ARGUMENT. No
 * counterpart in the reference; it is for callers that cannot allocate
 * (allocation-free serving loops, harnesses that forbid hipMalloc). */
QD_API qd_status qd_step_batch_noalloc(qd_engine *engine, uint32_t n_seq,
                                       const uint32_t *seq_ids,
                                       const uint32_t *tokens, float *logits,
                                       uint32_t *greedy);

/* Device-resident greedy generation: consumes first_token, then feeds each
 * argmax back on the device until max_tokens tokens were produced or eos
 * was produced; one host synchronisation at the end. Mirrors the resident
 * loop and embedding feedback of benchmarks/qwen_stateful_graph_kernel.cpp:358-390
 * driven by ResidentExecutor::launch (resident_executor.hpp:358-361).
 * out_tokens has room for max_tokens; all_logits (max_tokens * vocab floats)
 * may be NULL. eos = UINT32_MAX disables the EOS test. */
QD_API qd_status qd_generate_resident(qd_engine *engine, uint32_t seq,
                                      uint32_t first_token,
                                      uint32_t max_tokens, uint32_t eos,
                                      uint32_t *out_tokens,
                                      uint32_t *generated,
                                      uint32_t *stop_reason,
                                      float *all_logits);

/* Runs `tokens` greedy generate-mode steps from the slot's position with a
 * HIP event pair around every kernel launch on the engine stream, and
 * reports per-kernel totals (at most `capacity` entries). Advances the
 * position like qd_generate_resident; pair with qd_kv_reset. Plays the role
 * of the reference's stage profile (benchmarks/qwen_stateful_graph.cpp:547-602
 * byte model, qwen_stateful_graph_kernel.cpp:837-865 stage timing). */
QD_API qd_status qd_profile_kernels(qd_engine *engine, uint32_t seq,
                                    uint32_t first_token, uint32_t tokens,
                                    qd_kernel_stat *stats, uint32_t capacity,
                                    uint32_t *count);

/* Runs `steps` qd_step_batch steps of the n_seq listed slots (greedy
 * tokens fed back between steps, starting from `tokens`) with a HIP event
 * pair around every kernel launch, and reports per-kernel totals. Advances
 * each slot by `steps` positions. No reference counterpart: the reference
 * decodes one sequence at a time (examples/qwen/README.md:431-432). */
QD_API qd_status qd_profile_batch(qd_engine *engine, uint32_t n_seq,
                                  const uint32_t *seq_ids, const uint32_t *tokens,
                                  uint32_t steps, qd_kernel_stat *stats,
                                  uint32_t capacity, uint32_t *count);

/* Runs qd_prefill of the n tokens with a HIP event pair around every kernel
 * launch (the prompt GEMMs by projection) and reports per-kernel totals;
 * leaves the slot as qd_prefill does. The reference's Triton prompt path
 * (benchmarks/triton_mini_decoder_layer.cpp:817-834) has no profile. */
QD_API qd_status qd_profile_prefill(qd_engine *engine, uint32_t seq,
                                    const uint32_t *tokens, uint32_t n,
                                    qd_kernel_stat *stats, uint32_t capacity,
                                    uint32_t *count);

/* Runs qd_generate_resident's resident megakernel in its profiled form
 * (workgroup 0 stamps the end of every input wait and every stage) and
 * reports totals in microseconds as (wait, work) pairs for QKV, attention,
 * O projection, gate/up, down, LM head and argmax (14 entries), then three
 * sub-phases of the attention work (K/V staging, softmax math, emit) that
 * the attention "work" entry excludes (17 entries). Advances the position
 * like qd_generate_resident. The
 * counterpart of the reference's stage profile kernel
 * (benchmarks/qwen_stateful_graph_kernel.cpp:837-865). */
QD_API qd_status qd_profile_resident(qd_engine *engine, uint32_t seq,
                                     uint32_t first_token, uint32_t tokens,
                                     double *stage_us, uint32_t capacity,
                                     uint32_t *count);

/* Diagnostic timeline of the resident megakernel: runs like
 * qd_profile_resident and records, for token `trace_token` of the launch,
 * the 100 MHz timestamp at which every workgroup ended every stage:
 * timeline[workgroup][row][stage] with rows = layers + 1 (the last row holds
 * the LM head / argmax stages) and stages = the qd_profile_resident entries.
 * capacity is in entries; the dimensions are returned (also on a capacity
 * error). No counterpart in the reference; it locates the critical path
 * between the stages' producers and consumers. */
QD_API qd_status qd_trace_resident(qd_engine *engine, uint32_t seq,
                                   uint32_t first_token, uint32_t tokens,
                                   uint32_t trace_token, uint64_t *timeline,
                                   size_t capacity, uint32_t *workgroups,
                                   uint32_t *rows, uint32_t *stages);

/* Measured HBM bandwidth of `device`: the best of `iters` timed passes
 * (after one warm-up) of a streaming read and of a copy over `bytes`-byte
 * buffers (temporary, freed before returning), in bytes moved per second /
 * 1e9 (a copy moves 2 * bytes). The achievable peak the decode roofline is
 * also reported against. The reference reports achieved bandwidth against
 * its nominal peak (docs/stateful-graph.md:617-621). */
QD_API qd_status qd_probe_hbm(int32_t device, uint64_t bytes, uint32_t iters,
                              double *read_gbs, double *copy_gbs);

/* Timing of the last qd_generate_resident call. */
QD_API qd_status qd_last_timing(const qd_engine *engine, qd_timing *timing);

/* Waits for all work queued by the engine. */
QD_API qd_status qd_sync(qd_engine *engine);

/* ---- weight-bundle I/O (host only, no device needed) -----------------------
 * C-ABI form of load/write_decoder_layer_weights and
 * load/write_model_tail_weights (executor/qwen/weight_bundle.hpp:460-757):
 * same files, same validation, same diagnostics (qd_last_error).
 * shape6 = {keys, hidden, heads, kv_heads, head_dim, intermediate}; layer
 * tensors travel concatenated in bundle order (attention_norm, mlp_norm, q,
 * k, v, q_bias, k_bias, v_bias, out, gate, up, down). */
QD_API qd_status qd_bundle_write_layer(const char *manifest_path,
                                       const char *data_name,
                                       const uint32_t *shape6,
                                       float rope_theta,
                                       const float *tensors);
/* On success *count = floats written; capacity too small -> INVALID_ARGUMENT
 * with *count = floats needed. */
QD_API qd_status qd_bundle_read_layer(const char *manifest_path,
                                      uint32_t *shape6, float *rope_theta,
                                      float *tensors, size_t capacity,
                                      size_t *count);
QD_API qd_status qd_bundle_write_tail(const char *manifest_path,
                                      const char *data_name, uint32_t hidden,
                                      uint32_t vocab,
                                      const uint32_t *token_ids,
                                      size_t token_count,
                                      const float *token_embeddings,
                                      const float *final_norm,
                                      const float *lm_head);
/* Tensors concatenated: token_embeddings | final_norm | lm_head. */
QD_API qd_status qd_bundle_read_tail(const char *manifest_path,
                                     uint32_t *hidden, uint32_t *vocab,
                                     uint32_t *token_ids, size_t ids_capacity,
                                     size_t *token_count, float *tensors,
                                     size_t capacity, size_t *count);

#ifdef __cplusplus
}
#endif

#endif /* QD_QWEN_DECODE_H_ */
