// qd_run -- command-line runner of the decode engine that takes the command
// line of the reference's stack benchmark
// (benchmarks/triton_mini_decoder_layer.cpp:254-382, as built by
// tools/run_qwen_benchmark.py:115-149 and tools/run_qwen_e2e.py:667-693)
// and prints the reference's end-to-end stdout contract, so the reference's
// wrappers drive it by swapping the benchmark path
// (tools/run_qwen_e2e.py:28-35 regexes):
//
//   step N top_token=T logit=X vocab=V      one line per generated token
//   generated_token_ids=[t1,t2,...]
//   stop_reason=eos_token|max_new_tokens
//
// Flow, as in the reference benchmark: `count` timed prompt passes (after
// the warm-up passes) of the whole stack plus the model tail, reported as
// one summary line; then, with --max-new-tokens, greedy generation from
// the prompt's logits with every token fed back. The prompt pass is
// qd_prefill (dense MFMA GEMMs); generation is one qd_step per token, or
// with --sync-stack the reference's layer-by-layer decode
// (qd_embed_hidden, qd_layer_decode per layer with a synchronisation after
// each, qd_tail), or with --resident one device-resident launch.
// --e2e-check applies the reference's gate
// (benchmarks/triton_mini_decoder_layer.cpp:1369-1391): finite logits and the
// requested token count.
//
// Weights come from a reference bundle directory (--weights-dir, layer_<i>/
// and model_tail/) or from the seeded synthetic generator (--synthetic-seed).
#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "qd/qwen_decode.hpp"

namespace {

using Clock = std::chrono::steady_clock;

struct Options {
  std::string weights_dir;
  bool synthetic = false;
  uint64_t seed = 0;
  uint32_t layers = 0;
  uint32_t vocab = 151936;
  uint32_t keys = 0;
  uint32_t iterations = 20;  // the reference benchmark's default count
  bool iterations_set = false;
  uint32_t warmup = 0;
  bool warmup_set = false;
  bool no_warmup = false;
  uint32_t valid_keys = 0;
  bool valid_keys_set = false;
  std::vector<uint32_t> prompt;
  uint32_t max_new_tokens = 0;
  uint32_t eos = UINT32_MAX;
  bool no_model_tail = false;
  bool e2e_check = false;
  bool sync_stack = false;
  bool layer_sweep = false;
  bool trace_setup = false;
  bool trace_run = false;
  bool gpu_stage_profile = false;
  bool cpu_submit_profile = false;
  bool resident = false;
  int device = 0;
};

void usage(FILE *f) {
  std::fprintf(
      f,
      "usage: qd_run [count] (--weights-dir DIR --layers N | --synthetic-seed S [--layers N] "
      "[--vocab V])\n"
      "              [--valid-keys N] [--warmup-iterations N | --no-warmup] [--no-model-tail]\n"
      "              [--e2e-check] [--max-new-tokens N --prompt-token-ids a,b,c]\n"
      "              [--sync-stack | --resident] [--layer-sweep] [--trace-setup] [--trace-run]\n"
      "              [--gpu-stage-profile] [--cpu-submit-profile] [--keys CAPACITY]\n"
      "              [--eos-token-id T] [--device D]\n");
}

uint64_t parse_u64(const char *flag, const char *text) {
  char *end = nullptr;
  errno = 0;
  const unsigned long long v = std::strtoull(text, &end, 10);
  if (errno || !end || *end || !*text || text[0] == '-')
    throw std::invalid_argument(std::string(flag) + " requires a non-negative integer, got '" +
                                text + "'");
  return v;
}

uint32_t parse_u32(const char *flag, const char *text) {
  const uint64_t v = parse_u64(flag, text);
  if (v > UINT32_MAX) throw std::invalid_argument(std::string(flag) + " is out of range");
  return static_cast<uint32_t>(v);
}

std::vector<uint32_t> parse_ids(const char *text) {
  std::vector<uint32_t> ids;
  std::string cur;
  for (const char *p = text;; ++p) {
    if (*p == ',' || *p == '\0') {
      if (cur.empty()) throw std::invalid_argument("--prompt-token-ids has an empty entry");
      ids.push_back(parse_u32("--prompt-token-ids", cur.c_str()));
      cur.clear();
      if (*p == '\0') break;
    } else {
      cur += *p;
    }
  }
  return ids;
}

Options parse(int argc, char **argv) {
  Options o;
  for (int i = 1; i < argc; ++i) {
    const char *a = argv[i];
    auto value = [&]() -> const char * {
      if (i + 1 >= argc) throw std::invalid_argument(std::string(a) + " requires a value");
      return argv[++i];
    };
    if (!std::strcmp(a, "--help") || !std::strcmp(a, "-h")) {
      usage(stdout);
      std::exit(0);
    } else if (!std::strcmp(a, "--weights-dir")) {
      o.weights_dir = value();
    } else if (!std::strcmp(a, "--weights")) {
      throw std::invalid_argument(
          "--weights (one layer manifest without a model tail) is not supported; use "
          "--weights-dir with layer_<i>/ and model_tail/");
    } else if (!std::strcmp(a, "--synthetic-seed")) {
      o.synthetic = true;
      o.seed = parse_u64(a, value());
    } else if (!std::strcmp(a, "--layers")) {
      o.layers = parse_u32(a, value());
    } else if (!std::strcmp(a, "--vocab")) {
      o.vocab = parse_u32(a, value());
    } else if (!std::strcmp(a, "--keys")) {
      o.keys = parse_u32(a, value());
    } else if (!std::strcmp(a, "--valid-keys")) {
      o.valid_keys = parse_u32(a, value());
      o.valid_keys_set = true;
    } else if (!std::strcmp(a, "--warmup-iterations")) {
      o.warmup = parse_u32(a, value());
      o.warmup_set = true;
    } else if (!std::strcmp(a, "--no-warmup")) {
      o.no_warmup = true;
    } else if (!std::strcmp(a, "--no-model-tail")) {
      o.no_model_tail = true;
    } else if (!std::strcmp(a, "--e2e-check")) {
      o.e2e_check = true;
    } else if (!std::strcmp(a, "--prompt-token-ids") || !std::strcmp(a, "--token-ids")) {
      o.prompt = parse_ids(value());
    } else if (!std::strcmp(a, "--max-new-tokens")) {
      o.max_new_tokens = parse_u32(a, value());
    } else if (!std::strcmp(a, "--eos-token-id")) {
      o.eos = parse_u32(a, value());
    } else if (!std::strcmp(a, "--sync-stack")) {
      o.sync_stack = true;
    } else if (!std::strcmp(a, "--layer-sweep")) {
      o.layer_sweep = true;
    } else if (!std::strcmp(a, "--trace-setup")) {
      o.trace_setup = true;
    } else if (!std::strcmp(a, "--trace-run")) {
      o.trace_run = true;
    } else if (!std::strcmp(a, "--gpu-stage-profile")) {
      o.gpu_stage_profile = true;
    } else if (!std::strcmp(a, "--cpu-submit-profile")) {
      o.cpu_submit_profile = true;
    } else if (!std::strcmp(a, "--resident")) {
      o.resident = true;
    } else if (!std::strcmp(a, "--device")) {
      o.device = static_cast<int>(parse_u32(a, value()));
    } else if (a[0] != '-' && !o.iterations_set) {
      o.iterations = parse_u32("benchmark count", a);
      o.iterations_set = true;
    } else {
      throw std::invalid_argument(std::string("unknown option ") + a);
    }
  }
  // The reference's pairwise rules (benchmarks/triton_mini_decoder_layer.cpp:329-381).
  if (o.synthetic == !o.weights_dir.empty())
    throw std::invalid_argument("exactly one of --weights-dir and --synthetic-seed is required");
  if (!o.weights_dir.empty() && o.layers == 0) throw std::invalid_argument("--weights-dir requires --layers");
  if (o.synthetic && o.layers == 0) o.layers = 24;
  if (o.e2e_check && o.no_model_tail) throw std::invalid_argument("--e2e-check requires model tail");
  if (o.max_new_tokens && o.no_model_tail)
    throw std::invalid_argument("--max-new-tokens requires model tail");
  if (!o.prompt.empty() && o.no_model_tail)
    throw std::invalid_argument("--prompt-token-ids requires model tail");
  if (o.max_new_tokens && o.layer_sweep)
    throw std::invalid_argument("--max-new-tokens and --layer-sweep are mutually exclusive");
  if (o.gpu_stage_profile && o.sync_stack)
    throw std::invalid_argument("--gpu-stage-profile and --sync-stack are mutually exclusive");
  if (o.warmup_set && o.no_warmup)
    throw std::invalid_argument("--warmup-iterations and --no-warmup are mutually exclusive");
  if (o.sync_stack && o.resident)
    throw std::invalid_argument("--sync-stack and --resident are mutually exclusive");
  if (o.prompt.empty() && !o.no_model_tail) throw std::invalid_argument("--prompt-token-ids is required");
  if (o.no_model_tail) {
    // The stack alone runs on token 0's embedding at every prompt position.
    o.prompt.assign(o.valid_keys_set ? std::max<uint32_t>(o.valid_keys, 1) : 1, 0u);
  }
  if (o.valid_keys_set && o.valid_keys != o.prompt.size())
    throw std::invalid_argument("valid key count must match prompt token count");
  if (!o.warmup_set) o.warmup = o.no_warmup ? 0 : std::min<uint32_t>(o.iterations, 5);
  const uint64_t needed = o.prompt.size() + (o.max_new_tokens ? o.max_new_tokens - 1 : 0);
  if (o.keys != 0 && o.keys < needed)
    throw std::invalid_argument("--keys must cover the prompt and generated-token feedback");
  return o;
}

double ms_since(Clock::time_point t0) {
  return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

struct Spread {
  double median = 0, min = 0, max = 0, mean = 0;
};
Spread spread(std::vector<double> v) {
  Spread s;
  if (v.empty()) return s;
  std::sort(v.begin(), v.end());
  s.min = v.front();
  s.max = v.back();
  s.median = v.size() % 2 ? v[v.size() / 2] : 0.5 * (v[v.size() / 2 - 1] + v[v.size() / 2]);
  for (double x : v) s.mean += x;
  s.mean /= double(v.size());
  return s;
}

// The reference's sweep of stack depths (1, 2, 4, ... and the full count).
std::vector<uint32_t> sweep_counts(uint32_t layers) {
  std::vector<uint32_t> c;
  for (uint32_t k = 1; k < layers; k *= 2) c.push_back(k);
  c.push_back(layers);
  return c;
}

// Host top-1 (greater wins, the lower index on ties) and the non-finite count.
void top1(const std::vector<float> &logits, uint32_t *token, float *value, size_t *non_finite) {
  *token = UINT32_MAX;
  *value = -INFINITY;
  *non_finite = 0;
  for (size_t i = 0; i < logits.size(); ++i) {
    const float v = logits[i];
    if (!std::isfinite(v)) {
      ++*non_finite;
      continue;
    }
    if (*token == UINT32_MAX || v > *value) {
      *value = v;
      *token = static_cast<uint32_t>(i);
    }
  }
}

// An unsigned integer field of a bundle manifest (a small JSON object),
// found by its key; 0 when the file or the key is missing. Only sizes the
// engine: qd_load_bundle validates the whole bundle afterwards.
uint64_t manifest_field(const std::string &path, const char *key) {
  FILE *f = std::fopen(path.c_str(), "rb");
  if (!f) return 0;
  std::string text;
  char buf[4096];
  size_t n;
  while (text.size() < (1u << 20) && (n = std::fread(buf, 1, sizeof(buf), f)) > 0) text.append(buf, n);
  std::fclose(f);
  const std::string quoted = std::string("\"") + key + "\"";
  const size_t at = text.find(quoted);
  if (at == std::string::npos) return 0;
  size_t i = text.find(':', at + quoted.size());
  if (i == std::string::npos) return 0;
  ++i;
  while (i < text.size() && (text[i] == ' ' || text[i] == '\t' || text[i] == '\n' || text[i] == '\r')) ++i;
  uint64_t v = 0;
  bool any = false;
  while (i < text.size() && text[i] >= '0' && text[i] <= '9' && v < (uint64_t(1) << 40)) {
    v = v * 10 + uint64_t(text[i++] - '0');
    any = true;
  }
  return any ? v : 0;
}

// Engine capacity: --keys, else the bundle's key count, else what the run
// needs (plus room for the profiles' extra tokens).
uint32_t capacity(const Options &o) {
  uint64_t need = o.prompt.size() + o.max_new_tokens + 8;
  if (o.keys) return o.keys;
  if (!o.weights_dir.empty())
    need = std::max<uint64_t>(need, manifest_field(o.weights_dir + "/layer_0/weights.json", "keys"));
  return static_cast<uint32_t>(std::min<uint64_t>(need, UINT32_MAX));
}

// Vocabulary: the bundle's model tail, else --vocab.
uint32_t vocabulary(const Options &o) {
  if (!o.weights_dir.empty()) {
    const uint64_t v = manifest_field(o.weights_dir + "/model_tail/weights.json", "vocab");
    if (v > 0 && v <= UINT32_MAX) return static_cast<uint32_t>(v);
  }
  return o.vocab;
}

int run(const Options &o) {
  const auto t_setup = Clock::now();
  qd_config cfg = qd::qwen25_05b_config(capacity(o), 1);
  cfg.layers = o.layers;
  cfg.vocab = vocabulary(o);
  cfg.device = o.device;
  qd::Engine engine(cfg);
  const double create_ms = ms_since(t_setup);
  const auto t_load = Clock::now();
  if (o.synthetic) {
    engine.load_synthetic(o.seed);
  } else {
    engine.load_bundle(o.weights_dir);
  }
  const double load_ms = ms_since(t_load);
  if (o.trace_setup)
    std::fprintf(stderr, "qd_run trace setup engine_create_ms=%.3f weight_load_ms=%.3f device_mib=%.1f\n",
                 create_ms, load_ms, double(engine.device_bytes()) / (1 << 20));
  const qd_config got = engine.config();
  const uint32_t vocab = got.vocab, layers = got.layers;
  const uint32_t prompt_len = static_cast<uint32_t>(o.prompt.size());
  for (uint32_t t : o.prompt)
    if (t >= vocab) throw std::invalid_argument("prompt token id " + std::to_string(t) +
                                                " is outside the vocabulary");

  // Timed prompt passes: the whole stack plus the tail (qd_prefill), or with
  // --no-model-tail the stack alone on the last prompt position.
  std::vector<float> logits;
  float top_logit = 0.f;
  uint32_t token = UINT32_MAX;
  auto prompt_pass = [&] {
    engine.kv_reset(0, 0);
    if (o.no_model_tail) {
      if (prompt_len > 1)
        engine.prefill(0, std::vector<uint32_t>(o.prompt.begin(), o.prompt.end() - 1));
      qd::check(qd_embed_hidden(engine.get(), 0, o.prompt.back()));
      qd::check(qd_layer_decode(engine.get(), 0, 0, layers, prompt_len));
      engine.sync();
    } else {
      token = engine.prefill(0, o.prompt, &logits, &top_logit);
    }
  };
  for (uint32_t i = 0; i < o.warmup; ++i) prompt_pass();
  std::vector<double> pass_ms;
  for (uint32_t i = 0; i < o.iterations; ++i) {
    const auto t0 = Clock::now();
    prompt_pass();
    pass_ms.push_back(ms_since(t0));
    if (o.trace_run) std::fprintf(stderr, "qd_run trace run prompt_pass=%u ms=%.3f\n", i, pass_ms.back());
  }
  if (o.iterations == 0) prompt_pass();
  const Spread ps = spread(pass_ms);
  std::printf("qd_run benchmark prompt_tokens=%u layers=%u iterations=%u warmup=%u median_ms=%.3f "
              "min_ms=%.3f max_ms=%.3f mean_ms=%.3f model_tail=%s\n",
              prompt_len, layers, o.iterations, o.warmup, ps.median, ps.min, ps.max, ps.mean,
              o.no_model_tail ? "disabled" : "enabled");

  if (o.layer_sweep) {
    // Decode of the last prompt position through the first k layers.
    for (uint32_t k : sweep_counts(layers)) {
      std::vector<double> us;
      for (uint32_t i = 0; i < std::max<uint32_t>(o.iterations, 1); ++i) {
        const auto t0 = Clock::now();
        qd::check(qd_embed_hidden(engine.get(), 0, o.prompt.back()));
        qd::check(qd_layer_decode(engine.get(), 0, 0, k, prompt_len));
        engine.sync();
        us.push_back(ms_since(t0) * 1000.0);
      }
      const Spread s = spread(us);
      std::printf("qd_run layer_sweep layers=%u valid_keys=%u median_us=%.3f min_us=%.3f max_us=%.3f\n",
                  k, prompt_len, s.median, s.min, s.max);
    }
    // Leave the slot after the prompt again.
    prompt_pass();
  }

  if (o.cpu_submit_profile) {
    // Host cost of submitting one layer-by-layer decode (no waiting).
    const auto t0 = Clock::now();
    qd::check(qd_embed_hidden(engine.get(), 0, o.prompt.back()));
    qd::check(qd_layer_decode(engine.get(), 0, 0, layers, prompt_len));
    const double submit_us = ms_since(t0) * 1000.0;
    engine.sync();
    std::printf("qd_run cpu_submit layers=%u submit_us=%.3f per_layer_us=%.3f\n", layers, submit_us,
                submit_us / layers);
    prompt_pass();
  }

  std::vector<uint32_t> generated;
  bool eos_hit = false;
  size_t bad = 0;
  const auto t_gen = Clock::now();
  auto emit = [&](uint32_t step, const std::vector<float> &row) {
    uint32_t tok;
    float top;
    size_t non_finite;
    top1(row, &tok, &top, &non_finite);
    bad += non_finite;
    std::printf("step %u top_token=%u logit=%g vocab=%u\n", step, tok, top, vocab);
  };
  if (o.max_new_tokens) {
    emit(1, logits);
    generated.push_back(token);
    eos_hit = token == o.eos;
    if (!eos_hit && o.max_new_tokens > 1) {
      if (o.resident) {
        qd::ResidentExecutor exec(engine);
        std::vector<float> all;
        const auto r = exec.launch(token, o.max_new_tokens - 1, o.eos, &all);
        for (size_t i = 0; i < r.tokens.size(); ++i) {
          std::vector<float> row(all.begin() + i * vocab, all.begin() + (i + 1) * vocab);
          emit(static_cast<uint32_t>(i + 2), row);
          generated.push_back(r.tokens[i]);
        }
        eos_hit = r.stop_reason == QD_STOP_EOS_TOKEN;
      } else {
        std::vector<qd::DecoderLayer> stack;
        for (uint32_t l = 0; l < layers; ++l) stack.emplace_back(engine, l);
        qd::ModelTail tail(engine);
        for (uint32_t s = 2; s <= o.max_new_tokens; ++s) {
          const auto t0 = Clock::now();
          if (o.sync_stack) {
            // The reference driver's loop: embedding, layer to layer on the
            // device with a synchronisation per layer, then the tail.
            const uint32_t position = prompt_len + s - 2;
            stack.front().embed_token(position, token);
            for (uint32_t l = 0; l < layers; ++l) {
              if (l + 1 < layers)
                stack[l].decode_to_hidden_state(position + 1, stack[l + 1], position);
              else
                stack[l].decode_to_buffer(position + 1, tail.hidden_buffer());
              stack[l].synchronize();
            }
            tail.run();
            tail.copy_logits(logits);
            token = tail.top_token();
          } else {
            token = engine.step(0, token, &logits, &top_logit);
          }
          if (o.trace_run)
            std::fprintf(stderr, "qd_run trace run token=%u ms=%.3f\n", s, ms_since(t0));
          emit(s, logits);
          generated.push_back(token);
          if (token == o.eos) {
            eos_hit = true;
            break;
          }
        }
      }
    }
  }
  engine.sync();
  const double gen_ms = ms_since(t_gen);

  if (o.gpu_stage_profile) {
    // Per-kernel HIP-event times of stream-ordered decode steps from the
    // prompt (the slot is restored to the prompt afterwards).
    const uint32_t tokens = std::min<uint32_t>(4, got.capacity - prompt_len);
    if (tokens) {
      engine.kv_reset(0, prompt_len);
      std::vector<qd_kernel_stat> st(32);
      uint32_t n = 0;
      qd::check(qd_profile_kernels(engine.get(), 0, o.prompt.back(), tokens, st.data(), 32, &n));
      for (uint32_t i = 0; i < n; ++i)
        std::printf("qd_run gpu_stage kernel=%s launches=%u avg_us=%.3f avg_gbs=%.1f\n", st[i].name,
                    st[i].launches, st[i].total_us / st[i].launches,
                    st[i].bytes / (st[i].total_us * 1e-6) / 1e9);
    }
  }

  if (o.max_new_tokens) {
    std::printf("generated_token_ids=[");
    for (size_t i = 0; i < generated.size(); ++i) std::printf("%s%u", i ? "," : "", generated[i]);
    std::printf("]\n");
    std::printf("stop_reason=%s\n", eos_hit ? "eos_token" : "max_new_tokens");
  }
  std::printf("qd_run summary prompt_tokens=%u generated_tokens=%zu generation_ms=%.3f path=%s\n",
              prompt_len, generated.size(), gen_ms,
              o.resident ? "resident" : (o.sync_stack ? "layer-by-layer" : "step"));
  std::fflush(stdout);
  if (o.e2e_check) {
    if (bad) {
      std::fprintf(stderr, "qd_run e2e check failed: %zu non-finite logits\n", bad);
      return 1;
    }
    if (o.max_new_tokens && !eos_hit && generated.size() != o.max_new_tokens) {
      std::fprintf(stderr, "qd_run e2e check failed: generated token count mismatch\n");
      return 1;
    }
  }
  return 0;
}

}  // namespace

int main(int argc, char **argv) {
  Options o;
  try {
    o = parse(argc, argv);
  } catch (const std::exception &e) {
    std::fprintf(stderr, "qd_run: %s\n", e.what());
    usage(stderr);
    return 2;
  }
  try {
    return run(o);
  } catch (const qd::Error &e) {
    std::fprintf(stderr, "qd_run: %s\n", e.what());
    return 3;
  } catch (const std::exception &e) {
    std::fprintf(stderr, "qd_run: %s\n", e.what());
    return 2;
  }
}
