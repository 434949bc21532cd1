// qd_run -- command-line runner of the decode engine with the reference's
// end-to-end stdout contract, so wrappers that parse the reference runners
// (tools/run_qwen_e2e.py:28-35 regexes; lines printed by
// examples/iree/qwen/qwen_decode1_e2e.cpp:650,1068-1075) read it unchanged:
//
//   step N top_token=T logit=X vocab=V      one line per generated token
//   generated_token_ids=[t1,t2,...]
//   stop_reason=eos_token|max_new_tokens
//
// Weights come from a reference bundle directory (--weights-dir, layer_<i>/
// and model_tail/) or from the seeded synthetic generator (--synthetic-seed).
// The prompt is prefilled, the first generated token comes from the last
// prompt position's logits, and every generated token is fed back. With
// --resident the tokens after the first are produced by one device-resident
// launch; otherwise one host call per token. --e2e-check applies the
// reference's end-to-end gate (benchmarks/triton_mini_decoder_layer.cpp:
// 1369-1391): finite logits and the requested token count.
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

struct Options {
  std::string weights_dir;
  bool synthetic = false;
  uint64_t seed = 0;
  uint32_t layers = 24;
  uint32_t vocab = 151936;
  uint32_t keys = 0;
  std::vector<uint32_t> prompt;
  uint32_t max_new_tokens = 16;
  uint32_t eos = UINT32_MAX;
  bool resident = false;
  bool e2e_check = false;
  int device = 0;
};

void usage(FILE *f) {
  std::fprintf(f,
               "usage: qd_run (--weights-dir DIR --layers N | --synthetic-seed S [--layers N] "
               "[--vocab V])\n"
               "              --prompt-token-ids a,b,c [--max-new-tokens N] [--eos-token-id T]\n"
               "              [--keys CAPACITY] [--resident] [--e2e-check] [--device D]\n");
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
  bool layers_set = false;
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
    } else if (!std::strcmp(a, "--synthetic-seed")) {
      o.synthetic = true;
      o.seed = parse_u64(a, value());
    } else if (!std::strcmp(a, "--layers")) {
      o.layers = parse_u32(a, value());
      layers_set = true;
    } else if (!std::strcmp(a, "--vocab")) {
      o.vocab = parse_u32(a, value());
    } else if (!std::strcmp(a, "--keys")) {
      o.keys = parse_u32(a, value());
    } else if (!std::strcmp(a, "--prompt-token-ids") || !std::strcmp(a, "--token-ids")) {
      o.prompt = parse_ids(value());
    } else if (!std::strcmp(a, "--max-new-tokens")) {
      o.max_new_tokens = parse_u32(a, value());
    } else if (!std::strcmp(a, "--eos-token-id")) {
      o.eos = parse_u32(a, value());
    } else if (!std::strcmp(a, "--resident")) {
      o.resident = true;
    } else if (!std::strcmp(a, "--e2e-check")) {
      o.e2e_check = true;
    } else if (!std::strcmp(a, "--device")) {
      o.device = static_cast<int>(parse_u32(a, value()));
    } else {
      throw std::invalid_argument(std::string("unknown option ") + a);
    }
  }
  if (o.synthetic == !o.weights_dir.empty())
    throw std::invalid_argument("exactly one of --weights-dir and --synthetic-seed is required");
  if (!o.weights_dir.empty() && !layers_set)
    throw std::invalid_argument("--weights-dir requires --layers");
  if (o.prompt.empty()) throw std::invalid_argument("--prompt-token-ids is required");
  if (o.max_new_tokens == 0) throw std::invalid_argument("--max-new-tokens must be positive");
  if (o.layers == 0) throw std::invalid_argument("--layers must be positive");
  const uint64_t needed = o.prompt.size() + o.max_new_tokens;
  if (o.keys == 0) o.keys = static_cast<uint32_t>(needed);
  if (o.keys < needed - 1)
    throw std::invalid_argument("--keys must cover the prompt and generated-token feedback");
  return o;
}

// Host top-1 with the engine's tie rule; counts non-finite logits.
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

int run(const Options &o) {
  qd_config cfg = qd::qwen25_05b_config(o.keys, 1);
  cfg.layers = o.layers;
  cfg.vocab = o.vocab;
  cfg.device = o.device;
  qd::Engine engine(cfg);
  if (o.synthetic) {
    engine.load_synthetic(o.seed);
  } else {
    engine.load_bundle(o.weights_dir);
  }
  const uint32_t vocab = engine.config().vocab;
  for (uint32_t t : o.prompt)
    if (t >= vocab) throw std::invalid_argument("prompt token id " + std::to_string(t) +
                                                " is outside the vocabulary");

  const auto start = std::chrono::steady_clock::now();
  std::vector<uint32_t> generated;
  std::vector<float> logits;
  bool eos_hit = false;
  size_t bad = 0;
  auto emit = [&](uint32_t step, const std::vector<float> &row) {
    uint32_t tok;
    float top;
    size_t non_finite;
    top1(row, &tok, &top, &non_finite);
    bad += non_finite;
    std::printf("step %u top_token=%u logit=%g vocab=%u\n", step, tok, top, vocab);
  };

  float top_logit = 0.f;
  uint32_t token = engine.prefill(0, o.prompt, &logits, &top_logit);
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
      for (uint32_t s = 2; s <= o.max_new_tokens; ++s) {
        token = engine.step(0, token, &logits, &top_logit);
        emit(s, logits);
        generated.push_back(token);
        if (token == o.eos) {
          eos_hit = true;
          break;
        }
      }
    }
  }
  engine.sync();
  const double ms =
      std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start).count();

  std::printf("generated_token_ids=[");
  for (size_t i = 0; i < generated.size(); ++i) std::printf("%s%u", i ? "," : "", generated[i]);
  std::printf("]\n");
  std::printf("stop_reason=%s\n", eos_hit ? "eos_token" : "max_new_tokens");
  std::printf("qd_run summary prompt_tokens=%zu generated_tokens=%zu elapsed_ms=%.3f path=%s\n",
              o.prompt.size(), generated.size(), ms, o.resident ? "resident" : "step");
  std::fflush(stdout);
  if (o.e2e_check) {
    if (bad) {
      std::fprintf(stderr, "qd_run e2e check failed: %zu non-finite logits\n", bad);
      return 1;
    }
    if (!eos_hit && generated.size() != o.max_new_tokens) {
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
