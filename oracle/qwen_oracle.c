/*
 * CPU oracle for the Qwen2 FP32 decode step -- TEST INFRASTRUCTURE ONLY.
 * The header lists the reference file:line each function restates.
 * Built with -ffp-contract=off so FP32 products and sums round exactly where
 * the written expression says they do.
 */
#include "qwen_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

struct qo_layer_tensors {
  float *t[QO_LAYER_TENSORS];
};

struct qo_model {
  qo_shape shape;
  int tied;
  struct qo_layer_tensors *layers;
  float *embed;
  float *final_norm;
  float *lm_head; /* == embed when tied */
};

struct qo_cache {
  const qo_model *model;
  uint32_t capacity;
  float **k;
  float **v;
  float *cos_table;
  float *sin_table;
  float *final_normed;
};

int qo_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ---- counter-based generator -------------------------------------------
 * splitmix64 finaliser over a per-(seed, stream) key; the engine carries an
 * independent implementation of the same specification. */
static uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t qo_rng_u64(uint64_t seed, uint64_t stream, uint64_t counter) {
  const uint64_t key = mix64(seed * 0x9E3779B97F4A7C15ull +
                             stream * 0xC2B2AE3D27D4EB4Full +
                             0x165667B19E3779F9ull);
  return mix64(key + counter * 0x9E3779B97F4A7C15ull);
}

/* Box-Muller (cosine branch) on two 53-bit uniforms, u1 in (0, 1]. */
double qo_rng_normal(uint64_t seed, uint64_t stream, uint64_t index) {
  const uint64_t a = qo_rng_u64(seed, stream, 2u * index);
  const uint64_t b = qo_rng_u64(seed, stream, 2u * index + 1u);
  const double u1 = (double)((a >> 11) + 1u) * 0x1.0p-53;
  const double u2 = (double)(b >> 11) * 0x1.0p-53;
  const double two_pi = 6.283185307179586476925286766559;
  return sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
}

void qo_fill_normal(float *out, size_t count, uint64_t seed, uint64_t stream,
                    float mean, float stddev) {
  const long long n = (long long)count;
#pragma omp parallel for schedule(static)
  for (long long i = 0; i < n; ++i) {
    out[i] = (float)((double)mean +
                     (double)stddev * qo_rng_normal(seed, stream, (uint64_t)i));
  }
}

void qo_fill_tokens(uint32_t *out, size_t count, uint64_t seed,
                    uint64_t stream, uint32_t vocab) {
  for (size_t i = 0; i < count; ++i) {
    const uint64_t r = qo_rng_u64(seed, stream, i) >> 32;
    out[i] = (uint32_t)((r * (uint64_t)vocab) >> 32);
  }
}

uint64_t qo_layer_stream(uint32_t layer, uint32_t kind) {
  return ((uint64_t)(layer + 1u) << 8) | kind;
}

uint64_t qo_tail_stream(uint32_t kind) {
  return 0x7fff00ull | (uint64_t)(kind & 0xffu);
}

/* ---- storage ------------------------------------------------------------ */
static size_t layer_tensor_count(const qo_shape *s, uint32_t kind) {
  const size_t h = s->hidden, q = (size_t)s->heads * s->head_dim,
               kv = (size_t)s->kv_heads * s->head_dim, i = s->intermediate;
  switch (kind) {
  case QO_ATTN_NORM:
  case QO_MLP_NORM:
    return h;
  case QO_Q_W:
    return q * h;
  case QO_K_W:
  case QO_V_W:
    return kv * h;
  case QO_Q_B:
    return q;
  case QO_K_B:
  case QO_V_B:
    return kv;
  case QO_O_W:
    return h * q;
  case QO_GATE_W:
  case QO_UP_W:
    return i * h;
  case QO_DOWN_W:
    return h * i;
  }
  return 0;
}

qo_model *qo_model_create(const qo_shape *shape, int tied) {
  if (!shape || shape->hidden == 0 || shape->heads == 0 ||
      shape->kv_heads == 0 || shape->head_dim == 0 ||
      shape->head_dim % 2 != 0 || shape->heads % shape->kv_heads != 0 ||
      shape->intermediate == 0 || shape->vocab == 0 || shape->layers == 0) {
    return NULL;
  }
  qo_model *m = (qo_model *)calloc(1, sizeof(qo_model));
  if (!m) {
    return NULL;
  }
  m->shape = *shape;
  m->tied = tied != 0;
  m->layers = (struct qo_layer_tensors *)calloc(
      shape->layers, sizeof(struct qo_layer_tensors));
  int ok = m->layers != NULL;
  for (uint32_t l = 0; ok && l < shape->layers; ++l) {
    for (uint32_t t = 0; ok && t < QO_LAYER_TENSORS; ++t) {
      m->layers[l].t[t] =
          (float *)calloc(layer_tensor_count(shape, t), sizeof(float));
      ok = m->layers[l].t[t] != NULL;
    }
  }
  const size_t table = (size_t)shape->vocab * shape->hidden;
  if (ok) {
    m->embed = (float *)malloc(table * sizeof(float));
    m->final_norm = (float *)calloc(shape->hidden, sizeof(float));
    m->lm_head = m->tied ? m->embed : (float *)malloc(table * sizeof(float));
    ok = m->embed && m->final_norm && m->lm_head;
  }
  if (!ok) {
    qo_model_destroy(m);
    return NULL;
  }
  return m;
}

void qo_model_destroy(qo_model *m) {
  if (!m) {
    return;
  }
  if (m->layers) {
    for (uint32_t l = 0; l < m->shape.layers; ++l) {
      for (uint32_t t = 0; t < QO_LAYER_TENSORS; ++t) {
        free(m->layers[l].t[t]);
      }
    }
    free(m->layers);
  }
  if (!m->tied) {
    free(m->lm_head);
  }
  free(m->embed);
  free(m->final_norm);
  free(m);
}

float *qo_model_tensor(qo_model *m, uint32_t layer, uint32_t kind,
                       size_t *count) {
  if (!m) {
    return NULL;
  }
  const size_t table = (size_t)m->shape.vocab * m->shape.hidden;
  float *p = NULL;
  size_t n = 0;
  if (kind == QO_EMBED) {
    p = m->embed;
    n = table;
  } else if (kind == QO_FINAL_NORM) {
    p = m->final_norm;
    n = m->shape.hidden;
  } else if (kind == QO_LM_HEAD) {
    p = m->lm_head;
    n = table;
  } else if (kind < QO_LAYER_TENSORS && layer < m->shape.layers) {
    p = m->layers[layer].t[kind];
    n = layer_tensor_count(&m->shape, kind);
  }
  if (count) {
    *count = n;
  }
  return p;
}

static int is_norm(uint32_t kind) {
  return kind == QO_ATTN_NORM || kind == QO_MLP_NORM;
}

static int is_bias(uint32_t kind) {
  return kind == QO_Q_B || kind == QO_K_B || kind == QO_V_B;
}

void qo_model_fill_synthetic(qo_model *m, uint64_t seed, float weight_std,
                             float bias_std, float norm_gain) {
  for (uint32_t l = 0; l < m->shape.layers; ++l) {
    for (uint32_t t = 0; t < QO_LAYER_TENSORS; ++t) {
      const size_t n = layer_tensor_count(&m->shape, t);
      float *p = m->layers[l].t[t];
      if (is_norm(t)) {
        for (size_t i = 0; i < n; ++i) {
          p[i] = norm_gain;
        }
      } else {
        qo_fill_normal(p, n, seed, qo_layer_stream(l, t), 0.0f,
                       is_bias(t) ? bias_std : weight_std);
      }
    }
  }
  const size_t table = (size_t)m->shape.vocab * m->shape.hidden;
  qo_fill_normal(m->embed, table, seed, qo_tail_stream(QO_EMBED), 0.0f,
                 weight_std);
  for (uint32_t i = 0; i < m->shape.hidden; ++i) {
    m->final_norm[i] = norm_gain;
  }
  if (!m->tied) {
    qo_fill_normal(m->lm_head, table, seed, qo_tail_stream(QO_LM_HEAD), 0.0f,
                   weight_std);
  }
}

qo_cache *qo_cache_create(const qo_model *m, uint32_t capacity) {
  if (!m || capacity == 0) {
    return NULL;
  }
  const qo_shape *s = &m->shape;
  qo_cache *c = (qo_cache *)calloc(1, sizeof(qo_cache));
  if (!c) {
    return NULL;
  }
  c->model = m;
  c->capacity = capacity;
  c->k = (float **)calloc(s->layers, sizeof(float *));
  c->v = (float **)calloc(s->layers, sizeof(float *));
  const size_t per_layer = (size_t)capacity * s->kv_heads * s->head_dim;
  int ok = c->k && c->v;
  for (uint32_t l = 0; ok && l < s->layers; ++l) {
    c->k[l] = (float *)calloc(per_layer, sizeof(float));
    c->v[l] = (float *)calloc(per_layer, sizeof(float));
    ok = c->k[l] && c->v[l];
  }
  const size_t table = (size_t)capacity * (s->head_dim / 2u);
  if (ok) {
    c->cos_table = (float *)malloc(table * sizeof(float));
    c->sin_table = (float *)malloc(table * sizeof(float));
    c->final_normed = (float *)calloc(s->hidden, sizeof(float));
    ok = c->cos_table && c->sin_table && c->final_normed;
  }
  if (!ok) {
    qo_cache_destroy(c);
    return NULL;
  }
  qo_rope_tables(s->rope_theta, s->head_dim, capacity, c->cos_table,
                 c->sin_table);
  return c;
}

void qo_cache_destroy(qo_cache *c) {
  if (!c) {
    return;
  }
  if (c->k || c->v) {
    for (uint32_t l = 0; l < c->model->shape.layers; ++l) {
      if (c->k) {
        free(c->k[l]);
      }
      if (c->v) {
        free(c->v[l]);
      }
    }
  }
  free(c->k);
  free(c->v);
  free(c->cos_table);
  free(c->sin_table);
  free(c->final_normed);
  free(c);
}

float *qo_cache_layer(qo_cache *c, uint32_t layer, int value) {
  if (!c || layer >= c->model->shape.layers) {
    return NULL;
  }
  return value ? c->v[layer] : c->k[layer];
}

const float *qo_last_final_normed(const qo_cache *c) {
  return c ? c->final_normed : NULL;
}

/* ---- primitives ---------------------------------------------------------- */

/* y = x * rsqrt(mean(x^2) + eps) * w; the mean accumulates in double. */
void qo_rmsnorm(const float *x, const float *weight, uint32_t n, float eps,
                float *out) {
  double sum = 0.0;
  for (uint32_t i = 0; i < n; ++i) {
    sum += (double)x[i] * (double)x[i];
  }
  const double inv = 1.0 / sqrt(sum / (double)n + (double)eps);
  for (uint32_t i = 0; i < n; ++i) {
    out[i] = (float)((double)x[i] * inv) * weight[i];
  }
}

/* y[r] = W[r,:] . x (+ bias[r]), row-major W [rows, cols]. */
void qo_gemv(const float *weight, const float *x, const float *bias,
             uint32_t rows, uint32_t cols, float *y) {
  const long long n = rows;
#pragma omp parallel for schedule(static)
  for (long long r = 0; r < n; ++r) {
    const float *w = weight + (size_t)r * cols;
    double acc = 0.0;
#pragma omp simd reduction(+ : acc)
    for (uint32_t c = 0; c < cols; ++c) {
      acc += (double)w[c] * (double)x[c];
    }
    if (bias) {
      acc += (double)bias[r];
    }
    y[r] = (float)acc;
  }
}

/* inv_freq_i = 1 / theta^(2i/d) and angle = p * inv_freq_i, both in FP32, as
 * the Hugging Face rotary embedding computes them; cos/sin of that FP32
 * angle, rounded to FP32. Tables are [positions, d/2]. */
void qo_rope_tables(float theta, uint32_t head_dim, uint32_t positions,
                    float *cos_table, float *sin_table) {
  const uint32_t half = head_dim / 2u;
  for (uint32_t i = 0; i < half; ++i) {
    const float exponent = (float)(2u * i) / (float)head_dim;
    const float inv_freq = 1.0f / powf(theta, exponent);
    for (uint32_t p = 0; p < positions; ++p) {
      const float angle = (float)p * inv_freq;
      cos_table[(size_t)p * half + i] = (float)cos((double)angle);
      sin_table[(size_t)p * half + i] = (float)sin((double)angle);
    }
  }
}

/* rotate_half: (a, b) -> (a*c - b*s, b*c + a*s) for a = x[i], b = x[i+d/2]. */
void qo_rope_apply(float *vec, uint32_t n_heads, uint32_t head_dim,
                   const float *cos_row, const float *sin_row) {
  const uint32_t half = head_dim / 2u;
  for (uint32_t h = 0; h < n_heads; ++h) {
    float *x = vec + (size_t)h * head_dim;
    for (uint32_t i = 0; i < half; ++i) {
      const float a = x[i], b = x[i + half];
      const float c = cos_row[i], s = sin_row[i];
      const float first = a * c + (-b) * s;
      const float second = b * c + a * s;
      x[i] = first;
      x[i + half] = second;
    }
  }
}

/* Softmax attention of each query head over cache rows 0..length-1. */
void qo_attention(const float *q, const float *k_cache, const float *v_cache,
                  uint32_t heads, uint32_t kv_heads, uint32_t head_dim,
                  uint32_t length, float *out) {
  const uint32_t group = heads / kv_heads;
  const uint32_t kv_dim = kv_heads * head_dim;
  const double scale = 1.0 / sqrt((double)head_dim);
  double *scores = (double *)malloc((size_t)(length ? length : 1) * heads *
                                    sizeof(double));
  if (!scores) {
    abort();
  }
#pragma omp parallel for schedule(static)
  for (int h = 0; h < (int)heads; ++h) {
    const uint32_t kvh = (uint32_t)h / group;
    const float *qh = q + (size_t)h * head_dim;
    double *s = scores + (size_t)h * length;
    double maximum = -INFINITY;
    for (uint32_t j = 0; j < length; ++j) {
      const float *kj = k_cache + (size_t)j * kv_dim + (size_t)kvh * head_dim;
      double acc = 0.0;
      for (uint32_t d = 0; d < head_dim; ++d) {
        acc += (double)qh[d] * (double)kj[d];
      }
      s[j] = acc * scale;
      if (s[j] > maximum) {
        maximum = s[j];
      }
    }
    double denom = 0.0;
    for (uint32_t j = 0; j < length; ++j) {
      s[j] = exp(s[j] - maximum);
      denom += s[j];
    }
    for (uint32_t d = 0; d < head_dim; ++d) {
      double acc = 0.0;
      for (uint32_t j = 0; j < length; ++j) {
        acc += s[j] *
               (double)v_cache[(size_t)j * kv_dim + (size_t)kvh * head_dim + d];
      }
      out[(size_t)h * head_dim + d] = (float)(acc / denom);
    }
  }
  free(scores);
}

float qo_silu_mul(float gate, float up) {
  const double g = gate;
  return (float)(g / (1.0 + exp(-g)) * (double)up);
}

/* Greatest value, lowest index on ties, NaN never wins; UINT32_MAX when no
 * element qualifies (all NaN). */
uint32_t qo_argmax(const float *values, uint32_t n, float *best) {
  float best_value = -INFINITY;
  uint32_t best_index = UINT32_MAX;
  for (uint32_t i = 0; i < n; ++i) {
    const float v = values[i];
    if (v > best_value || (v == best_value && i < best_index)) {
      best_value = v;
      best_index = i;
    }
  }
  if (best) {
    *best = best_value;
  }
  return best_index;
}

/* ---- decoder layer and model step ----------------------------------------- */
void qo_layer_step(const qo_model *m, uint32_t layer, float *hidden,
                   float *k_cache, float *v_cache, uint32_t position,
                   const float *cos_table, const float *sin_table) {
  const qo_shape *s = &m->shape;
  float *const *w = m->layers[layer].t;
  const uint32_t h = s->hidden, qd = s->heads * s->head_dim,
                 kvd = s->kv_heads * s->head_dim, inter = s->intermediate;
  const uint32_t half = s->head_dim / 2u;
  float *xn = (float *)malloc(h * sizeof(float));
  float *q = (float *)malloc(qd * sizeof(float));
  float *k = (float *)malloc(kvd * sizeof(float));
  float *v = (float *)malloc(kvd * sizeof(float));
  float *attn = (float *)malloc(qd * sizeof(float));
  float *proj = (float *)malloc(h * sizeof(float));
  float *gate = (float *)malloc(inter * sizeof(float));
  float *up = (float *)malloc(inter * sizeof(float));
  if (!xn || !q || !k || !v || !attn || !proj || !gate || !up) {
    abort();
  }

  qo_rmsnorm(hidden, w[QO_ATTN_NORM], h, s->eps, xn);
  qo_gemv(w[QO_Q_W], xn, w[QO_Q_B], qd, h, q);
  qo_gemv(w[QO_K_W], xn, w[QO_K_B], kvd, h, k);
  qo_gemv(w[QO_V_W], xn, w[QO_V_B], kvd, h, v);
  const float *cos_row = cos_table + (size_t)position * half;
  const float *sin_row = sin_table + (size_t)position * half;
  qo_rope_apply(q, s->heads, s->head_dim, cos_row, sin_row);
  qo_rope_apply(k, s->kv_heads, s->head_dim, cos_row, sin_row);
  memcpy(k_cache + (size_t)position * kvd, k, kvd * sizeof(float));
  memcpy(v_cache + (size_t)position * kvd, v, kvd * sizeof(float));
  qo_attention(q, k_cache, v_cache, s->heads, s->kv_heads, s->head_dim,
               position + 1u, attn);
  qo_gemv(w[QO_O_W], attn, NULL, h, qd, proj);
  for (uint32_t i = 0; i < h; ++i) {
    hidden[i] += proj[i];
  }

  qo_rmsnorm(hidden, w[QO_MLP_NORM], h, s->eps, xn);
  qo_gemv(w[QO_GATE_W], xn, NULL, inter, h, gate);
  qo_gemv(w[QO_UP_W], xn, NULL, inter, h, up);
  for (uint32_t i = 0; i < inter; ++i) {
    gate[i] = qo_silu_mul(gate[i], up[i]);
  }
  qo_gemv(w[QO_DOWN_W], gate, NULL, h, inter, proj);
  for (uint32_t i = 0; i < h; ++i) {
    hidden[i] += proj[i];
  }

  free(xn);
  free(q);
  free(k);
  free(v);
  free(attn);
  free(proj);
  free(gate);
  free(up);
}

static void run_layers(const qo_model *m, qo_cache *c, uint32_t token,
                       uint32_t position, float *hidden) {
  const qo_shape *s = &m->shape;
  memcpy(hidden, m->embed + (size_t)token * s->hidden,
         s->hidden * sizeof(float));
  for (uint32_t l = 0; l < s->layers; ++l) {
    qo_layer_step(m, l, hidden, c->k[l], c->v[l], position, c->cos_table,
                  c->sin_table);
  }
}

uint32_t qo_decode_step(const qo_model *m, qo_cache *c, uint32_t token,
                        uint32_t position, float *logits, float *top_logit) {
  const qo_shape *s = &m->shape;
  if (token >= s->vocab || position >= c->capacity) {
    if (top_logit) {
      *top_logit = NAN;
    }
    return UINT32_MAX;
  }
  float *hidden = (float *)malloc(s->hidden * sizeof(float));
  float *local = logits ? NULL : (float *)malloc(s->vocab * sizeof(float));
  float *out = logits ? logits : local;
  if (!hidden || !out) {
    abort();
  }
  run_layers(m, c, token, position, hidden);
  qo_rmsnorm(hidden, m->final_norm, s->hidden, s->eps, c->final_normed);
  qo_gemv(m->lm_head, c->final_normed, NULL, s->vocab, s->hidden, out);
  const uint32_t best = qo_argmax(out, s->vocab, top_logit);
  free(hidden);
  free(local);
  return best;
}

/* Only the last prompt position needs the LM head; earlier positions run the
 * decoder layers to fill the KV cache. */
uint32_t qo_prefill(const qo_model *m, qo_cache *c, const uint32_t *tokens,
                    uint32_t n, uint32_t start, float *last_logits,
                    float *top_logit) {
  const qo_shape *s = &m->shape;
  if (n == 0) {
    return UINT32_MAX;
  }
  float *hidden = (float *)malloc(s->hidden * sizeof(float));
  if (!hidden) {
    abort();
  }
  for (uint32_t i = 0; i + 1u < n; ++i) {
    if (tokens[i] >= s->vocab || start + i >= c->capacity) {
      free(hidden);
      return UINT32_MAX;
    }
    run_layers(m, c, tokens[i], start + i, hidden);
  }
  free(hidden);
  return qo_decode_step(m, c, tokens[n - 1u], start + n - 1u, last_logits,
                        top_logit);
}
