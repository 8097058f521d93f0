/*
 * cpu_ref.c -- CPU restatement of the reference MiniMind fp32 decode path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker).  Loaded by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg; never by the
 * product library.
 *
 * Arithmetic order follows the reference line by line (cited per function)
 * so that a build with gcc -O2 -ffp-contract=off on x86-64 is bit-identical to
 * the reference's own CPU path built the same way.
 */
#include "cpu_ref.h"

#include <ctype.h>
#include <errno.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ---- primitives -------------------------------------------------------- */

/* decoder_layer.cpp:32-42 (rms_norm_inplace): sequential sum of squares,
 * scale = 1/sqrt(sum/n + eps), values *= scale * weight. */
void orc_rms_norm_layer(const float* x, const float* w, int64_t n, float eps, float* out) {
  float sum = 0.0f;
  for (int64_t i = 0; i < n; ++i) sum += x[i] * x[i];
  const float scale = 1.0f / sqrtf(sum / (float)n + eps);
  for (int64_t i = 0; i < n; ++i) out[i] = x[i] * (scale * w[i]);
}

/* language_model.cpp:24-38 (final rms_norm): output = input * scale * weight,
 * evaluated left to right. */
void orc_rms_norm_final(const float* x, const float* w, int64_t n, float eps, float* out) {
  float sum = 0.0f;
  for (int64_t i = 0; i < n; ++i) sum += x[i] * x[i];
  const float scale = 1.0f / sqrtf(sum / (float)n + eps);
  for (int64_t i = 0; i < n; ++i) out[i] = (x[i] * scale) * w[i];
}

/* decoder_layer.cpp:65-78 (cpu_matvec) */
void orc_matvec(const float* w, int64_t rows, int64_t cols, const float* x, float* y) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = w + r * cols;
    float sum = 0.0f;
    for (int64_t c = 0; c < cols; ++c) sum += row[c] * x[c];
    y[r] = sum;
  }
}

/* decoder_layer.cpp:109-119: inv_freq = 1/powf(theta, (2i)/d),
 * angle = float(position) * inv_freq, cosf/sinf.  Row `position` of the
 * reference's [max_position, d/2] tables. */
void orc_rope_row(int64_t position, int64_t head_dim, float theta, float* cos_out, float* sin_out) {
  const int64_t half = head_dim / 2;
  for (int64_t i = 0; i < half; ++i) {
    const float inv_freq = 1.0f / powf(theta, (float)(i * 2) / (float)head_dim);
    const float angle = (float)position * inv_freq;
    cos_out[i] = cosf(angle);
    sin_out[i] = sinf(angle);
  }
}

/* decoder_layer.cpp:139-152: pairs (i, i + d/2), x1' = x1 c - x2 s, x2' = x2 c + x1 s */
void orc_apply_rope(float* values, int64_t heads, int64_t head_dim, int64_t position, float theta) {
  const int64_t half = head_dim / 2;
  float* c = (float*)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
  float* s = (float*)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
  orc_rope_row(position, head_dim, theta, c, s);
  for (int64_t h = 0; h < heads; ++h) {
    float* base = values + h * head_dim;
    for (int64_t i = 0; i < half; ++i) {
      const float first = base[i];
      const float second = base[i + half];
      base[i] = first * c[i] - second * s[i];
      base[i + half] = second * c[i] + first * s[i];
    }
  }
  free(c);
  free(s);
}

/* decoder_layer.cpp:155-157 */
float orc_silu(float v) { return v / (1.0f + expf(-v)); }

/* decoder_layer.cpp:175-182 */
void orc_swiglu_from_gate_up(const float* gate_up, int64_t F, float* out) {
  for (int64_t i = 0; i < F; ++i) out[i] = orc_silu(gate_up[i]) * gate_up[i + F];
}

/* decoder_layer.cpp:200-233: per q head (kv = h / (Hq/Hkv)): scores = dot/sqrt(d),
 * running max, exp(score - max), sequential denominator, then
 * out[h][dim] += (e_t / den) * v_t[dim] in token order. */
void orc_attention_step(const float* query, const float* keys, const float* values, int64_t tokens,
                        int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out) {
  const int64_t repeat = q_heads / kv_heads;
  float* scores = (float*)malloc(sizeof(float) * (size_t)(tokens > 0 ? tokens : 1));
  for (int64_t i = 0; i < q_heads * head_dim; ++i) out[i] = 0.0f;
  for (int64_t h = 0; h < q_heads; ++h) {
    const int64_t kvh = h / repeat;
    float max_score = -INFINITY;
    for (int64_t t = 0; t < tokens; ++t) {
      float dot = 0.0f;
      for (int64_t d = 0; d < head_dim; ++d)
        dot += query[h * head_dim + d] * keys[(t * kv_heads + kvh) * head_dim + d];
      const float score = dot / sqrtf((float)head_dim);
      scores[t] = score;
      max_score = (max_score < score) ? score : max_score; /* std::max(max_score, score) */
    }
    float denom = 0.0f;
    for (int64_t t = 0; t < tokens; ++t) {
      scores[t] = expf(scores[t] - max_score);
      denom += scores[t];
    }
    for (int64_t t = 0; t < tokens; ++t) {
      const float weight = scores[t] / denom;
      for (int64_t d = 0; d < head_dim; ++d)
        out[h * head_dim + d] += weight * values[(t * kv_heads + kvh) * head_dim + d];
    }
  }
  free(scores);
}

/* decoder_layer.cpp:342-352 */
void orc_qk_norm_rope(float* query, float* key, const float* q_norm, const float* k_norm, int64_t q_heads,
                      int64_t kv_heads, int64_t head_dim, int64_t position, float eps, float theta) {
  for (int64_t h = 0; h < q_heads; ++h)
    orc_rms_norm_layer(query + h * head_dim, q_norm, head_dim, eps, query + h * head_dim);
  for (int64_t h = 0; h < kv_heads; ++h)
    orc_rms_norm_layer(key + h * head_dim, k_norm, head_dim, eps, key + h * head_dim);
  orc_apply_rope(query, q_heads, head_dim, position, theta);
  orc_apply_rope(key, kv_heads, head_dim, position, theta);
}

/* language_model.cpp:408-413: std::max_element keeps the first maximum. */
int32_t orc_argmax(const float* logits, int64_t n) {
  if (n <= 0) return -1;
  int64_t best = 0;
  for (int64_t i = 1; i < n; ++i)
    if (logits[best] < logits[i]) best = i;
  return (int32_t)best;
}

uint16_t orc_f32_to_f16(float v) {
  uint32_t x;
  memcpy(&x, &v, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t absx = x & 0x7fffffffu;
  if (absx >= 0x7f800000u) /* inf / nan */
    return (uint16_t)(sign | 0x7c00u | (absx > 0x7f800000u ? 0x200u | ((absx >> 13) & 0x3ffu) : 0u));
  if (absx >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
  if (absx < 0x38800000u) {                                      /* subnormal half (or zero) */
    /* value = absx as float; half subnormal unit is 2^-24 */
    float f;
    memcpy(&f, &absx, 4);
    const float scaled = f * 16777216.0f; /* 2^24, exact */
    /* round half to even via nearbyintf under the default rounding mode */
    const uint32_t m = (uint32_t)nearbyintf(scaled);
    return (uint16_t)(sign | m);
  }
  const uint32_t exp = ((absx >> 23) - 112u) << 10; /* rebias 127 -> 15 */
  const uint32_t mant = absx & 0x7fffffu;
  uint32_t h = exp | (mant >> 13);
  const uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0) {
    const float f = (float)m * (1.0f / 16777216.0f);
    memcpy(&bits, &f, 4);
    bits |= sign;
  } else if (e == 31) {
    bits = sign | 0x7f800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

/* ---- model ------------------------------------------------------------- */

typedef struct {
  float *input_norm, *post_norm, *q_norm, *k_norm;
  float *qkv, *o, *gate_up, *down; /* fused like language_model.cpp:95-119 */
} orc_layer;

struct orc_model {
  orc_config cfg;
  float *embed, *final_norm, *lm_head;
  orc_layer* layers;
};

typedef struct {
  float *keys, *values; /* [tokens][kv_heads][d], decoder_layer.h LayerKvCache */
  int64_t tokens, cap;
} orc_kv;

struct orc_state {
  orc_kv* layers;
  int64_t n_layers, position;
};

static void set_err(char* err, size_t n, const char* fmt, const char* a) {
  if (err && n) snprintf(err, n, fmt, a ? a : "");
}

static char* trim(char* s) {
  while (*s && isspace((unsigned char)*s)) ++s;
  size_t n = strlen(s);
  while (n > 0 && isspace((unsigned char)s[n - 1])) s[--n] = '\0';
  return s;
}

/* minimind/config.cpp:7-13 default_minimind_config */
static void default_config(orc_config* c) {
  memset(c, 0, sizeof(*c));
  c->hidden_size = 768;
  c->num_hidden_layers = 8;
  c->vocab_size = 6400;
  c->num_attention_heads = 8;
  c->num_key_value_heads = 4;
  c->head_dim = 768 / 8;
  c->intermediate_size = (int64_t)ceil(768 * 3.14159265358979323846 / 64.0) * 64;
  c->max_position_embeddings = 32768;
  c->bos_token_id = 1;
  c->eos_token_id = 2;
  c->use_moe = 0;
  c->tie_word_embeddings = 1;
  c->rms_norm_eps = 1e-6f;
  c->rope_theta = 1000000.0f;
}

typedef struct {
  char key[64];
  char val[128];
} kv_pair;

static const char* find_key(const kv_pair* kv, int n, const char* key) {
  const char* found = NULL;
  for (int i = 0; i < n; ++i)
    if (strcmp(kv[i].key, key) == 0) found = kv[i].val; /* later lines win, like the map */
  return found;
}

static int64_t get_i64(const kv_pair* kv, int n, const char* key, int64_t fallback) {
  const char* v = find_key(kv, n, key);
  return v ? strtoll(v, NULL, 10) : fallback;
}

static int get_bool(const kv_pair* kv, int n, const char* key, int fallback) {
  const char* v = find_key(kv, n, key);
  if (!v) return fallback;
  return strcmp(v, "1") == 0 || strcmp(v, "true") == 0 || strcmp(v, "True") == 0;
}

/* runtime_loader.cpp:29-88, plus the rms_norm_eps / rope_theta keys the
 * reference loader leaves unparsed. */
static int load_config(const char* path, orc_config* c, char* err, size_t err_len) {
  FILE* f = fopen(path, "r");
  if (!f) {
    set_err(err, err_len, "failed to open runtime config: %s", path);
    return -1;
  }
  kv_pair kv[256];
  int n = 0;
  char line[512];
  while (fgets(line, sizeof line, f)) {
    char* t = trim(line);
    if (!*t || *t == '#') continue;
    char* eq = strchr(t, '=');
    if (!eq) {
      fclose(f);
      set_err(err, err_len, "invalid runtime config line: %s", t);
      return -1;
    }
    *eq = '\0';
    if (n < 256) {
      snprintf(kv[n].key, sizeof kv[n].key, "%s", trim(t));
      snprintf(kv[n].val, sizeof kv[n].val, "%s", trim(eq + 1));
      ++n;
    }
  }
  fclose(f);
  default_config(c);
  c->hidden_size = get_i64(kv, n, "hidden_size", c->hidden_size);
  c->num_hidden_layers = get_i64(kv, n, "num_hidden_layers", c->num_hidden_layers);
  c->use_moe = get_bool(kv, n, "use_moe", 0);
  c->vocab_size = get_i64(kv, n, "vocab_size", c->vocab_size);
  c->num_attention_heads = get_i64(kv, n, "num_attention_heads", c->num_attention_heads);
  c->num_key_value_heads = get_i64(kv, n, "num_key_value_heads", c->num_key_value_heads);
  c->head_dim = get_i64(kv, n, "head_dim", c->num_attention_heads ? c->hidden_size / c->num_attention_heads : 0);
  c->intermediate_size = get_i64(kv, n, "intermediate_size", c->intermediate_size);
  c->max_position_embeddings = get_i64(kv, n, "max_position_embeddings", c->max_position_embeddings);
  c->tie_word_embeddings = get_bool(kv, n, "tie_word_embeddings", c->tie_word_embeddings);
  const char* eps = find_key(kv, n, "rms_norm_eps");
  if (eps) c->rms_norm_eps = strtof(eps, NULL);
  const char* theta = find_key(kv, n, "rope_theta");
  if (theta) c->rope_theta = strtof(theta, NULL);
  /* minimind/config.cpp:15-78 (validate_config), the dense subset */
  if (c->hidden_size <= 0 || c->num_hidden_layers <= 0 || c->vocab_size <= 0 || c->num_attention_heads <= 0 ||
      c->num_key_value_heads <= 0 || c->head_dim <= 0 || c->intermediate_size <= 0 ||
      c->max_position_embeddings <= 0) {
    set_err(err, err_len, "invalid MiniMind config: %s", "non-positive dimension");
    return -1;
  }
  if (c->hidden_size % c->num_attention_heads != 0 || c->head_dim != c->hidden_size / c->num_attention_heads ||
      c->num_attention_heads % c->num_key_value_heads != 0 || !(c->rope_theta > 0.0f) ||
      !(c->rms_norm_eps > 0.0f)) {
    set_err(err, err_len, "invalid MiniMind config: %s", "inconsistent heads / eps / theta");
    return -1;
  }
  if (c->use_moe) {
    set_err(err, err_len, "%s", "the oracle restates the dense path only (use_moe=0)");
    return -1;
  }
  return 0;
}

static float* read_tensor(FILE* f, const char* name, int64_t expected, char* err, size_t err_len) {
  uint64_t len = 0;
  if (fread(&len, 8, 1, f) != 1 || len > 4096) {
    set_err(err, err_len, "failed to read %s", name);
    return NULL;
  }
  char got[4097];
  if (fread(got, 1, (size_t)len, f) != (size_t)len) {
    set_err(err, err_len, "failed to read %s", name);
    return NULL;
  }
  got[len] = '\0';
  if (strcmp(got, name) != 0) {
    set_err(err, err_len, "expected tensor %s", name);
    return NULL;
  }
  uint64_t count = 0;
  if (fread(&count, 8, 1, f) != 1 || (int64_t)count != expected) {
    set_err(err, err_len, "tensor %s has invalid size", name);
    return NULL;
  }
  float* data = (float*)malloc(sizeof(float) * (size_t)(count ? count : 1));
  if (count && fread(data, sizeof(float), (size_t)count, f) != (size_t)count) {
    free(data);
    set_err(err, err_len, "failed to read %s", name);
    return NULL;
  }
  return data;
}

static float* concat3(float* a, int64_t na, float* b, int64_t nb, float* c, int64_t nc) {
  float* out = (float*)malloc(sizeof(float) * (size_t)(na + nb + nc));
  memcpy(out, a, sizeof(float) * (size_t)na);
  memcpy(out + na, b, sizeof(float) * (size_t)nb);
  if (c) memcpy(out + na + nb, c, sizeof(float) * (size_t)nc);
  free(a);
  free(b);
  free(c);
  return out;
}

void orc_model_free(orc_model* m) {
  if (!m) return;
  free(m->embed);
  free(m->final_norm);
  free(m->lm_head);
  if (m->layers) {
    for (int64_t l = 0; l < m->cfg.num_hidden_layers; ++l) {
      orc_layer* L = &m->layers[l];
      free(L->input_norm);
      free(L->post_norm);
      free(L->q_norm);
      free(L->k_norm);
      free(L->qkv);
      free(L->o);
      free(L->gate_up);
      free(L->down);
    }
    free(m->layers);
  }
  free(m);
}

/* runtime_loader.cpp:121-167 (fixed tensor order, MMRTW001 magic) */
orc_model* orc_model_load(const char* model_dir, char* err, size_t err_len) {
  char path[4096];
  orc_model* m = (orc_model*)calloc(1, sizeof(orc_model));
  snprintf(path, sizeof path, "%s/minimind_runtime_config.txt", model_dir);
  if (load_config(path, &m->cfg, err, err_len) != 0) {
    free(m);
    return NULL;
  }
  const orc_config* c = &m->cfg;
  snprintf(path, sizeof path, "%s/weights.bin", model_dir);
  FILE* f = fopen(path, "rb");
  if (!f) {
    set_err(err, err_len, "failed to open runtime weights: %s", path);
    free(m);
    return NULL;
  }
  char magic[8];
  if (fread(magic, 1, 8, f) != 8 || memcmp(magic, "MMRTW001", 8) != 0) {
    fclose(f);
    set_err(err, err_len, "%s", "unsupported runtime weight format");
    free(m);
    return NULL;
  }
  const int64_t H = c->hidden_size, V = c->vocab_size, D = c->head_dim;
  const int64_t qs = c->num_attention_heads * D, kvs = c->num_key_value_heads * D, F = c->intermediate_size;
  int ok = 1;
  ok = ok && (m->embed = read_tensor(f, "model.embed_tokens.weight", V * H, err, err_len));
  ok = ok && (m->final_norm = read_tensor(f, "model.norm.weight", H, err, err_len));
  ok = ok && (m->lm_head = read_tensor(f, "lm_head.weight", V * H, err, err_len));
  if (ok) m->layers = (orc_layer*)calloc((size_t)c->num_hidden_layers, sizeof(orc_layer));
  for (int64_t l = 0; ok && l < c->num_hidden_layers; ++l) {
    orc_layer* L = &m->layers[l];
    char name[256];
#define RT(field, suffix, count)                                                     \
  do {                                                                               \
    snprintf(name, sizeof name, "model.layers.%lld.%s", (long long)l, suffix);      \
    ok = ok && ((field) = read_tensor(f, name, (count), err, err_len)) != NULL;     \
  } while (0)
    float *q = NULL, *k = NULL, *v = NULL, *g = NULL, *u = NULL;
    RT(L->input_norm, "input_layernorm.weight", H);
    RT(L->post_norm, "post_attention_layernorm.weight", H);
    RT(L->q_norm, "self_attn.q_norm.weight", D);
    RT(L->k_norm, "self_attn.k_norm.weight", D);
    RT(q, "self_attn.q_proj.weight", qs * H);
    RT(k, "self_attn.k_proj.weight", kvs * H);
    RT(v, "self_attn.v_proj.weight", kvs * H);
    RT(L->o, "self_attn.o_proj.weight", H * qs);
    RT(g, "mlp.gate_proj.weight", F * H);
    RT(u, "mlp.up_proj.weight", F * H);
    RT(L->down, "mlp.down_proj.weight", H * F);
#undef RT
    if (ok) {
      L->qkv = concat3(q, qs * H, k, kvs * H, v, kvs * H);
      L->gate_up = concat3(g, F * H, u, F * H, NULL, 0);
    } else {
      free(q);
      free(k);
      free(v);
      free(g);
      free(u);
    }
  }
  fclose(f);
  if (!ok) {
    orc_model_free(m);
    return NULL;
  }
  return m;
}

const orc_config* orc_model_config(const orc_model* m) { return &m->cfg; }

orc_state* orc_state_new(const orc_model* m) {
  orc_state* s = (orc_state*)calloc(1, sizeof(orc_state));
  s->n_layers = m->cfg.num_hidden_layers;
  s->layers = (orc_kv*)calloc((size_t)s->n_layers, sizeof(orc_kv));
  return s;
}

void orc_state_free(orc_state* s) {
  if (!s) return;
  for (int64_t l = 0; l < s->n_layers; ++l) {
    free(s->layers[l].keys);
    free(s->layers[l].values);
  }
  free(s->layers);
  free(s);
}

int64_t orc_state_position(const orc_state* s) { return s->position; }

static void kv_append(orc_kv* kv, const float* k, const float* v, int64_t n) {
  if (kv->tokens * n + n > kv->cap) {
    int64_t cap = kv->cap ? kv->cap * 2 : n * 64;
    while (cap < kv->tokens * n + n) cap *= 2;
    kv->keys = (float*)realloc(kv->keys, sizeof(float) * (size_t)cap);
    kv->values = (float*)realloc(kv->values, sizeof(float) * (size_t)cap);
    kv->cap = cap;
  }
  memcpy(kv->keys + kv->tokens * n, k, sizeof(float) * (size_t)n);
  memcpy(kv->values + kv->tokens * n, v, sizeof(float) * (size_t)n);
  kv->tokens += 1;
}

/* decoder_layer.cpp:312-407 (run_dense_decoder_layer, dense branch), in place on hidden */
static void layer_step(const orc_config* c, const orc_layer* L, orc_kv* kv, float* hidden, int64_t position) {
  const int64_t H = c->hidden_size, D = c->head_dim, Hq = c->num_attention_heads, Hkv = c->num_key_value_heads;
  const int64_t qs = Hq * D, kvs = Hkv * D, F = c->intermediate_size;
  float* normed = (float*)malloc(sizeof(float) * (size_t)H);
  float* qkv = (float*)malloc(sizeof(float) * (size_t)(qs + 2 * kvs));
  float* ctx = (float*)malloc(sizeof(float) * (size_t)qs);
  float* attn = (float*)malloc(sizeof(float) * (size_t)H);
  float* gu = (float*)malloc(sizeof(float) * (size_t)(2 * F));
  float* act = (float*)malloc(sizeof(float) * (size_t)F);
  float* mlp = (float*)malloc(sizeof(float) * (size_t)H);

  orc_rms_norm_layer(hidden, L->input_norm, H, c->rms_norm_eps, normed);    /* :327 */
  orc_matvec(L->qkv, qs + 2 * kvs, H, normed, qkv);                          /* :331-335 */
  float* q = qkv;
  float* k = qkv + qs;
  float* v = qkv + qs + kvs;
  orc_qk_norm_rope(q, k, L->q_norm, L->k_norm, Hq, Hkv, D, position, c->rms_norm_eps, c->rope_theta); /* :342-352 */
  kv_append(kv, k, v, kvs);                                                  /* :354-359 */
  orc_attention_step(q, kv->keys, kv->values, kv->tokens, Hq, Hkv, D, ctx);  /* :361 */
  orc_matvec(L->o, H, qs, ctx, attn);                                        /* :362 */
  for (int64_t i = 0; i < H; ++i) hidden[i] = hidden[i] + attn[i];           /* :364-367 */
  orc_rms_norm_layer(hidden, L->post_norm, H, c->rms_norm_eps, normed);      /* :369 */
  orc_matvec(L->gate_up, 2 * F, H, normed, gu);                              /* :393 */
  orc_swiglu_from_gate_up(gu, F, act);                                       /* :394 */
  orc_matvec(L->down, H, F, act, mlp);                                       /* :400 */
  for (int64_t i = 0; i < H; ++i) hidden[i] += mlp[i];                       /* :403-405 */

  free(normed);
  free(qkv);
  free(ctx);
  free(attn);
  free(gu);
  free(act);
  free(mlp);
}

/* decoder_layer.cpp:312-407 for one layer of the model on its own: hidden is
 * updated in place, the layer's KV cache in `s` grows by one token.  The same
 * layer_step the model uses, exposed for the per-layer boundary test. */
int orc_decoder_layer(const orc_model* m, orc_state* s, int64_t layer, float* hidden, int64_t position) {
  if (layer < 0 || layer >= m->cfg.num_hidden_layers) return -1;
  layer_step(&m->cfg, &m->layers[layer], &s->layers[layer], hidden, position);
  return 0;
}

/* Keys / values of one layer's cache, [tokens][kv_heads][d]; returns tokens. */
int64_t orc_state_layer_cache(const orc_state* s, int64_t layer, const float** keys, const float** values) {
  if (layer < 0 || layer >= s->n_layers) return -1;
  *keys = s->layers[layer].keys;
  *values = s->layers[layer].values;
  return s->layers[layer].tokens;
}

/* language_model.cpp:297-308 (forward_token) */
int orc_forward_token(const orc_model* m, orc_state* s, int32_t token, float* logits_out) {
  const orc_config* c = &m->cfg;
  const int64_t H = c->hidden_size;
  if (token < 0 || token >= c->vocab_size) return -1; /* :71-73 out_of_range */
  float* hidden = (float*)malloc(sizeof(float) * (size_t)H);
  float* normed = (float*)malloc(sizeof(float) * (size_t)H);
  memcpy(hidden, m->embed + (int64_t)token * H, sizeof(float) * (size_t)H);
  for (int64_t l = 0; l < c->num_hidden_layers; ++l) layer_step(c, &m->layers[l], &s->layers[l], hidden, s->position);
  s->position += 1;
  orc_rms_norm_final(hidden, m->final_norm, H, c->rms_norm_eps, normed);
  orc_matvec(m->lm_head, c->vocab_size, H, normed, logits_out);
  free(hidden);
  free(normed);
  return 0;
}

/* language_model.cpp:310-333 (CPU branch): argmax of the same logits */
int32_t orc_forward_next_token(const orc_model* m, orc_state* s, int32_t token) {
  float* logits = (float*)malloc(sizeof(float) * (size_t)m->cfg.vocab_size);
  int32_t next = -1;
  if (orc_forward_token(m, s, token, logits) == 0) next = orc_argmax(logits, m->cfg.vocab_size);
  free(logits);
  return next;
}

/* language_model.cpp:368-406 (generate_stream without Ascend: token-by-token prefill) */
int orc_generate(const orc_model* m, const int32_t* prompt, int64_t prompt_len, int64_t max_new, int32_t* out,
                 int64_t* out_n, float* last_logits) {
  *out_n = 0;
  if (prompt_len <= 0 || max_new < 0) return -1;
  const int64_t V = m->cfg.vocab_size;
  orc_state* s = orc_state_new(m);
  float* logits = (float*)malloc(sizeof(float) * (size_t)V);
  int32_t next = 0;
  int rc = 0;
  for (int64_t i = 0; i < prompt_len && rc == 0; ++i) {
    rc = orc_forward_token(m, s, prompt[i], logits);
    next = orc_argmax(logits, V);
  }
  if (rc == 0 && last_logits) memcpy(last_logits, logits, sizeof(float) * (size_t)V);
  for (int64_t i = 0; rc == 0 && i < max_new; ++i) {
    out[(*out_n)++] = next;
    if (next == m->cfg.eos_token_id || i + 1 == max_new) break;
    rc = orc_forward_token(m, s, next, logits);
    next = orc_argmax(logits, V);
    if (rc == 0 && last_logits) memcpy(last_logits, logits, sizeof(float) * (size_t)V);
  }
  free(logits);
  orc_state_free(s);
  return rc;
}
