/*
 * cpu_ref.h -- CPU restatement of the MiniMind dense decode step.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the
 * HIP runtime: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product (libmmr.so) never links it.
 *
 * Every function restates the fp32 CPU path of the reference runtime
 * (lvyufeng/minimind-orangepi), keeping its arithmetic order so that results
 * are bit-identical to a build of the reference sources with the same
 * compiler flags (no FMA contraction, SSE float math, glibc libm).
 * Citations are path:line into the reference tree.
 */
#ifndef MMR_ORACLE_CPU_REF_H
#define MMR_ORACLE_CPU_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- primitives -------------------------------------------------------- */

/* decoder_layer.cpp:32-42  y = x * (scale * w), scale = 1/sqrt(sum(x^2)/n + eps) */
void orc_rms_norm_layer(const float* x, const float* w, int64_t n, float eps, float* out);
/* language_model.cpp:24-38 y = (x * scale) * w  (final norm association) */
void orc_rms_norm_final(const float* x, const float* w, int64_t n, float eps, float* out);
/* decoder_layer.cpp:65-78  y[r] = sum_c W[r*cols+c]*x[c], sequential c order */
void orc_matvec(const float* w, int64_t rows, int64_t cols, const float* x, float* y);
/* decoder_layer.cpp:97-122 one row of the cos/sin tables for `position` */
void orc_rope_row(int64_t position, int64_t head_dim, float theta, float* cos_out, float* sin_out);
/* decoder_layer.cpp:124-153 rotate-half RoPE on `heads` consecutive heads, in place */
void orc_apply_rope(float* values, int64_t heads, int64_t head_dim, int64_t position, float theta);
/* decoder_layer.cpp:155-157 */
float orc_silu(float v);
/* decoder_layer.cpp:175-182 act[i] = silu(gu[i]) * gu[i+F] */
void orc_swiglu_from_gate_up(const float* gate_up, int64_t F, float* out);
/* decoder_layer.cpp:184-234 decode attention over `tokens` cached keys,
 * keys/values layout [token][kv_head][d] */
void orc_attention_step(const float* query, const float* keys, const float* values, int64_t tokens,
                        int64_t q_heads, int64_t kv_heads, int64_t head_dim, float* out);
/* decoder_layer.cpp:342-352 per-head q/k RMSNorm followed by RoPE, in place */
void orc_qk_norm_rope(float* query, float* key, const float* q_norm, const float* k_norm, int64_t q_heads,
                      int64_t kv_heads, int64_t head_dim, int64_t position, float eps, float theta);
/* language_model.cpp:408-413 index of the first maximum; -1 when n == 0 */
int32_t orc_argmax(const float* logits, int64_t n);
/* IEEE binary16 round-to-nearest-even and back (the weight rounding the
 * GPU runtime applies on upload). */
uint16_t orc_f32_to_f16(float v);
float orc_f16_to_f32(uint16_t h);

/* ---- model ------------------------------------------------------------- */

typedef struct orc_config {
  int64_t hidden_size, num_hidden_layers, vocab_size, num_attention_heads, num_key_value_heads, head_dim,
      intermediate_size, max_position_embeddings;
  int32_t bos_token_id, eos_token_id, use_moe, tie_word_embeddings;
  float rms_norm_eps, rope_theta;
} orc_config;

typedef struct orc_model orc_model;
typedef struct orc_state orc_state;

/* runtime_loader.cpp:71-88 (+ rms_norm_eps / rope_theta keys) and :121-167.
 * Returns NULL and fills err on failure. */
orc_model* orc_model_load(const char* model_dir, char* err, size_t err_len);
void orc_model_free(orc_model* m);
const orc_config* orc_model_config(const orc_model* m);

orc_state* orc_state_new(const orc_model* m);
void orc_state_free(orc_state* s);
int64_t orc_state_position(const orc_state* s);

/* decoder_layer.cpp:312-407: one decoder layer of the model, in place on
 * hidden [hidden_size], appending to that layer's KV cache in `s` (the
 * state's position is not advanced).  Returns 0, or -1 on a bad layer. */
int orc_decoder_layer(const orc_model* m, orc_state* s, int64_t layer, float* hidden, int64_t position);
/* That layer's cache ([tokens][kv_heads][d] keys and values); returns tokens. */
int64_t orc_state_layer_cache(const orc_state* s, int64_t layer, const float** keys, const float** values);

/* language_model.cpp:297-308 logits of one step; returns 0, or -1 when the token is out of range */
int orc_forward_token(const orc_model* m, orc_state* s, int32_t token, float* logits_out);
/* language_model.cpp:310-333 greedy next token; -1 on a bad token */
int32_t orc_forward_next_token(const orc_model* m, orc_state* s, int32_t token);
/* language_model.cpp:368-406 greedy generate with EOS stop.  Writes up to
 * max_new ids to out, the count to *out_n.  When last_logits is not NULL it
 * receives the logits of the step that produced the last emitted token
 * (after the prompt only: requires max_new >= 1).  Returns 0 or -1. */
int orc_generate(const orc_model* m, const int32_t* prompt, int64_t prompt_len, int64_t max_new, int32_t* out,
                 int64_t* out_n, float* last_logits);

#ifdef __cplusplus
}
#endif
#endif
