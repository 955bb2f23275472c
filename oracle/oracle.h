/*
 * CPU oracle: a C restatement of the reference engine's CPU path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (libqwen_hip.so, the
 * Node-API addon, the JS driver) links, loads or calls this library. Only the
 * tests under tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * use it, and only as the checker (or, for the baseline, as the timed CPU port).
 *
 * Semantics follow the reference exactly: storage is f32, every reduction is
 * accumulated in f64 (a JavaScript number), and every store into a
 * Float32Array is a round-to-nearest-even narrowing. The translation unit is
 * compiled with -ffp-contract=off so that no multiply-add is fused, which JS
 * never does.
 *
 * Each function cites the reference file:line it restates. Functions whose
 * results no reference-held data or closed form pins are marked
 * "parity unpinned" at their definition.
 */
#ifndef QWEN_ORACLE_H
#define QWEN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- float formats: src/core/dtype.js ---------------------------------- */
float or_bf16_to_f32(uint16_t bits);                 /* dtype.js:17-20 */
uint16_t or_f32_to_bf16(float x);                    /* dtype.js:23-35 */
float or_f16_to_f32(uint16_t bits);                  /* dtype.js:55-78 */
uint16_t or_f32_to_f16(float x);                     /* dtype.js:81-113 */
void or_f32_to_f16_array(const float* src, uint16_t* dst, size_t n);  /* dtype.js:122-127 */
void or_f16_to_f32_array(const uint16_t* src, float* dst, size_t n);  /* dtype.js:115-120 */
void or_bf16_to_f32_array(const uint16_t* src, float* dst, size_t n); /* dtype.js:43-48 */

/* ---- quantizer: src/core/quantize.js ------------------------------------ */
void or_quantize_int8(const float* W, int rows, int cols, int8_t* q, float* scales);   /* :36-58 */
void or_dequantize_int8(const int8_t* q, const float* scales, int rows, int cols,
                        float* out);                                                   /* :60-68 */
/* Returns 0, or -1 for a group size below 2 and -2 for one that does not divide cols (:81-86). */
int or_quantize_int4(const float* W, int rows, int cols, int group, uint8_t* q, float* scales,
                     float* zeros);                                                    /* :80-132 */
void or_dequantize_int4(const uint8_t* q, const float* scales, const float* zeros, int rows,
                        int cols, int group, float* out);                              /* :134-151 */
double or_bits_per_weight(int scheme /*8,4,16,32*/, int cols, int group);            /* :171-177 */

/* ---- numeric ops: src/core/ops.js --------------------------------------- */
void or_rmsnorm(const float* x, const float* weight, double eps, int n, float* out);  /* :17-24 */
void or_matvec(const float* W, const float* x, int rows, int cols, const float* bias,
               float* out);                                                            /* :33-41 */
void or_matvec_bf16(const uint16_t* W, const float* x, int rows, int cols, float* out); /* :49-63 */
void or_softmax(float* x, int n);                                                      /* :66-78 */
double or_silu(double x);                                                              /* :81-83 */
void or_swiglu(float* gate, const float* up, int n);                                   /* :88-91 */
void or_rope_freqs(int head_dim, double theta, double* inv);                           /* :99-104 */
void or_rope_tables(int head_dim, double theta, int positions, float* cos_t, float* sin_t); /* :123-136 */
void or_rope_inplace(float* v, int offset, int head_dim, int position, const double* inv); /* :147-159 */

/* ---- attention: src/core/attention.js ------------------------------------ */
void or_grouped_attention(const float* q, const float* keys, const float* values, float* out,
                          float* scores, int seq, int past, int num_heads, int num_kv_heads,
                          int head_dim);                                               /* :32-66 */
int or_kv_head_for(int query_head, int num_heads, int num_kv_heads);                   /* :74-76 */

/* ---- model: src/cpu/model.js, src/cpu/cache.js --------------------------- */
typedef struct {
  int hidden, intermediate, layers, heads, kv_heads, head_dim, vocab;
  double rope_theta, eps;
} or_config;

/* One layer's tensors, as f32 (already dequantized when the run is quantized). */
typedef struct {
  const float *input_norm, *wq, *bq, *wk, *bk, *wv, *bv, *wo, *post_norm, *w_gate, *w_up, *w_down;
} or_layer;

typedef struct {
  or_config cfg;
  const or_layer* layers;      /* [cfg.layers] */
  const float* final_norm;     /* [hidden] */
  const uint16_t* embed_bf16;  /* [vocab, hidden] bf16 bits: the input gather (model.js:190-209) */
  /* The output projection. NULL: the unquantized bf16 embedding streamed through matVecBf16, as
   * ReferenceModel#logits does (model.js:218-228). Non-NULL: an f32 matrix, which is how a
   * quantized run states the loader's round-tripped tied embedding (src/gpu/model.js:156-163,184). */
  const float* lm_head_f32;
  /* Non-zero: keys and values are rounded through f16 when written into the cache, so the CPU sees
   * the same cache contents as a device that stores f16 (the "same-f16" comparison of
   * web/kernels.html:51-54). Zero: the reference's f32 cache (cache.js:18-35). */
  int kv_f16;
} or_model;

typedef struct or_cache or_cache;
or_cache* or_cache_new(const or_config* cfg, int capacity);   /* cache.js:20-31 */
void or_cache_free(or_cache* c);
int or_cache_length(const or_cache* c);                         /* cache.js:34 */
void or_cache_set_length(or_cache* c, int length);              /* rewind, as web/decode-profile.html:151 */
/* writeAt (cache.js:66-71): `count` positions of k and v [count, kv_dim] at `at`; returns -3
 * when at + count exceeds the capacity. Rounds through f16 when kv_f16 is non-zero. */
int or_cache_write(or_cache* c, int layer, int at, const float* k, const float* v, int count,
                   int kv_f16);
/* [kv_heads, length, head_dim] per layer (cache.js:97-115). */
void or_cache_present(const or_cache* c, int layer, float* key, float* value);
/* Positions below `positions` keep what or_cache_write put there when a forward pass appends
 * over them: the pass computes its own keys and values for those positions but attends to the
 * loaded ones. With a device's f16 cache loaded this way, the CPU path and the device read the
 * same K/V at every position, so their difference is each position's own arithmetic, not a
 * cache entry that rounded to the neighbouring f16 value on one side (the same-input
 * comparison of web/kernels.html:51-54, applied to a whole forward pass). 0 (the default)
 * is the reference's cache. No counterpart in src/cpu/cache.js. */
void or_cache_pin(or_cache* c, int positions);
/* What forward passes computed for pinned rows 0..n-1 of `layer` (unrounded f32, in the present
 * layout [kv_heads, n, head_dim]); -3 when nothing is pinned or n exceeds the pinned rows. */
int or_cache_shadow(const or_cache* c, int layer, int n, float* key, float* value);

/*
 * ReferenceModel.forward (model.js:55-166) over `seq` token ids continuing from `cache`.
 * `logits` receives the final position's [vocab] logits (may be NULL to skip the output head).
 * Returns 0, -1 for an empty sequence, -2 for a token outside the vocabulary (model.js:63,199-201),
 * -3 for a cache overflow (cache.js:52-60).
 */
int or_forward(const or_model* m, or_cache* cache, const int32_t* ids, int seq, float* logits);
/* As or_forward, but the caller supplies the embedded input [seq, hidden] (src/gpu/model.js:221-227). */
int or_forward_hidden(const or_model* m, or_cache* cache, const float* hidden, int seq,
                      float* logits);
/* Strict-'>' argmax, lowest index on ties (model.js:181-182, web/bench.html:129-131). */
int32_t or_argmax(const float* v, int n);
/* Negative log-likelihood of `target` under logits[0..n), as the reference's perplexity page
 * computes it (web/perplexity.html:158-166). */
double or_nll(const float* logits, int n, int target);
/* ReferenceModel.generate (model.js:174-187) with greedy tokens written to `tokens` [max_tokens]. */
int or_generate(const or_model* m, or_cache* cache, const int32_t* prompt, int prompt_len,
                int max_tokens, int32_t* tokens);

/* Threads the row-parallel loops may use (results do not depend on it). */
void or_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
