/*
 * CPU oracle: a C restatement of the reference engine's CPU path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg. The product never links or loads it.
 *
 * Reference: abho7/llm-inference-webgpu. Every function cites the file:line it
 * restates. JavaScript semantics are kept where they decide bits:
 *   - reductions accumulate in double, from the value the reference starts at;
 *   - a store into a Float32Array is a (float) cast, round-to-nearest-even;
 *   - Math.round on a non-negative argument is C round() (ties away from zero);
 *   - Math.min / Math.max propagate NaN and order -0 below +0 (js_min/js_max);
 *   - no multiply-add is fused (built with -ffp-contract=off).
 *
 * Pinning (see tests/test_oracle_*.py): the reference's own known-answer tests
 * (test/ops.test.js, test/quantize.test.js, test/attention.test.js,
 * test/cache.test.js) are transcribed as tests of these functions; the f16
 * conversions are checked exhaustively against numpy's independent float16;
 * the quantizer against hand-computed tie cases and its invariants; attention
 * against an expanded-heads brute force (exact) and an independent numpy
 * float64 formula; the model forward against incremental-vs-full bit equality
 * and a numpy float64 re-derivation of one layer.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

void or_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------------------ helpers */

static uint32_t f32_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float bits_f32(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* Math.min / Math.max: NaN if either is NaN; -0 < +0. */
static double js_min(double a, double b) {
  if (isnan(a) || isnan(b)) return NAN;
  if (a == 0 && b == 0) return (signbit(a) || signbit(b)) ? -0.0 : 0.0;
  return a < b ? a : b;
}
static double js_max(double a, double b) {
  if (isnan(a) || isnan(b)) return NAN;
  if (a == 0 && b == 0) return (signbit(a) && signbit(b)) ? -0.0 : 0.0;
  return a > b ? a : b;
}

/* roundHalfAwayFromZero, src/core/quantize.js:25-27. For x >= 0 Math.round rounds ties up,
 * which is away from zero, and the negative branch mirrors it: C round() exactly. */
static double round_half_away(double x) { return round(x); }

/* ToInt32 as applied by the reference's typed-array stores and bit operators: NaN -> 0. */
static int js_to_int(double v) { return isnan(v) ? 0 : (int)v; }

/* ------------------------------------------------------------ dtype.js ---- */

/* dtype.js:17-20: bf16 is the top half of an f32; widening is a shift. */
float or_bf16_to_f32(uint16_t bits) { return bits_f32((uint32_t)bits << 16); }

/* dtype.js:23-35: round to nearest even, NaN kept NaN with a forced payload bit. */
uint16_t or_f32_to_bf16(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0) {
    return (uint16_t)(((u >> 16) | 0x0040u) & 0xffffu);
  }
  uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)(((u + 0x7fffu + lsb) >> 16) & 0xffffu);
}

/* dtype.js:55-78 */
float or_f16_to_f32(uint16_t bits) {
  uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
  uint32_t exp = (bits >> 10) & 0x1fu;
  uint32_t mant = bits & 0x3ffu;
  uint32_t out;
  if (exp == 0x1f) {
    out = sign | 0x7f800000u | (mant << 13);
  } else if (exp == 0) {
    if (mant == 0) {
      out = sign;
    } else {
      int e = -1;
      uint32_t m = mant;
      do { m <<= 1; e++; } while ((m & 0x400u) == 0);
      out = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3ffu) << 13);
    }
  } else {
    out = sign | ((exp - 15 + 127) << 23) | (mant << 13);
  }
  return bits_f32(out);
}

/* dtype.js:81-113: round to nearest even, overflow to inf, gradual underflow. */
uint16_t or_f32_to_f16(float x) {
  uint32_t u = f32_bits(x);
  uint32_t sign = (u >> 16) & 0x8000u;
  int exp = (int)((u >> 23) & 0xffu);
  uint32_t mant = u & 0x7fffffu;
  if (exp == 0xff) {
    return (uint16_t)(sign | 0x7c00u | (mant != 0 ? ((mant >> 13) | 0x200u) : 0u));
  }
  int e = exp - 127 + 15;
  if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    uint32_t m = mant | 0x800000u;
    int shift = 14 - e;
    uint32_t half = 1u << (shift - 1);
    uint32_t lsb = (m >> shift) & 1u;
    return (uint16_t)(sign | ((m + half - 1 + lsb) >> shift));
  }
  uint32_t lsb = (mant >> 13) & 1u;
  uint32_t rounded = mant + 0x0fffu + lsb;
  return (uint16_t)(sign | (((uint32_t)e << 10) + (rounded >> 13)));
}

void or_f32_to_f16_array(const float* src, uint16_t* dst, size_t n) {   /* dtype.js:122-127 */
  for (size_t i = 0; i < n; i++) dst[i] = or_f32_to_f16(src[i]);
}
void or_f16_to_f32_array(const uint16_t* src, float* dst, size_t n) {   /* dtype.js:115-120 */
  for (size_t i = 0; i < n; i++) dst[i] = or_f16_to_f32(src[i]);
}
void or_bf16_to_f32_array(const uint16_t* src, float* dst, size_t n) {  /* dtype.js:43-48 */
  for (size_t i = 0; i < n; i++) dst[i] = or_bf16_to_f32(src[i]);
}

/* ---------------------------------------------------------- quantize.js ---- */

/* quantize.js:36-58: symmetric int8, one f64 scale per row stored as f32; the inverse is taken
 * from the f64 scale, not the stored f32 one. An all-zero row keeps scale 0 and zero codes. */
void or_quantize_int8(const float* W, int rows, int cols, int8_t* q, float* scales) {
  for (int r = 0; r < rows; r++) {
    const size_t base = (size_t)r * cols;
    double peak = 0;
    for (int c = 0; c < cols; c++) {
      double magnitude = fabs((double)W[base + c]);
      if (magnitude > peak) peak = magnitude;
    }
    double scale = peak / 127;
    scales[r] = (float)scale;
    memset(q + base, 0, (size_t)cols);
    if (scale == 0) continue;
    double inverse = 1 / scale;
    for (int c = 0; c < cols; c++) {
      double level = round_half_away((double)W[base + c] * inverse);
      q[base + c] = (int8_t)js_to_int(js_max(-127, js_min(127, level)));
    }
  }
}

/* quantize.js:60-68: w = q * scale, the f64 product stored to f32. */
void or_dequantize_int8(const int8_t* q, const float* scales, int rows, int cols, float* out) {
  for (int r = 0; r < rows; r++) {
    const size_t base = (size_t)r * cols;
    double scale = scales[r];
    for (int c = 0; c < cols; c++) out[base + c] = (float)((double)q[base + c] * scale);
  }
}

/* quantize.js:80-132: asymmetric int4 per group; the range always includes zero; integer zero
 * point; levels clamped after adding the zero; two codes per byte, low nibble = even flat index. */
int or_quantize_int4(const float* W, int rows, int cols, int group, uint8_t* q, float* scales,
                     float* zeros) {
  if (group < 2) return -1;
  if (cols % group != 0) return -2;
  const int gpr = cols / group;
  memset(q, 0, (size_t)rows * cols / 2);
  for (int r = 0; r < rows; r++) {
    for (int g = 0; g < gpr; g++) {
      const size_t base = (size_t)r * cols + (size_t)g * group;
      double lo = INFINITY, hi = -INFINITY;
      for (int i = 0; i < group; i++) {
        double value = W[base + i];
        if (value < lo) lo = value;
        if (value > hi) hi = value;
      }
      lo = js_min(lo, 0);
      hi = js_max(hi, 0);
      double scale = (hi - lo) / 15;
      const size_t index = (size_t)r * gpr + g;
      scales[index] = (float)scale;
      if (scale == 0) {
        zeros[index] = 0;
        continue;
      }
      double zero = js_max(0, js_min(15, round_half_away(-lo / scale)));
      zeros[index] = (float)zero;
      double inverse = 1 / scale;
      for (int i = 0; i < group; i++) {
        double level_d = js_max(0, js_min(15, round_half_away((double)W[base + i] * inverse) + zero));
        uint32_t level = (uint32_t)js_to_int(level_d) & 0xffu;
        size_t at = base + i;
        size_t byte = at >> 1;
        if ((at & 1) == 0) q[byte] = (uint8_t)((q[byte] & 0xf0u) | level);
        else q[byte] = (uint8_t)((q[byte] & 0x0fu) | (level << 4));
      }
    }
  }
  return 0;
}

/* quantize.js:134-151: w = (level - zero) * scale, stored to f32. */
void or_dequantize_int4(const uint8_t* q, const float* scales, const float* zeros, int rows,
                        int cols, int group, float* out) {
  const int gpr = cols / group;
  for (int r = 0; r < rows; r++) {
    for (int g = 0; g < gpr; g++) {
      const size_t base = (size_t)r * cols + (size_t)g * group;
      const size_t index = (size_t)r * gpr + g;
      double scale = scales[index];
      double zero = zeros[index];
      for (int i = 0; i < group; i++) {
        size_t at = base + i;
        uint8_t byte = q[at >> 1];
        int level = (at & 1) == 0 ? (byte & 0x0f) : (byte >> 4);
        out[at] = (float)(((double)level - zero) * scale);
      }
    }
  }
}

/* quantize.js:171-177 */
double or_bits_per_weight(int scheme, int cols, int group) {
  if (scheme == 8) return 8 + 32.0 / cols;
  if (scheme == 4) return 4 + 64.0 / group;
  if (scheme == 16) return 16;
  if (scheme == 32) return 32;
  return NAN;
}

/* --------------------------------------------------------------- ops.js ---- */

/* ops.js:17-24: eps inside the root; x*scale*weight evaluated left to right in f64. */
void or_rmsnorm(const float* x, const float* weight, double eps, int n, float* out) {
  double sum_squares = 0;
  for (int i = 0; i < n; i++) sum_squares += (double)x[i] * (double)x[i];
  double scale = 1 / sqrt(sum_squares / n + eps);
  for (int i = 0; i < n; i++) out[i] = (float)((double)x[i] * scale * (double)weight[i]);
}

/* ops.js:33-41: the sum starts from the bias and runs in column order in f64. Four rows are
 * summed side by side (each still in its own column order, so every output is the same), which
 * keeps four independent add chains in flight instead of one. */
void or_matvec(const float* W, const float* x, int rows, int cols, const float* bias,
               float* out) {
  const int quads = rows / 4;
#pragma omp parallel for schedule(static) if ((size_t)rows * cols > (1u << 18))
  for (int g = 0; g < quads; g++) {
    const int r = 4 * g;
    const float* w0 = W + (size_t)r * cols;
    const float* w1 = w0 + cols;
    const float* w2 = w1 + cols;
    const float* w3 = w2 + cols;
    double a0 = bias ? (double)bias[r] : 0, a1 = bias ? (double)bias[r + 1] : 0;
    double a2 = bias ? (double)bias[r + 2] : 0, a3 = bias ? (double)bias[r + 3] : 0;
    for (int c = 0; c < cols; c++) {
      const double xc = (double)x[c];
      a0 += (double)w0[c] * xc;
      a1 += (double)w1[c] * xc;
      a2 += (double)w2[c] * xc;
      a3 += (double)w3[c] * xc;
    }
    out[r] = (float)a0;
    out[r + 1] = (float)a1;
    out[r + 2] = (float)a2;
    out[r + 3] = (float)a3;
  }
  for (int r = 4 * quads; r < rows; r++) {
    const float* row = W + (size_t)r * cols;
    double acc = bias ? (double)bias[r] : 0;
    for (int c = 0; c < cols; c++) acc += (double)row[c] * (double)x[c];
    out[r] = (float)acc;
  }
}

/* ops.js:49-63: as matVec, W widened from bf16 per element, no bias. */
void or_matvec_bf16(const uint16_t* W, const float* x, int rows, int cols, float* out) {
#pragma omp parallel for schedule(static) if ((size_t)rows * cols > (1u << 18))
  for (int r = 0; r < rows; r++) {
    const uint16_t* row = W + (size_t)r * cols;
    double acc = 0;
    for (int c = 0; c < cols; c++) acc += (double)or_bf16_to_f32(row[c]) * (double)x[c];
    out[r] = (float)acc;
  }
}

/* ops.js:66-78: the exponentials are stored to f32 but summed unrounded in f64. */
void or_softmax(float* x, int n) {
  double max = -INFINITY;
  for (int i = 0; i < n; i++) if (x[i] > max) max = x[i];
  double sum = 0;
  for (int i = 0; i < n; i++) {
    double e = exp((double)x[i] - max);
    x[i] = (float)e;
    sum += e;
  }
  double inv = 1 / sum;
  for (int i = 0; i < n; i++) x[i] = (float)((double)x[i] * inv);
}

double or_silu(double x) { return x / (1 + exp(-x)); }   /* ops.js:81-83 */

void or_swiglu(float* gate, const float* up, int n) {     /* ops.js:88-91 */
  for (int i = 0; i < n; i++) gate[i] = (float)(or_silu((double)gate[i]) * (double)up[i]);
}

/* ops.js:99-104: inv_freq[j] = theta^(-2j/headDim). */
void or_rope_freqs(int head_dim, double theta, double* inv) {
  int half = head_dim >> 1;
  for (int j = 0; j < half; j++) inv[j] = pow(theta, (-2.0 * j) / head_dim);
}

/* ops.js:123-136: [positions, headDim/2] cos and sin, f64 angles stored f32. */
void or_rope_tables(int head_dim, double theta, int positions, float* cos_t, float* sin_t) {
  int half = head_dim >> 1;
  double* inv = (double*)malloc(sizeof(double) * (size_t)half);
  or_rope_freqs(head_dim, theta, inv);
  for (int p = 0; p < positions; p++) {
    for (int j = 0; j < half; j++) {
      double angle = p * inv[j];
      cos_t[(size_t)p * half + j] = (float)cos(angle);
      sin_t[(size_t)p * half + j] = (float)sin(angle);
    }
  }
  free(inv);
}

/* ops.js:147-159: half-split rotation, j pairs with j + headDim/2, angles in f64. */
void or_rope_inplace(float* v, int offset, int head_dim, int position, const double* inv) {
  int half = head_dim >> 1;
  for (int j = 0; j < half; j++) {
    double angle = position * inv[j];
    double c = cos(angle);
    double s = sin(angle);
    double lo = v[offset + j];
    double hi = v[offset + j + half];
    v[offset + j] = (float)(lo * c - hi * s);
    v[offset + j + half] = (float)(hi * c + lo * s);
  }
}

/* --------------------------------------------------------- attention.js ---- */

/* attention.js:74-76: blocked head map. */
int or_kv_head_for(int query_head, int num_heads, int num_kv_heads) {
  return query_head / (num_heads / num_kv_heads);
}

/* attention.js:32-66. Scores: f64 dot, scaled, stored f32; softmax as ops.js; the output
 * accumulates sequentially in the f32 output array (each += is an f64 sum stored to f32).
 * Heads are independent, so they run in parallel without changing any result. */
void or_grouped_attention(const float* q, const float* keys, const float* values, float* out,
                          float* scores, int seq, int past, int num_heads, int num_kv_heads,
                          int head_dim) {
  const int group = num_heads / num_kv_heads;
  const int q_dim = num_heads * head_dim;
  const int kv_dim = num_kv_heads * head_dim;
  const double scale = 1 / sqrt((double)head_dim);
  const int total = past + seq;
  memset(out, 0, sizeof(float) * (size_t)seq * q_dim);
  (void)scores;

#pragma omp parallel if ((size_t)num_heads * seq * total * head_dim > (1u << 20))
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)(total > 0 ? total : 1));
    /* (head, query) pairs write disjoint outputs, each in its own sequential order. */
#pragma omp for schedule(dynamic)
    for (int ht = 0; ht < num_heads * seq; ht++) {
      const int h = ht / seq;
      const int kv_base = (h / group) * head_dim;
      {
        const int t = ht % seq;
        const int q_base = t * q_dim + h * head_dim;
        const int up_to = past + t;
        for (int s = 0; s <= up_to; s++) {
          const size_t k_base = (size_t)s * kv_dim + kv_base;
          double dot = 0;
          for (int i = 0; i < head_dim; i++) dot += (double)q[q_base + i] * (double)keys[k_base + i];
          sc[s] = (float)(dot * scale);
        }
        or_softmax(sc, up_to + 1);
        const int out_base = t * q_dim + h * head_dim;
        for (int s = 0; s <= up_to; s++) {
          const double weight = sc[s];
          const size_t v_base = (size_t)s * kv_dim + kv_base;
          for (int i = 0; i < head_dim; i++) {
            out[out_base + i] = (float)((double)out[out_base + i] + weight * (double)values[v_base + i]);
          }
        }
      }
    }
    free(sc);
  }
}

/* ------------------------------------------------------- cpu/cache.js ---- */

struct or_cache {
  int layers, kv_dim, kv_heads, head_dim, capacity, length;
  int pinned;  /* positions below this keep their contents when a forward pass writes them */
  float** keys;
  float** values;
  /* While pinned: what a forward pass computed for the pinned rows, unrounded f32. */
  float** shadow_keys;
  float** shadow_values;
};

/* cache.js:20-31: [capacity, kvDim] f32 per layer for keys and for values. */
or_cache* or_cache_new(const or_config* cfg, int capacity) {
  if (capacity < 1) return NULL;
  or_cache* c = (or_cache*)calloc(1, sizeof(or_cache));
  c->layers = cfg->layers;
  c->kv_heads = cfg->kv_heads;
  c->head_dim = cfg->head_dim;
  c->kv_dim = cfg->kv_heads * cfg->head_dim;
  c->capacity = capacity;
  c->keys = (float**)calloc((size_t)cfg->layers, sizeof(float*));
  c->values = (float**)calloc((size_t)cfg->layers, sizeof(float*));
  for (int l = 0; l < cfg->layers; l++) {
    c->keys[l] = (float*)calloc((size_t)capacity * c->kv_dim, sizeof(float));
    c->values[l] = (float*)calloc((size_t)capacity * c->kv_dim, sizeof(float));
  }
  return c;
}

void or_cache_free(or_cache* c) {
  if (!c) return;
  for (int l = 0; l < c->layers; l++) {
    free(c->keys[l]);
    free(c->values[l]);
    if (c->shadow_keys) free(c->shadow_keys[l]);
    if (c->shadow_values) free(c->shadow_values[l]);
  }
  free(c->keys);
  free(c->values);
  free(c->shadow_keys);
  free(c->shadow_values);
  free(c);
}

int or_cache_length(const or_cache* c) { return c->length; }
void or_cache_set_length(or_cache* c, int length) { c->length = length; }
void or_cache_pin(or_cache* c, int positions) {
  c->pinned = positions < 0 ? 0 : positions > c->capacity ? c->capacity : positions;
  if (c->pinned && !c->shadow_keys) {
    c->shadow_keys = (float**)calloc((size_t)c->layers, sizeof(float*));
    c->shadow_values = (float**)calloc((size_t)c->layers, sizeof(float*));
    for (int l = 0; l < c->layers; l++) {
      c->shadow_keys[l] = (float*)calloc((size_t)c->capacity * c->kv_dim, sizeof(float));
      c->shadow_values[l] = (float*)calloc((size_t)c->capacity * c->kv_dim, sizeof(float));
    }
  }
}

/* The shadow rows 0..n-1 of a layer in the present layout [kv_heads, n, head_dim]. */
int or_cache_shadow(const or_cache* c, int layer, int n, float* key, float* value) {
  if (!c->shadow_keys || layer < 0 || layer >= c->layers || n < 0 || n > c->pinned) return -3;
  for (int h = 0; h < c->kv_heads; h++) {
    for (int t = 0; t < n; t++) {
      const size_t from = (size_t)t * c->kv_dim + (size_t)h * c->head_dim;
      const size_t to = ((size_t)h * n + t) * c->head_dim;
      memcpy(key + to, c->shadow_keys[layer] + from, sizeof(float) * (size_t)c->head_dim);
      memcpy(value + to, c->shadow_values[layer] + from, sizeof(float) * (size_t)c->head_dim);
    }
  }
  return 0;
}

/* cache.js:97-115: stored [position, kvHead*headDim], published [kvHead, position, headDim]. */
void or_cache_present(const or_cache* c, int layer, float* key, float* value) {
  const int n = c->length;
  for (int h = 0; h < c->kv_heads; h++) {
    for (int t = 0; t < n; t++) {
      const size_t from = (size_t)t * c->kv_dim + (size_t)h * c->head_dim;
      const size_t to = ((size_t)h * n + t) * c->head_dim;
      memcpy(key + to, c->keys[layer] + from, sizeof(float) * (size_t)c->head_dim);
      memcpy(value + to, c->values[layer] + from, sizeof(float) * (size_t)c->head_dim);
    }
  }
}

/* cache.js:66-71 (writeAt), with the optional same-f16 rounding. Rows below `floor` are left
 * as they are. */
static void cache_write_from(or_cache* c, int layer, int at, const float* k, const float* v, int count,
                             int kv_f16, int floor) {
  const size_t first = at < floor ? (size_t)(floor - at) * c->kv_dim : 0;
  const size_t n = (size_t)count * c->kv_dim;
  float* kd = c->keys[layer] + (size_t)at * c->kv_dim;
  float* vd = c->values[layer] + (size_t)at * c->kv_dim;
  for (size_t i = first; i < n; i++) {
    kd[i] = kv_f16 ? or_f16_to_f32(or_f32_to_f16(k[i])) : k[i];
    vd[i] = kv_f16 ? or_f16_to_f32(or_f32_to_f16(v[i])) : v[i];
  }
}

/* A forward pass's append: pinned rows keep the contents loaded into them, and what the pass
 * computed for them goes to the shadow rows unrounded. */
static void cache_write(or_cache* c, int layer, int at, const float* k, const float* v, int count,
                        int kv_f16) {
  for (int t = at; t < at + count && t < c->pinned; t++) {
    const size_t o = (size_t)t * c->kv_dim, i = (size_t)(t - at) * c->kv_dim;
    memcpy(c->shadow_keys[layer] + o, k + i, sizeof(float) * (size_t)c->kv_dim);
    memcpy(c->shadow_values[layer] + o, v + i, sizeof(float) * (size_t)c->kv_dim);
  }
  cache_write_from(c, layer, at, k, v, count, kv_f16, c->pinned);
}

int or_cache_write(or_cache* c, int layer, int at, const float* k, const float* v, int count,
                   int kv_f16) {
  if (layer < 0 || layer >= c->layers || at < 0 || count < 0 || at + count > c->capacity) return -3;
  cache_write_from(c, layer, at, k, v, count, kv_f16, 0);
  return 0;
}

/* ------------------------------------------------------- cpu/model.js ---- */

int32_t or_argmax(const float* v, int n) {       /* model.js:181-182 */
  int32_t best = 0;
  for (int i = 1; i < n; i++) if (v[i] > v[best]) best = i;
  return best;
}

/* web/perplexity.html:158-166: -log softmax(logits)[target] with the max shift, in doubles,
 * the exps summed in index order. */
double or_nll(const float* logits, int n, int target) {
  double max = -INFINITY;
  for (int i = 0; i < n; i++) if (logits[i] > max) max = logits[i];
  double sum_exp = 0;
  for (int i = 0; i < n; i++) sum_exp += exp((double)logits[i] - max);
  return -((double)logits[target] - max - log(sum_exp));
}

/* model.js:55-166 with the embedded input supplied by the caller. */
int or_forward_hidden(const or_model* m, or_cache* cache, const float* hidden, int seq,
                      float* logits) {
  const or_config* cfg = &m->cfg;
  if (seq <= 0) return -1;
  const int d = cfg->hidden;
  const int hd = cfg->head_dim;
  const int kv_dim = cfg->kv_heads * hd;
  const int ffn = cfg->intermediate;
  /* cache.js:52-60: refuse before anything is written. */
  if (cache->length + seq > cache->capacity) return -3;
  const int past = cache->length;
  const int total = past + seq;

  float* x = (float*)malloc(sizeof(float) * (size_t)seq * d);
  memcpy(x, hidden, sizeof(float) * (size_t)seq * d);
  float* q = (float*)malloc(sizeof(float) * (size_t)seq * d);
  float* k = (float*)malloc(sizeof(float) * (size_t)seq * kv_dim);
  float* v = (float*)malloc(sizeof(float) * (size_t)seq * kv_dim);
  float* attn = (float*)malloc(sizeof(float) * (size_t)seq * d);
  float* scores = (float*)malloc(sizeof(float) * (size_t)total);
  double* inv = (double*)malloc(sizeof(double) * (size_t)(hd / 2));
  or_rope_freqs(hd, cfg->rope_theta, inv);
  /* Positions are independent within each of the three per-position loops below, and every
   * output keeps its own summation order, so running positions on several threads (several
   * positions) or a matvec's rows on several threads (one position) gives the same bits. */
  const int by_position = seq >= 4;

  for (int layer = 0; layer < cfg->layers; layer++) {
    const or_layer* w = &m->layers[layer];
#pragma omp parallel if (by_position)
    {
      float* normed = (float*)malloc(sizeof(float) * d);
#pragma omp for schedule(dynamic)
      for (int t = 0; t < seq; t++) {          /* model.js:96-114 */
        or_rmsnorm(x + (size_t)t * d, w->input_norm, cfg->eps, d, normed);
        or_matvec(w->wq, normed, d, d, w->bq, q + (size_t)t * d);
        or_matvec(w->wk, normed, kv_dim, d, w->bk, k + (size_t)t * kv_dim);
        or_matvec(w->wv, normed, kv_dim, d, w->bv, v + (size_t)t * kv_dim);
        const int position = past + t;
        for (int h = 0; h < cfg->heads; h++) or_rope_inplace(q, t * d + h * hd, hd, position, inv);
        for (int h = 0; h < cfg->kv_heads; h++) or_rope_inplace(k, t * kv_dim + h * hd, hd, position, inv);
      }
      free(normed);
    }
    cache_write(cache, layer, past, k, v, seq, m->kv_f16);   /* model.js:116 */
    or_grouped_attention(q, cache->keys[layer], cache->values[layer], attn, scores, seq, past,
                         cfg->heads, cfg->kv_heads, hd);      /* model.js:121-123 */
#pragma omp parallel if (by_position)
    {
      float* normed = (float*)malloc(sizeof(float) * d);
      float* projected = (float*)malloc(sizeof(float) * d);
      float* gate = (float*)malloc(sizeof(float) * ffn);
      float* up = (float*)malloc(sizeof(float) * ffn);
#pragma omp for schedule(dynamic)
      for (int t = 0; t < seq; t++) {          /* model.js:125-128 */
        or_matvec(w->wo, attn + (size_t)t * d, d, d, NULL, projected);
        float* row = x + (size_t)t * d;
        for (int i = 0; i < d; i++) row[i] = (float)((double)row[i] + (double)projected[i]);
      }
#pragma omp for schedule(dynamic)
      for (int t = 0; t < seq; t++) {          /* model.js:131-140 */
        float* row = x + (size_t)t * d;
        or_rmsnorm(row, w->post_norm, cfg->eps, d, normed);
        or_matvec(w->w_gate, normed, ffn, d, NULL, gate);
        or_matvec(w->w_up, normed, ffn, d, NULL, up);
        or_swiglu(gate, up, ffn);
        or_matvec(w->w_down, gate, d, ffn, NULL, projected);
        for (int i = 0; i < d; i++) row[i] = (float)((double)row[i] + (double)projected[i]);
      }
      free(normed); free(projected); free(gate); free(up);
    }
  }
  cache->length += seq;                        /* model.js:146 */

  if (logits) {                                /* model.js:151-157, 218-228 */
    float* normed = (float*)malloc(sizeof(float) * d);
    or_rmsnorm(x + (size_t)(seq - 1) * d, m->final_norm, cfg->eps, d, normed);
    if (m->lm_head_f32) or_matvec(m->lm_head_f32, normed, cfg->vocab, d, NULL, logits);
    else or_matvec_bf16(m->embed_bf16, normed, cfg->vocab, d, logits);
    free(normed);
  }

  free(x); free(q); free(k); free(v); free(attn); free(scores); free(inv);
  return 0;
}

/* model.js:190-209: ids checked against the vocabulary, rows widened from bf16. */
int or_forward(const or_model* m, or_cache* cache, const int32_t* ids, int seq, float* logits) {
  if (seq <= 0) return -1;
  const int d = m->cfg.hidden;
  for (int t = 0; t < seq; t++) if (ids[t] < 0 || ids[t] >= m->cfg.vocab) return -2;
  float* hidden = (float*)malloc(sizeof(float) * (size_t)seq * d);
  for (int t = 0; t < seq; t++) {
    or_bf16_to_f32_array(m->embed_bf16 + (size_t)ids[t] * d, hidden + (size_t)t * d, (size_t)d);
  }
  int rc = or_forward_hidden(m, cache, hidden, seq, logits);
  free(hidden);
  return rc;
}

/* model.js:174-187: the prompt in one pass, then one token per pass, greedy. */
int or_generate(const or_model* m, or_cache* cache, const int32_t* prompt, int prompt_len,
                int max_tokens, int32_t* tokens) {
  float* logits = (float*)malloc(sizeof(float) * (size_t)m->cfg.vocab);
  const int32_t* next = prompt;
  int len = prompt_len;
  int32_t one = 0;
  int rc = 0;
  for (int step = 0; step < max_tokens; step++) {
    rc = or_forward(m, cache, next, len, logits);
    if (rc) break;
    one = or_argmax(logits, m->cfg.vocab);
    tokens[step] = one;
    next = &one;
    len = 1;
  }
  free(logits);
  return rc;
}
