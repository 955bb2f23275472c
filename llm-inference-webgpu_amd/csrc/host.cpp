// Host helpers of the load path: the weight quantizer (the reference's packing
// and scale granularity, so the device kernels consume its arrays verbatim),
// the rope tables, and the seeded synthetic-input generator.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

#include "qh_internal.h"

namespace {

// Math.min / Math.max: NaN propagates and -0 orders below +0.
double js_min(double a, double b) {
  if (std::isnan(a) || std::isnan(b)) return NAN;
  if (a == 0 && b == 0) return (std::signbit(a) || std::signbit(b)) ? -0.0 : 0.0;
  return a < b ? a : b;
}
double js_max(double a, double b) {
  if (std::isnan(a) || std::isnan(b)) return NAN;
  if (a == 0 && b == 0) return (std::signbit(a) && std::signbit(b)) ? -0.0 : 0.0;
  return a > b ? a : b;
}
// A typed-array store of a Number: NaN becomes 0.
int store_int(double v) { return std::isnan(v) ? 0 : (int)v; }

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t fnv1a(const char* s) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (; *s; s++) {
    h ^= (uint8_t)*s;
    h *= 0x100000001b3ull;
  }
  return h;
}

uint64_t stream_key(uint64_t seed, const char* name) { return mix64(fnv1a(name) + kGolden * (seed + 1)); }

// The c-th output of a SplitMix64 stream started at `key`.
uint64_t draw(uint64_t key, uint64_t c) { return mix64(key + kGolden * (c + 1)); }

// Irwin-Hall(12): the sum of 12 uniform u32 over 2^32, minus 6. Integer sum, one exact
// subtraction and one exact power-of-two division: the same bits everywhere.
double irwin_hall(uint64_t key, uint64_t i) {
  uint64_t sum = 0;
  for (uint64_t j = 0; j < 6; j++) {
    const uint64_t r = draw(key, 6 * i + j);
    sum += (r & 0xffffffffull) + (r >> 32);
  }
  const int64_t centred = (int64_t)sum - (int64_t)(6ull << 32);
  return (double)centred / 4294967296.0;
}

uint16_t f32_to_bf16(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0) {
    return (uint16_t)(((u >> 16) | 0x0040u) & 0xffffu);
  }
  const uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)(((u + 0x7fffu + lsb) >> 16) & 0xffffu);
}

}  // namespace

namespace qh {

// src/core/ops.js:99-136: inv_freq = theta^(-2j/headDim); angle = p * inv_freq in f64.
void rope_tables_f64(int head_dim, double theta, int positions, double* cos_t, double* sin_t) {
  const int half = head_dim / 2;
  double inv[4096];
  for (int j = 0; j < half && j < 4096; j++) inv[j] = std::pow(theta, (-2.0 * j) / head_dim);
#pragma omp parallel for schedule(static)
  for (int p = 0; p < positions; p++) {
    for (int j = 0; j < half; j++) {
      const double angle = p * inv[j];
      cos_t[(size_t)p * half + j] = std::cos(angle);
      sin_t[(size_t)p * half + j] = std::sin(angle);
    }
  }
}

}  // namespace qh

using qh::fail;

extern "C" {

// src/core/quantize.js:36-58. The scale is peak/127 in f64, stored f32; codes use the
// inverse of the f64 scale and round half away from zero; an all-zero row keeps scale 0.
int qh_quantize_int8(const float* h_w, int32_t rows, int32_t cols, int8_t* h_q, float* h_scales) {
  QH_CHECK(h_w && h_q && h_scales && rows >= 1 && cols >= 1, QH_ERR_INVALID,
           "quantize_int8 needs a non-empty matrix and outputs");
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; r++) {
    const float* row = h_w + (size_t)r * cols;
    int8_t* q = h_q + (size_t)r * cols;
    double peak = 0;
    for (int c = 0; c < cols; c++) {
      const double m = std::fabs((double)row[c]);
      if (m > peak) peak = m;
    }
    const double scale = peak / 127;
    h_scales[r] = (float)scale;
    std::memset(q, 0, (size_t)cols);
    if (scale == 0) continue;
    const double inverse = 1 / scale;
    for (int c = 0; c < cols; c++) {
      q[c] = (int8_t)store_int(js_max(-127, js_min(127, std::round((double)row[c] * inverse))));
    }
  }
  return QH_OK;
}

// src/core/quantize.js:80-132. Per group: range widened to include 0, scale (hi-lo)/15,
// integer zero point round(-lo/scale) clamped to [0,15], levels clamped after adding the
// zero, two levels per byte with the even flat index in the low nibble.
int qh_quantize_int4(const float* h_w, int32_t rows, int32_t cols, int32_t group, uint8_t* h_q,
                     float* h_scales, float* h_zeros) {
  QH_CHECK(h_w && h_q && h_scales && h_zeros && rows >= 1 && cols >= 1, QH_ERR_INVALID,
           "quantize_int4 needs a non-empty matrix and outputs");
  QH_CHECK(group >= 2, QH_ERR_RANGE, "groupSize must be an integer of at least 2, got %d", group);
  QH_CHECK(cols % group == 0, QH_ERR_RANGE, "groupSize %d does not divide %d columns", group, cols);
  QH_CHECK(cols % 2 == 0, QH_ERR_INVALID, "cols %d must be even to pack two codes per byte", cols);
  const int gpr = cols / group;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; r++) {
    std::memset(h_q + (size_t)r * cols / 2, 0, (size_t)cols / 2);
    for (int g = 0; g < gpr; g++) {
      const size_t base = (size_t)r * cols + (size_t)g * group;
      double lo = INFINITY, hi = -INFINITY;
      for (int i = 0; i < group; i++) {
        const double v = h_w[base + i];
        if (v < lo) lo = v;
        if (v > hi) hi = v;
      }
      lo = js_min(lo, 0);
      hi = js_max(hi, 0);
      const double scale = (hi - lo) / 15;
      const size_t index = (size_t)r * gpr + g;
      h_scales[index] = (float)scale;
      if (scale == 0) {
        h_zeros[index] = 0;
        continue;
      }
      const double zero = js_max(0, js_min(15, std::round(-lo / scale)));
      h_zeros[index] = (float)zero;
      const double inverse = 1 / scale;
      for (int i = 0; i < group; i++) {
        const double level = js_max(0, js_min(15, std::round((double)h_w[base + i] * inverse) + zero));
        const uint32_t code = (uint32_t)store_int(level) & 0xffu;
        const size_t at = base + i;
        uint8_t& byte = h_q[at >> 1];
        byte = (at & 1) == 0 ? (uint8_t)((byte & 0xf0u) | code) : (uint8_t)((byte & 0x0fu) | (code << 4));
      }
    }
  }
  return QH_OK;
}

// src/core/ops.js:99-136: inv_freq = theta^(-2j/headDim), angles and cos/sin in f64, stored f32.
int qh_rope_tables(int32_t head_dim, double theta, int32_t positions, float* h_cos, float* h_sin) {
  QH_CHECK(h_cos && h_sin && head_dim >= 2 && head_dim % 2 == 0 && positions >= 1, QH_ERR_INVALID,
           "rope_tables needs an even head_dim, positions >= 1 and outputs");
  const int half = head_dim / 2;
  QH_CHECK(half <= 4096, QH_ERR_INVALID, "head_dim %d too large", head_dim);
  std::vector<double> c((size_t)positions * half), s((size_t)positions * half);
  qh::rope_tables_f64(head_dim, theta, positions, c.data(), s.data());
  for (size_t i = 0; i < c.size(); i++) {
    h_cos[i] = (float)c[i];
    h_sin[i] = (float)s[i];
  }
  return QH_OK;
}

int qh_synth_f32(uint64_t seed, const char* name, double std_dev, size_t offset, size_t n,
                 float* h_out) {
  QH_CHECK(name && (h_out || !n), QH_ERR_INVALID, "synth needs a stream name and an output");
  const uint64_t key = stream_key(seed, name);
#pragma omp parallel for schedule(static) if (n > (1u << 16))
  for (int64_t i = 0; i < (int64_t)n; i++) {
    h_out[i] = (float)(std_dev * irwin_hall(key, offset + (uint64_t)i));
  }
  return QH_OK;
}

int qh_synth_bf16(uint64_t seed, const char* name, double std_dev, size_t offset, size_t n,
                  uint16_t* h_out) {
  QH_CHECK(name && (h_out || !n), QH_ERR_INVALID, "synth needs a stream name and an output");
  const uint64_t key = stream_key(seed, name);
#pragma omp parallel for schedule(static) if (n > (1u << 16))
  for (int64_t i = 0; i < (int64_t)n; i++) {
    h_out[i] = f32_to_bf16((float)(std_dev * irwin_hall(key, offset + (uint64_t)i)));
  }
  return QH_OK;
}

int qh_synth_tokens(uint64_t seed, const char* name, int32_t vocab, size_t n, int32_t* h_out) {
  QH_CHECK(name && (h_out || !n) && vocab >= 1, QH_ERR_INVALID, "synth_tokens needs vocab >= 1");
  const uint64_t key = stream_key(seed, name);
  for (size_t i = 0; i < n; i++) {
    const uint64_t u = draw(key, i) >> 32;
    h_out[i] = (int32_t)((u * (uint64_t)vocab) >> 32);
  }
  return QH_OK;
}

}  // extern "C"
