// The loader's per-tensor conversion (GpuModel.load, src/gpu/model.js:147-207) on the
// device: checkpoint values (bf16 bits, widened exactly, or f32) quantized with the
// reference quantizer's arithmetic (src/core/quantize.js:36-132) or narrowed to f16
// (src/core/dtype.js:81-113). The codes, scales and zero points equal the host
// restatement's (qh_quantize_int8 / qh_quantize_int4 in host.cpp) bit for bit: the same
// f64 expressions -- the peak or the group range, scale = peak/127 or (hi-lo)/15, the
// inverse of the f64 scale, round half away from zero, Math.min/Math.max semantics for
// NaN and signed zeros -- evaluated per element; only the max/min reductions run in
// parallel, and they are order-free (the maximum of a set, NaN skipped as the host's
// `v > peak` skips it).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "qh_internal.h"

namespace qh {

namespace {

constexpr int kQBlock = 256;

__device__ __forceinline__ double js_min(double a, double b) {
  if (a != a || b != b) return NAN;
  if (a == 0 && b == 0) return (signbit(a) || signbit(b)) ? -0.0 : 0.0;
  return a < b ? a : b;
}
__device__ __forceinline__ double js_max(double a, double b) {
  if (a != a || b != b) return NAN;
  if (a == 0 && b == 0) return (signbit(a) && signbit(b)) ? -0.0 : 0.0;
  return a > b ? a : b;
}
// A typed-array store of a Number: NaN becomes 0.
__device__ __forceinline__ int store_int(double v) { return v != v ? 0 : (int)v; }

template <bool BF16>
__device__ __forceinline__ float src_at(const void* src, size_t i) {
  if constexpr (BF16) return __uint_as_float((uint32_t)static_cast<const uint16_t*>(src)[i] << 16);
  else return static_cast<const float*>(src)[i];
}

// The larger of two candidates as `if (v > best) best = v` keeps it: NaN never wins.
__device__ __forceinline__ double keep_max(double best, double v) { return v > best ? v : best; }
__device__ __forceinline__ double keep_min(double best, double v) { return v < best ? v : best; }

template <typename F>
__device__ __forceinline__ double wave_reduce(double v, F f) {
  for (int off = 32; off > 0; off >>= 1) v = f(v, __shfl_xor(v, off));
  return v;
}

// src/core/quantize.js:36-58, one block per row.
template <bool BF16>
__global__ __launch_bounds__(kQBlock) void k_quant_int8(const void* __restrict__ src, int cols,
                                                        int8_t* __restrict__ q, float* __restrict__ scales) {
  __shared__ double red[kQBlock / 64];
  const int r = blockIdx.x;
  const size_t base = (size_t)r * cols;
  double peak = 0;
  for (int c = threadIdx.x; c < cols; c += kQBlock) peak = keep_max(peak, fabs((double)src_at<BF16>(src, base + c)));
  peak = wave_reduce(peak, keep_max);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = peak;
  __syncthreads();
  peak = 0;
  for (int w = 0; w < kQBlock / 64; w++) peak = keep_max(peak, red[w]);
  const double scale = peak / 127;
  if (threadIdx.x == 0) scales[r] = (float)scale;
  const double inverse = 1 / scale;
  for (int c = threadIdx.x; c < cols; c += kQBlock) {
    int8_t code = 0;
    if (scale != 0) {
      code = (int8_t)store_int(js_max(-127, js_min(127, round((double)src_at<BF16>(src, base + c) * inverse))));
    }
    q[base + c] = code;
  }
}

// src/core/quantize.js:80-132, one wave per (row, group); an even group, so the two
// codes of a byte are in the same group: lane l packs elements 2p, 2p+1 of pair p.
template <bool BF16>
__global__ __launch_bounds__(kQBlock) void k_quant_int4(const void* __restrict__ src, int rows, int cols, int group,
                                                        uint8_t* __restrict__ q, float* __restrict__ scales,
                                                        float* __restrict__ zeros) {
  const int gpr = cols / group;
  const size_t item = (size_t)blockIdx.x * (kQBlock / 64) + (threadIdx.x >> 6);
  if (item >= (size_t)rows * gpr) return;
  const int lane = threadIdx.x & 63;
  const size_t base = (item / gpr) * (size_t)cols + (item % gpr) * (size_t)group;
  double lo = INFINITY, hi = -INFINITY;
  for (int i = lane; i < group; i += 64) {
    const double v = src_at<BF16>(src, base + i);
    lo = keep_min(lo, v);
    hi = keep_max(hi, v);
  }
  lo = wave_reduce(lo, keep_min);
  hi = wave_reduce(hi, keep_max);
  lo = js_min(lo, 0);
  hi = js_max(hi, 0);
  const double scale = (hi - lo) / 15;
  const double zero = scale == 0 ? 0.0 : js_max(0, js_min(15, round(-lo / scale)));
  if (lane == 0) {
    scales[item] = (float)scale;
    zeros[item] = (float)zero;
  }
  const double inverse = 1 / scale;
  for (int p = lane; p < group / 2; p += 64) {
    uint32_t code[2] = {0, 0};
    if (scale != 0) {
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const double level =
            js_max(0, js_min(15, round((double)src_at<BF16>(src, base + 2 * p + k) * inverse) + zero));
        code[k] = (uint32_t)store_int(level) & 0xfu;
      }
    }
    q[(base >> 1) + p] = (uint8_t)(code[0] | (code[1] << 4));
  }
}

// ------------------------------------------------------------------ row-per-wave forms
// The kernels above are the general forms. Where a row is a whole number of 16-byte chunks
// (8 bf16 or 4 f32 values) and the buffers are aligned, one wave takes a row: each lane loads
// its chunks (chunk lane + 64k) once into registers, the peak or the group ranges are reduced
// in f32 compare-selects (exact for a maximum or minimum; NaN never taken, as above), and the
// codes come from the held values with the same f64 expressions, written as one store per chunk.

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <bool BF16>
struct Chunk {
  static constexpr int kVals = BF16 ? 8 : 4;
  // Value j (0..kVals-1) of a 16-byte chunk, widened exactly.
  static __device__ __forceinline__ float at(const u32x4& c, int j) {
    const uint32_t w = j < (BF16 ? 2 : 1) ? c.x : j < (BF16 ? 4 : 2) ? c.y : j < (BF16 ? 6 : 3) ? c.z : c.w;
    if constexpr (BF16) return __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
    else return __uint_as_float(w);
  }
};

__device__ __forceinline__ float take_max(float best, float v) { return v > best ? v : best; }
__device__ __forceinline__ float take_min(float best, float v) { return v < best ? v : best; }

// round(t), half away from zero, as an int for |t| < 2^31: the integer part and the exact
// remainder t - trunc(t) decide it.
__device__ __forceinline__ int round_away(double t) {
  const int i = (int)t;
  const double f = t - (double)i;
  return i + (f >= 0.5 ? 1 : 0) - (f <= -0.5 ? 1 : 0);
}

// The code expressions above, restated in integers. Every product t = x * inverse that is not
// NaN is bounded: |x| <= peak gives |t| <= 127 (1 + 2^-51) for int8, and lo <= x <= hi gives
// |t| <= 15 (1 + 2^-51) for int4 (an infinite x makes the scale infinite, the inverse 0 and t
// NaN). So round(t) fits an int, the clamps are integer clamps, and NaN -- of t, or of an int4
// zero point, which is otherwise an integer in [0, 15] -- is the typed-array store's 0.
__device__ __forceinline__ int code_int8(float x, double inverse) {
  const double t = (double)x * inverse;
  if (t != t) return 0;
  return min(max(round_away(t), -127), 127);
}
__device__ __forceinline__ uint32_t code_int4(float x, double inverse, double zero) {
  const double t = (double)x * inverse;
  if (t != t || zero != zero) return 0;
  return (uint32_t)min(max(round_away(t) + (int)zero, 0), 15);
}

// The same codes from an f32 product where that is safe. t32 = x * f32(inverse) differs from
// the f64 product t the expressions above round by at most |t| 2^-23 (the two roundings to f32,
// 2^-24 each relative; f32(inverse) is never subnormal: |x| < 2^128 bounds the scale), and
// |t| <= 16 (int4) or 128 (int8). So wherever t32 lies farther than kSafe from every
// half-integer, t rounds half away from zero to the integer nearest t32; nearer a half-integer,
// and for NaN or an infinite t32, the f64 expression decides. The codes are those of the f64
// expressions bit for bit, at a fraction of their arithmetic.
constexpr float kSafeInt4 = 0x1p-16f;  // > 16 * 2^-23
constexpr float kSafeInt8 = 0x1p-13f;  // > 128 * 2^-23
__device__ __forceinline__ int code_int8_f32(float x, float inv32, double inverse) {
#pragma clang fp contract(off)
  const float t = x * inv32;
  const float r = __builtin_rintf(t);
  if (!(fabsf(t - r) <= 0.5f - kSafeInt8)) return code_int8(x, inverse);
  return (int)fminf(fmaxf(r, -127.f), 127.f);
}
__device__ __forceinline__ uint32_t code_int4_f32(float x, float inv32, double inverse, double zero, float zf) {
#pragma clang fp contract(off)
  const float t = x * inv32;
  const float r = __builtin_rintf(t);
  if (!(fabsf(t - r) <= 0.5f - kSafeInt4)) return code_int4(x, inverse, zero);
  return (uint32_t)fminf(fmaxf(r + zf, 0.f), 15.f);  // r and the zero point are small integers: exact
}

// src/core/quantize.js:36-58, one wave per row, four rows per block; MAXC chunks per lane.
template <bool BF16, int MAXC>
__global__ __launch_bounds__(kQBlock) void k_quant_int8_rows(const void* __restrict__ src, int rows, int cols,
                                                             int8_t* __restrict__ q, float* __restrict__ scales) {
  using C = Chunk<BF16>;
  const int row = blockIdx.x * (kQBlock / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int nchunks = cols / C::kVals;
  const u32x4* in = reinterpret_cast<const u32x4*>(src) + (size_t)row * nchunks;
  u32x4 c[MAXC];
  float peak = 0;
#pragma unroll
  for (int k = 0; k < MAXC; k++) {
    const int ci = lane + 64 * k;
    c[k] = ci < nchunks ? __builtin_nontemporal_load(in + ci) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < C::kVals; j++) peak = take_max(peak, fabsf(C::at(c[k], j)));
  }
  for (int off = 32; off > 0; off >>= 1) peak = take_max(peak, __shfl_xor(peak, off));
  const double scale = (double)peak / 127;
  if (lane == 0) scales[row] = (float)scale;
  const double inverse = 1 / scale;
  const float inv32 = (float)inverse;
  int8_t* out = q + (size_t)row * cols;
#pragma unroll
  for (int k = 0; k < MAXC; k++) {
    const int ci = lane + 64 * k;
    if (ci >= nchunks) break;
    uint32_t w[C::kVals / 4];
#pragma unroll
    for (int j = 0; j < C::kVals; j++) {
      const uint32_t b = scale != 0 ? (uint32_t)(uint8_t)(int8_t)code_int8_f32(C::at(c[k], j), inv32, inverse) : 0u;
      if (j % 4 == 0) w[j / 4] = b;
      else w[j / 4] |= b << (8 * (j % 4));
    }
    if constexpr (BF16) *reinterpret_cast<uint2*>(out + (size_t)ci * 8) = uint2{w[0], w[1]};
    else *reinterpret_cast<uint32_t*>(out + (size_t)ci * 4) = w[0];
  }
}

// src/core/quantize.js:80-132, one wave per row: a group is G = group / chunk-values
// consecutive chunks (G a power of two up to 64), so at step k lanes [G*i, G*i + G) hold group
// (64k + G*i) / G and its range is a segmented reduction over those lanes.
template <bool BF16, int MAXC>
__global__ __launch_bounds__(kQBlock) void k_quant_int4_rows(const void* __restrict__ src, int rows, int cols,
                                                             int G, uint8_t* __restrict__ q,
                                                             float* __restrict__ scales, float* __restrict__ zeros) {
  using C = Chunk<BF16>;
  const int row = blockIdx.x * (kQBlock / 64) + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int nchunks = cols / C::kVals;
  const int gpr = nchunks / G;
  const u32x4* in = reinterpret_cast<const u32x4*>(src) + (size_t)row * nchunks;
  u32x4 c[MAXC];
#pragma unroll
  for (int k = 0; k < MAXC; k++) {
    const int ci = lane + 64 * k;
    c[k] = ci < nchunks ? __builtin_nontemporal_load(in + ci) : u32x4{0, 0, 0, 0};
  }
  uint8_t* out = q + (size_t)row * (cols / 2);
  if (MAXC <= 4 && gpr <= 64) {
    // A row of at most 64 groups and 4 chunks per lane: each group's f64 parameters (the
    // divisions and Math.min / Math.max of src/core/quantize.js:95-104) are worked out once,
    // by lane g for group g, not by each of the group's G lanes at every step, and handed back
    // by shuffles (with more chunks per lane, the held ranges and shuffles cost more than the
    // divisions they save: 4864-column rows ran 29% -> 19% of HBM).
    const int steps = (nchunks + 63) / 64, per = 64 / G;  // groups per step: segment s of step k is group k*per + s
    float los[MAXC], his[MAXC];
#pragma unroll
    for (int k = 0; k < MAXC; k++) {
      float lo = INFINITY, hi = -INFINITY;
      if (k < steps) {  // wave-uniform: the segmented reduction needs every lane
#pragma unroll
        for (int j = 0; j < C::kVals; j++) {
          const float v = C::at(c[k], j);
          lo = take_min(lo, v);
          hi = take_max(hi, v);
        }
        for (int off = 1; off < G; off <<= 1) {
          lo = take_min(lo, __shfl_xor(lo, off));
          hi = take_max(hi, __shfl_xor(hi, off));
        }
      }
      los[k] = lo;
      his[k] = hi;
    }
    // Lane g collects group g's range (segment g % per of step g / per).
    float glo = INFINITY, ghi = -INFINITY;
#pragma unroll
    for (int k = 0; k < MAXC; k++) {
      if (k >= steps) break;
      const float a = __shfl(los[k], (lane % per) * G), b = __shfl(his[k], (lane % per) * G);
      if (k == lane / per) {
        glo = a;
        ghi = b;
      }
    }
    double ginverse = 0;
    float gzero = -1.f;  // -1: a zero scale, whose codes are 0
    if (lane < gpr) {
      const double dlo = js_min(glo, 0), dhi = js_max(ghi, 0);
      const double scale = (dhi - dlo) / 15;
      const double zero = scale == 0 ? 0.0 : js_max(0, js_min(15, round(-dlo / scale)));
      scales[(size_t)row * gpr + lane] = (float)scale;
      zeros[(size_t)row * gpr + lane] = (float)zero;
      ginverse = 1 / scale;
      if (scale != 0) gzero = (float)zero;  // an integer in [0, 15], or NaN
    }
#pragma unroll
    for (int k = 0; k < MAXC; k++) {
      if (k >= steps) break;
      const int ci = lane + 64 * k, owner = min(ci / G, gpr - 1);  // the chunk's group (clamped past the row)
      const double inverse = __shfl(ginverse, owner);
      const float zf = __shfl(gzero, owner);
      if (ci >= nchunks || zf == -1.f) {
        if (ci < nchunks) {
          if constexpr (BF16) *reinterpret_cast<uint32_t*>(out + (size_t)ci * 4) = 0u;
          else *reinterpret_cast<uint16_t*>(out + (size_t)ci * 2) = (uint16_t)0;
        }
        continue;
      }
      const float inv32 = (float)inverse;
      uint32_t w = 0;
#pragma unroll
      for (int j = 0; j < C::kVals; j++) w |= code_int4_f32(C::at(c[k], j), inv32, inverse, (double)zf, zf) << (4 * j);
      if constexpr (BF16) *reinterpret_cast<uint32_t*>(out + (size_t)ci * 4) = w;
      else *reinterpret_cast<uint16_t*>(out + (size_t)ci * 2) = (uint16_t)w;
    }
    return;
  }
#pragma unroll
  for (int k = 0; k < MAXC; k++) {
    const int ci = lane + 64 * k;
    if (64 * k >= nchunks) break;   // wave-uniform: the segmented reduction needs every lane
    float lo = INFINITY, hi = -INFINITY;
#pragma unroll
    for (int j = 0; j < C::kVals; j++) {
      const float v = C::at(c[k], j);
      lo = take_min(lo, v);
      hi = take_max(hi, v);
    }
    for (int off = 1; off < G; off <<= 1) {
      lo = take_min(lo, __shfl_xor(lo, off));
      hi = take_max(hi, __shfl_xor(hi, off));
    }
    if (ci >= nchunks) continue;
    const double dlo = js_min(lo, 0), dhi = js_max(hi, 0);
    const double scale = (dhi - dlo) / 15;
    const double zero = scale == 0 ? 0.0 : js_max(0, js_min(15, round(-dlo / scale)));
    if ((lane & (G - 1)) == 0) {
      const size_t gi = (size_t)row * gpr + ci / G;
      scales[gi] = (float)scale;
      zeros[gi] = (float)zero;
    }
    const double inverse = 1 / scale;
    const float inv32 = (float)inverse, zf = (float)zero;
    uint32_t w = 0;
    if (scale != 0) {
#pragma unroll
      for (int j = 0; j < C::kVals; j++) w |= code_int4_f32(C::at(c[k], j), inv32, inverse, zero, zf) << (4 * j);
    }
    if constexpr (BF16) *reinterpret_cast<uint32_t*>(out + (size_t)ci * 4) = w;
    else *reinterpret_cast<uint16_t*>(out + (size_t)ci * 2) = (uint16_t)w;
  }
}

// src/core/dtype.js:81-113: round to nearest even with gradual underflow and overflow to
// infinity, which the hardware conversion does for every number; a NaN keeps its sign and the
// top ten payload bits with the quiet bit set (dtype.js:88-90).
__device__ __forceinline__ uint16_t narrow_f16(float x) {
  const uint32_t u = __float_as_uint(x);
  return x != x ? (uint16_t)(((u >> 16) & 0x8000u) | 0x7c00u | ((u & 0x7fffffu) >> 13) | 0x200u)
                : __builtin_bit_cast(uint16_t, (_Float16)x);
}

template <bool BF16>
__global__ void k_to_f16(const void* __restrict__ src, size_t n, uint16_t* __restrict__ out) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = narrow_f16(src_at<BF16>(src, i));
}

template <bool BF16>
__global__ void k_to_f32(const void* __restrict__ src, size_t n, float* __restrict__ out) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = src_at<BF16>(src, i);
}

// Eight values per thread with 16-byte accesses; the n % 8 tail by the first threads.
template <bool BF16, bool F16>
__global__ __launch_bounds__(kQBlock) void k_widen_narrow8(const void* __restrict__ src, size_t n,
                                                           void* __restrict__ out) {
  const size_t n8 = n / 8;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += (size_t)gridDim.x * blockDim.x) {
    float v[8];
    if constexpr (BF16) {
      const u32x4 c = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + i);
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = Chunk<true>::at(c, j);
    } else {
      const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + 2 * i);
      const u32x4 b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + 2 * i + 1);
#pragma unroll
      for (int j = 0; j < 4; j++) v[j] = Chunk<false>::at(a, j), v[4 + j] = Chunk<false>::at(b, j);
    }
    if constexpr (F16) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; j++) w[j] = (uint32_t)narrow_f16(v[2 * j]) | ((uint32_t)narrow_f16(v[2 * j + 1]) << 16);
      reinterpret_cast<u32x4*>(out)[i] = u32x4{w[0], w[1], w[2], w[3]};
    } else {
      float4* o = reinterpret_cast<float4*>(out) + 2 * i;
      o[0] = float4{v[0], v[1], v[2], v[3]};
      o[1] = float4{v[4], v[5], v[6], v[7]};
    }
  }
  const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t < n - n8 * 8) {
    const float x = src_at<BF16>(src, n8 * 8 + t);
    if constexpr (F16) static_cast<uint16_t*>(out)[n8 * 8 + t] = narrow_f16(x);
    else static_cast<float*>(out)[n8 * 8 + t] = x;
  }
}

unsigned grid_for(size_t n) { return (unsigned)std::min<size_t>((n + kQBlock - 1) / kQBlock, 16384); }

bool aligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

// Chunks per lane of the row-per-wave kernels for `nchunks` chunks a row; 0 when too many.
int chunks_per_lane(int nchunks) {
  const int per = (nchunks + 63) / 64;
  return per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : per <= 16 ? 16 : 0;
}

template <bool BF16, int MAXC>
void launch_int8_rows(hipStream_t s, const void* src, int rows, int cols, int8_t* q, float* scales) {
  hipLaunchKernelGGL((k_quant_int8_rows<BF16, MAXC>), dim3((rows + 3) / 4), dim3(kQBlock), 0, s, src, rows, cols, q,
                     scales);
}
template <bool BF16, int MAXC>
void launch_int4_rows(hipStream_t s, const void* src, int rows, int cols, int G, uint8_t* q, float* scales,
                      float* zeros) {
  hipLaunchKernelGGL((k_quant_int4_rows<BF16, MAXC>), dim3((rows + 3) / 4), dim3(kQBlock), 0, s, src, rows, cols, G,
                     q, scales, zeros);
}

template <bool BF16>
hipError_t convert_t(hipStream_t s, const void* src, int rows, int cols, int format, int group, void* data,
                     float* scales, float* zeros) {
  const size_t n = (size_t)rows * cols;
  constexpr int kVals = Chunk<BF16>::kVals;
  const int nchunks = cols / kVals;
  const bool rows_vec = cols % kVals == 0 && aligned(src, 16);
  const int maxc = rows_vec ? chunks_per_lane(nchunks) : 0;
  switch (format) {
    case QH_FMT_F32:
    case QH_FMT_F16: {
      const bool f16 = format == QH_FMT_F16;
      if (aligned(src, 16) && aligned(data, 16)) {
        const unsigned grid = (unsigned)std::min<size_t>(std::max<size_t>((n / 8 + kQBlock - 1) / kQBlock, 1), 16384);
        if (f16) hipLaunchKernelGGL((k_widen_narrow8<BF16, true>), dim3(grid), dim3(kQBlock), 0, s, src, n, data);
        else hipLaunchKernelGGL((k_widen_narrow8<BF16, false>), dim3(grid), dim3(kQBlock), 0, s, src, n, data);
      } else if (f16) {
        hipLaunchKernelGGL(k_to_f16<BF16>, dim3(grid_for(n)), dim3(kQBlock), 0, s, src, n,
                           static_cast<uint16_t*>(data));
      } else {
        hipLaunchKernelGGL(k_to_f32<BF16>, dim3(grid_for(n)), dim3(kQBlock), 0, s, src, n, static_cast<float*>(data));
      }
      break;
    }
    case QH_FMT_INT8: {
      int8_t* q = static_cast<int8_t*>(data);
      if (maxc && aligned(data, BF16 ? 8 : 4)) {
        if (maxc == 2) launch_int8_rows<BF16, 2>(s, src, rows, cols, q, scales);
        else if (maxc == 4) launch_int8_rows<BF16, 4>(s, src, rows, cols, q, scales);
        else if (maxc == 8) launch_int8_rows<BF16, 8>(s, src, rows, cols, q, scales);
        else launch_int8_rows<BF16, 16>(s, src, rows, cols, q, scales);
      } else {
        hipLaunchKernelGGL(k_quant_int8<BF16>, dim3(rows), dim3(kQBlock), 0, s, src, cols, q, scales);
      }
      break;
    }
    case QH_FMT_INT4: {
      uint8_t* q = static_cast<uint8_t*>(data);
      const int G = group / kVals;
      if (maxc && group % kVals == 0 && G <= 64 && (G & (G - 1)) == 0 && aligned(data, BF16 ? 4 : 2)) {
        if (maxc == 2) launch_int4_rows<BF16, 2>(s, src, rows, cols, G, q, scales, zeros);
        else if (maxc == 4) launch_int4_rows<BF16, 4>(s, src, rows, cols, G, q, scales, zeros);
        else if (maxc == 8) launch_int4_rows<BF16, 8>(s, src, rows, cols, G, q, scales, zeros);
        else launch_int4_rows<BF16, 16>(s, src, rows, cols, G, q, scales, zeros);
      } else {
        const size_t items = (size_t)rows * (cols / group);
        hipLaunchKernelGGL(k_quant_int4<BF16>, dim3((unsigned)((items + 3) / 4)), dim3(kQBlock), 0, s, src, rows,
                           cols, group, q, scales, zeros);
      }
      break;
    }
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_convert(hipStream_t s, bool bf16, const void* src, int rows, int cols, int format, int group,
                          void* data, float* scales, float* zeros) {
  return bf16 ? convert_t<true>(s, src, rows, cols, format, group, data, scales, zeros)
              : convert_t<false>(s, src, rows, cols, format, group, data, scales, zeros);
}

}  // namespace qh
