// Device building blocks shared by every kernel: wave64 reductions on DPP and
// ds_swizzle, the weight-chunk dot products for the three weight formats, the
// row-team matvec core, and block-level staging helpers.
//
// Arithmetic follows the reference CPU path step for step (src/core/ops.js:
// f32 storage, f64 accumulation). A weight is first dequantized to the f32 the
// reference's loader would hold -- f32(q*scale), f32((level-zero)*scale), or the
// f16 value -- and then multiplied into an f64 accumulator, so the only
// difference from the CPU is the order of an f64 sum (~1e-16 relative), which
// almost never survives the final rounding to f32.
//
// The matvec core is shared by decode and the batched prefill path, so each
// output row is summed in one order whatever the number of positions: lane-
// sequential over that lane's 16-byte chunks, then a fixed butterfly across the
// team. Prefill and decode therefore agree bit for bit, the property the
// reference's batchedMatvec was written to keep (src/gpu/kernels.js:217-231).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "qh_internal.h"

namespace qh {

// 16 bytes of one weight row, loaded with one global_load_dwordx4.
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kBlock = 256;

// ------------------------------------------------------------- reductions --
// Butterflies inside a team of TL lanes (TL = 16, 32 or 64): steps of 1, 2, 4
// and 8 lanes on DPP (quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror), 16 on ds_swizzle, 32 on a bpermute. Each step
// adds a symmetric pair, so every lane ends with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)u, CTRL, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ float swz_xor16(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
__device__ __forceinline__ double swz_xor16(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_swizzle((int)(uint32_t)u, 0x401F);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_swizzle((int)(uint32_t)(u >> 32), 0x401F);
  return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

constexpr int kDppQuadXor1 = 0xB1, kDppQuadXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

template <int TL>
__device__ __forceinline__ float team_sum(float v) {
  static_assert(TL == 16 || TL == 32 || TL == 64, "team width");
  v += dpp32<kDppQuadXor1>(v);
  v += dpp32<kDppQuadXor2>(v);
  v += dpp32<kDppHalfMirror>(v);
  v += dpp32<kDppMirror>(v);
  if constexpr (TL >= 32) v += swz_xor16(v);
  if constexpr (TL >= 64) v += __shfl_xor(v, 32);
  return v;
}

template <int TL>
__device__ __forceinline__ double team_sum(double v) {
  static_assert(TL == 16 || TL == 32 || TL == 64, "team width");
  v += dpp64<kDppQuadXor1>(v);
  v += dpp64<kDppQuadXor2>(v);
  v += dpp64<kDppHalfMirror>(v);
  v += dpp64<kDppMirror>(v);
  if constexpr (TL >= 32) v += swz_xor16(v);
  if constexpr (TL >= 64) v += __shfl_xor(v, 32);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// Sum over the block (blockDim.x == kBlock) in f64. `red` is LDS of kBlock/kWave doubles.
// Every thread returns the same value.
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = team_sum<64>(v);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  double t = 0;
#pragma unroll
  for (int w = 0; w < kBlock / kWave; w++) t += red[w];
  __syncthreads();
  return t;
}

// ------------------------------------------------------------ chunk dots --
template <int FMT> struct Fmt;
template <> struct Fmt<QH_FMT_F16> { static constexpr int kW = 8; };
template <> struct Fmt<QH_FMT_INT8> { static constexpr int kW = 16; };
template <> struct Fmt<QH_FMT_INT4> { static constexpr int kW = 32; };

__device__ __forceinline__ float f16_lo(uint32_t u) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xffffu));
}
__device__ __forceinline__ float f16_hi(uint32_t u) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
}

// acc += sum over one chunk of w[i] * x[i] in f64, sequentially in i, where w[i]
// is the f32 weight the reference loader holds:
//   f16:  the f16 value (exact in f32);
//   int8: f32(q * scale)          (src/core/quantize.js:60-68);
//   int4: f32((level - zero) * scale), low nibble = even index (:134-151).
// Each f32 product here is a single correctly rounded multiply of exact
// operands, which is what the reference's f64 product stored to f32 is.
__device__ __forceinline__ double chunk_f16(const v4u w, const double* __restrict__ x, double acc) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; j++) {
    acc = fma((double)f16_lo(u[j]), x[2 * j], acc);
    acc = fma((double)f16_hi(u[j]), x[2 * j + 1], acc);
  }
  return acc;
}
__device__ __forceinline__ double chunk_int8(const v4u w, const double* __restrict__ x, float s,
                                             double acc) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; j++) {
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const float wf = (float)(int8_t)(uint8_t)(u[j] >> (8 * b)) * s;
      acc = fma((double)wf, x[4 * j + b], acc);
    }
  }
  return acc;
}
__device__ __forceinline__ double chunk_int4(const v4u w, const double* __restrict__ x, float s,
                                             float z, double acc) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; j++) {
#pragma unroll
    for (int n = 0; n < 8; n++) {
      const float wf = ((float)((u[j] >> (4 * n)) & 0xfu) - z) * s;
      acc = fma((double)wf, x[8 * j + n], acc);
    }
  }
  return acc;
}

// ------------------------------------------------------------ matvec core --
// A team of TL lanes computes R rows (row indices in `rows`, each < m.rows) for
// NB positions. Lane `tl` handles chunks tl, tl+TL, ... of every row, so the x
// chunk it reads is reused across the R rows. x for position b is f64 at
// xs + b*xstride (LDS or global). On return every lane of the team holds the
// R*NB f64 sums.
template <int FMT, int R, int NB, int TL>
__device__ __forceinline__ void mv_team(const DMat& m, const int (&rows)[R], const double* xs,
                                        int xstride, int tl, double (&acc)[NB][R]) {
  constexpr int W = Fmt<FMT>::kW;
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int i = 0; i < R; i++) acc[b][i] = 0.0;

  const v4u* rp[R];
#pragma unroll
  for (int i = 0; i < R; i++) rp[i] = reinterpret_cast<const v4u*>(m.data + (size_t)rows[i] * m.row_bytes);
  float srow[R];
  if constexpr (FMT == QH_FMT_INT8) {
#pragma unroll
    for (int i = 0; i < R; i++) srow[i] = m.scales[rows[i]];
  }
  for (int c = tl; c < m.nchunks; c += TL) {
    v4u w[R];
#pragma unroll
    for (int i = 0; i < R; i++) w[i] = __builtin_nontemporal_load(&rp[i][c]);
    float s[R], z[R];
    if constexpr (FMT == QH_FMT_INT4) {
      const int g = c / m.cpg;
#pragma unroll
      for (int i = 0; i < R; i++) {
        s[i] = m.scales[(size_t)rows[i] * m.gpr + g];
        z[i] = m.zeros[(size_t)rows[i] * m.gpr + g];
      }
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const double* xc = xs + (size_t)b * xstride + (size_t)c * W;
#pragma unroll
      for (int i = 0; i < R; i++) {
        if constexpr (FMT == QH_FMT_F16) acc[b][i] = chunk_f16(w[i], xc, acc[b][i]);
        else if constexpr (FMT == QH_FMT_INT8) acc[b][i] = chunk_int8(w[i], xc, srow[i], acc[b][i]);
        else acc[b][i] = chunk_int4(w[i], xc, s[i], z[i], acc[b][i]);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int i = 0; i < R; i++) acc[b][i] = team_sum<TL>(acc[b][i]);
}

// Team width of a matrix: 32 lanes when a row has at most 32 chunks, else 64.
// It fixes which chunks a lane sums and the butterfly, so it is a function of
// the shape alone and every path over a given matrix sums in one order.
__host__ __device__ inline int team_width(int nchunks) { return nchunks <= 32 ? 32 : 64; }

// Teams of TL lanes over a block of kBlock threads.
template <int TL>
struct Teams {
  static constexpr int kTeams = kBlock / TL;
  __device__ static int team() { return threadIdx.x / TL; }
  __device__ static int lane() { return threadIdx.x & (TL - 1); }
};

// --------------------------------------------------------- block staging --
// xs = x / sqrt(mean(x^2) + eps) * gain as f64 values of the f32 result, with
// the statistic and the products in f64 as src/core/ops.js:17-24 evaluates
// them, so the normalized vector is the CPU's up to the order of the f64 sum.
__device__ __forceinline__ void stage_rmsnorm(const float* __restrict__ x,
                                              const float* __restrict__ gain, double eps, int cols,
                                              double* xs, double* red) {
  double ss = 0;
  for (int i = threadIdx.x; i < cols; i += kBlock) {
    const double v = x[i];
    xs[i] = v;
    ss = fma(v, v, ss);  // v*v is exact in f64, so the fused form rounds once like the CPU's
  }
  ss = block_sum_f64(ss, red);
  const double scale = 1.0 / sqrt(ss / cols + eps);
  for (int i = threadIdx.x; i < cols; i += kBlock) {
    xs[i] = (double)(float)(xs[i] * scale * (double)gain[i]);
  }
  __syncthreads();
}

// xs = (double)x for an f32 vector.
__device__ __forceinline__ void stage_copy(const float* __restrict__ x, int n, double* xs) {
  for (int i = threadIdx.x; i < n; i += kBlock) xs[i] = (double)x[i];
  __syncthreads();
}

struct ArgPair {
  float v;
  int i;
};

// (value, index) ordering of the reference's strict '>' argmax scan: a larger
// value wins; equal values go to the lower index; NaN never wins.
__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
  if (v > bv) return true;
  if (v == bv && i < bi) return true;
  if (bv != bv && v == v) return true;  // anything beats a NaN candidate
  if (bv != bv && v != v && i < bi) return true;
  return false;
}

__device__ __forceinline__ void argmax_wave(float& v, int& i) {
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(v, off);
    const int oi = __shfl_xor(i, off);
    if (argmax_better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

// Reduces (v, i) over the block; thread 0 returns the block's best.
__device__ __forceinline__ void argmax_block(float& v, int& i, ArgPair* red) {
  argmax_wave(v, i);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = {v, i};
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kBlock / kWave; w++) {
      if (argmax_better(red[w].v, red[w].i, v, i)) {
        v = red[w].v;
        i = red[w].i;
      }
    }
  }
}

// The reference's rotation (src/core/ops.js:147-159) of the pair (lo, hi) by
// f64 cos/sin, without contracting the products into a fused multiply-add, so
// each product and the difference round separately as they do in JavaScript.
__device__ __forceinline__ void rope_pair(float lo, float hi, double c, double s, float* out_lo,
                                          float* out_hi) {
#pragma clang fp contract(off)
  const double l = lo, h = hi;
  *out_lo = (float)(l * c - h * s);
  *out_hi = (float)(h * c + l * s);
}

}  // namespace qh
