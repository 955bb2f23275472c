// Device building blocks shared by every kernel: wave64 reductions on DPP and
// ds_swizzle, the 16-byte weight-chunk dot products for the three weight
// formats, the row-team matvec core, and block-level staging helpers.
//
// The matvec core is what both decode and the batched prefill path use, so
// every output row is summed in one order whatever the number of positions:
// lane-sequential over that lane's chunks, then a fixed butterfly across the
// team. That keeps prefill and decode bit-identical, the property the
// reference's batchedMatvec was written to preserve (src/gpu/kernels.js:217-231).
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
// Butterfly sums inside a team of TL lanes (TL = 16, 32 or 64). Steps of 1, 2,
// 4 and 8 lanes use DPP (quad_perm, row_half_mirror, row_mirror), 16 uses
// ds_swizzle, 32 a bpermute. Every lane ends with the same bits.
__device__ __forceinline__ float dpp_quad_xor1(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_quad_xor2(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_half_mirror(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_mirror(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
}
__device__ __forceinline__ float swz_xor16(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}

template <int TL>
__device__ __forceinline__ float team_sum(float v) {
  static_assert(TL == 16 || TL == 32 || TL == 64, "team width");
  v += dpp_quad_xor1(v);
  v += dpp_quad_xor2(v);
  v += dpp_half_mirror(v);
  v += dpp_mirror(v);
  if constexpr (TL >= 32) v += swz_xor16(v);
  if constexpr (TL >= 64) v += __shfl_xor(v, 32);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}
__device__ __forceinline__ double wave_sum_f64(double v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Sum over the block (blockDim.x == kBlock) in f64. `red` is LDS of kBlock/kWave doubles.
// Every thread returns the same value.
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
  v = wave_sum_f64(v);
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
__device__ __forceinline__ float s8(uint32_t u, int byte) {
  return (float)(int8_t)(uint8_t)(u >> (8 * byte));
}
__device__ __forceinline__ float u8(uint32_t u, int byte) {
  return (float)((u >> (8 * byte)) & 0xffu);
}

// acc += sum over the chunk of w[i] * x[i], sequentially in i.
__device__ __forceinline__ float chunk_f16(const v4u w, const float* __restrict__ x, float acc) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; j++) {
    acc = fmaf(f16_lo(u[j]), x[2 * j], acc);
    acc = fmaf(f16_hi(u[j]), x[2 * j + 1], acc);
  }
  return acc;
}
__device__ __forceinline__ float chunk_int8(const v4u w, const float* __restrict__ x, float acc) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; j++) {
#pragma unroll
    for (int b = 0; b < 4; b++) acc = fmaf(s8(u[j], b), x[4 * j + b], acc);
  }
  return acc;
}
// Returns sum over the 32 nibbles of level[i] * x[i] (levels 0..15, low nibble = even index).
__device__ __forceinline__ float chunk_int4(const v4u w, const float* __restrict__ x) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
  float d = 0.f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t lo = u[j] & 0x0F0F0F0Fu;
    const uint32_t hi = (u[j] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      d = fmaf(u8(lo, b), x[8 * j + 2 * b], d);
      d = fmaf(u8(hi, b), x[8 * j + 2 * b + 1], d);
    }
  }
  return d;
}

// ------------------------------------------------------------ matvec core --
// A team of TL lanes computes R consecutive rows starting at row0 for NB
// positions. Lane `tl` handles chunks tl, tl+TL, ... of every row, so the x
// chunk it reads is reused across the R rows. x for position b is at
// xs + b*xstride (LDS or global), and for int4 the per-chunk sums of x at
// xcs + b*cstride. Rows past the end are computed on a clamped row and must
// not be stored. On return every lane of the team holds the R*NB sums; int8
// sums still need the row scale.
template <int FMT, int R, int NB, int TL>
__device__ __forceinline__ void mv_team(const DMat& m, int row0, const float* xs, int xstride,
                                        const float* xcs, int cstride, int tl,
                                        float (&acc)[NB][R]) {
  constexpr int W = Fmt<FMT>::kW;
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int i = 0; i < R; i++) acc[b][i] = 0.f;

  int rr[R];
  const v4u* rp[R];
#pragma unroll
  for (int i = 0; i < R; i++) {
    rr[i] = min(row0 + i, m.rows - 1);
    rp[i] = reinterpret_cast<const v4u*>(m.data + (size_t)rr[i] * m.row_bytes);
  }
  for (int c = tl; c < m.nchunks; c += TL) {
    v4u w[R];
#pragma unroll
    for (int i = 0; i < R; i++) w[i] = __builtin_nontemporal_load(&rp[i][c]);
    if constexpr (FMT == QH_FMT_INT4) {
      const int g = c / m.cpg;
      float s[R], z[R];
#pragma unroll
      for (int i = 0; i < R; i++) {
        s[i] = m.scales[(size_t)rr[i] * m.gpr + g];
        z[i] = m.zeros[(size_t)rr[i] * m.gpr + g];
      }
#pragma unroll
      for (int b = 0; b < NB; b++) {
        const float* xc = xs + (size_t)b * xstride + (size_t)c * W;
        const float xsum = xcs[(size_t)b * cstride + c];
#pragma unroll
        for (int i = 0; i < R; i++) {
          const float d = chunk_int4(w[i], xc);
          acc[b][i] = fmaf(s[i], fmaf(-z[i], xsum, d), acc[b][i]);
        }
      }
    } else {
#pragma unroll
      for (int b = 0; b < NB; b++) {
        const float* xc = xs + (size_t)b * xstride + (size_t)c * W;
#pragma unroll
        for (int i = 0; i < R; i++) {
          if constexpr (FMT == QH_FMT_F16) acc[b][i] = chunk_f16(w[i], xc, acc[b][i]);
          else acc[b][i] = chunk_int8(w[i], xc, acc[b][i]);
        }
      }
    }
  }
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int i = 0; i < R; i++) acc[b][i] = team_sum<TL>(acc[b][i]);
}

// Teams of TL lanes with R rows each, laid over a block of kBlock threads.
template <int TL, int R>
struct TeamMap {
  static constexpr int kTeams = kBlock / TL;
  static constexpr int kRowsPerBlock = kTeams * R;
  __device__ static int team() { return threadIdx.x / TL; }
  __device__ static int lane() { return threadIdx.x & (TL - 1); }
  __device__ static int row0(int block) { return (block * kTeams + team()) * R; }
};

// --------------------------------------------------------- block staging --
// y = x / sqrt(mean(x^2) + eps) * gain into LDS, with the statistic and the
// products in f64 exactly as the reference CPU path evaluates them
// (src/core/ops.js:17-24), so the normalized vector matches it to the bit
// up to the order of the f64 sum.
__device__ __forceinline__ void stage_rmsnorm(const float* __restrict__ x,
                                              const float* __restrict__ gain, double eps, int cols,
                                              float* xs, double* red) {
  double ss = 0;
  for (int i = threadIdx.x; i < cols; i += kBlock) {
    const float v = x[i];
    xs[i] = v;
    ss += (double)v * (double)v;
  }
  ss = block_sum_f64(ss, red);
  const double scale = 1.0 / sqrt(ss / cols + eps);
  for (int i = threadIdx.x; i < cols; i += kBlock) {
    xs[i] = (float)((double)xs[i] * scale * (double)gain[i]);
  }
  __syncthreads();
}

// Per-chunk sums of x (32 columns each), for the int4 zero-point term.
__device__ __forceinline__ void stage_chunk_sums(const float* xs, int cols, float* xcs) {
  const int n = cols / 32;
  for (int c = threadIdx.x; c < n; c += kBlock) {
    float s = 0.f;
#pragma unroll 8
    for (int j = 0; j < 32; j++) s += xs[c * 32 + j];
    xcs[c] = s;
  }
  __syncthreads();
}

__device__ __forceinline__ void stage_copy(const float* __restrict__ x, int n, float* xs) {
  for (int i = threadIdx.x; i < n; i += kBlock) xs[i] = x[i];
  __syncthreads();
}

// Team width of a matrix: 32 lanes when a row has at most 32 chunks, else 64.
// It fixes which chunks a lane sums and the butterfly, so it is a function of
// the shape alone and every path over a given matrix sums in one order.
__host__ __device__ inline int team_width(int nchunks) { return nchunks <= 32 ? 32 : 64; }

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

}  // namespace qh
