// Batched-prefill contraction on the matrix cores: Y[M, N] = X[M, K] . W^T for
// int8 (per-row scale) and int4 (per-group scale and zero point) weights in the
// reference quantizer's layout (src/core/quantize.js:36-151). The reference has no
// GEMM: its prefill reads each weight once per <= 8 positions (batchedMatvec,
// src/gpu/kernels.js:232-290); this is the M = 512 contraction that replaces it.
//
// Arithmetic. A weight code is an exact bf16: int8 q in [-127, 127], int4
// (level - zero) in [-15, 15]. The activation is split into three bf16 terms
// that sum to it exactly (x = t0 + t1 + t2: t0 = bf16(x), t1 = bf16(x - t0),
// t2 = x - t0 - t1, each difference exact in f32 and the last one 8 significant
// bits), and all three go through v_mfma_f32_16x16x32_bf16 into one f32
// accumulator, so every product is exact and only the f32 accumulation rounds. The scale is
// factored out of the code sum: per output column for int8, per 128-column group
// for int4 (the group's partial sum is scaled into the running total). The
// reference's own GPU path accumulates in f32 as well (kernels.js:56-76).
//
// Tiling. A block computes a 64 (positions) x 64 (weight rows) tile with four
// waves of 32 x 32 (2 x 2 MFMA tiles of 16 x 16), stepping K by 32: each step the
// block stages the three activation terms (64 x 32 bf16 each) and the weights,
// widened to bf16 (64 x 32), in LDS rows padded by 16 bytes, while the next
// step's global loads are already in flight in registers. Long K is split over
// gridDim.z; partial tiles are summed in a fixed order by k_gemm_finish.
#include <algorithm>

#include "device_common.h"

namespace qh {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kGM = 64, kGN = 64, kGK = 32;
constexpr int kTerms = 3;       // bf16 terms of an activation
constexpr int kGRow = kGK + 8;  // bf16 per LDS row: 64 bytes + 16 of padding

struct GemmArgs {
  DMat w;                 // int8 | int4, rows = N, cols = K
  const uint16_t* xt;     // bf16 [kTerms][M][K]: the activation's terms
  float* out;             // splits == 1: Y [M][N]; else partials [splits][M][N]
  const float* bias;      // [N] or NULL (splits == 1 only)
  int M, N, K;
  int steps_per_split;    // K steps (of 32) per gridDim.z slice
};

__device__ __forceinline__ uint32_t bf16_bits_rne(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;  // finite inputs
}

// An exact small integer as bf16 bits (|v| < 256): the f32 has no low half.
__device__ __forceinline__ uint32_t small_int_bf16(int v) {
  return __builtin_bit_cast(uint32_t, (float)v) >> 16;
}

// The activation split: t0 = bf16(x), t1 = bf16(x - t0), t2 = bf16(x - t0 - t1) = x - t0 - t1.
__global__ void k_split_bf16(const float* __restrict__ x, uint16_t* __restrict__ t, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float r = x[i];
#pragma unroll
  for (int k = 0; k < kTerms; k++) {
    const uint32_t b = bf16_bits_rne(r);
    t[(size_t)k * n + i] = (uint16_t)b;
    r -= __builtin_bit_cast(float, b << 16);  // exact
  }
}

// Weights of one K step for thread t: row n0 + t/4, columns k0 + 8*(t%4) .. +7,
// as eight bf16 (packed in a v4u), int4 codes offset by the group's zero point.
template <int FMT>
struct WStep {
  uint32_t raw[2];  // int8: 8 codes; int4: raw[0] = 8 nibbles
  float zero;       // int4
};

template <int FMT>
__device__ __forceinline__ void wstep_load(const DMat& w, int n, int k, WStep<FMT>& s) {
  const uint8_t* row = w.data + (size_t)n * w.row_bytes;
  if constexpr (FMT == QH_FMT_INT8) {
    const uint2 v = *reinterpret_cast<const uint2*>(row + k);
    s.raw[0] = v.x;
    s.raw[1] = v.y;
  } else {
    s.raw[0] = *reinterpret_cast<const uint32_t*>(row + k / 2);
    s.zero = w.zeros[(size_t)n * w.gpr + k / (w.cpg * 32)];
  }
}

template <int FMT>
__device__ __forceinline__ v4u wstep_widen(const WStep<FMT>& s) {
  uint32_t b[8];
  if constexpr (FMT == QH_FMT_INT8) {
#pragma unroll
    for (int e = 0; e < 8; e++) b[e] = small_int_bf16((int)(int8_t)(uint8_t)(s.raw[e / 4] >> (8 * (e % 4))));
  } else {
    const int z = (int)s.zero;  // an integer in [0, 15] (src/core/quantize.js:115)
#pragma unroll
    for (int e = 0; e < 8; e++) b[e] = small_int_bf16((int)((s.raw[0] >> (4 * e)) & 0xfu) - z);
  }
  return v4u{b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16)};
}

template <int FMT>
__global__ __launch_bounds__(kBlock) void k_gemm(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[kTerms][kGM][kGRow];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[kGN][kGRow];
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  const int m0 = blockIdx.y * kGM, n0 = blockIdx.x * kGN;
  const int s0 = blockIdx.z * a.steps_per_split;
  const int s1 = min(s0 + a.steps_per_split, a.K / kGK);

  // Staging map: thread t owns row t/4 (of A and of B), columns 8*(t%4) .. +7.
  const int sr = tid >> 2, sc = 8 * (tid & 3);
  const size_t arow = (size_t)min(m0 + sr, a.M - 1) * a.K;  // rows past M: results discarded
  const int brow = min(n0 + sr, a.N - 1);

  // Wave tile: rows wm*32 .. +31, columns wn*32 .. +31 of the block tile.
  const int wm = wave >> 1, wn = wave & 1;
  const int fr = lane & 15, fk = 8 * (lane >> 4);  // fragment row and k offset

  f32x4 grp[2][2];
  double acc[2][2][4];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      grp[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < 4; r++) acc[i][j][r] = 0.0;
    }

  // Column scales of this lane's output columns (int8: one per row of W).
  float cs[2] = {1.f, 1.f};
  if constexpr (FMT == QH_FMT_INT8) {
#pragma unroll
    for (int j = 0; j < 2; j++) cs[j] = a.w.scales[min(n0 + wn * 32 + 16 * j + fr, a.N - 1)];
  }
  // K steps per f32 partial: an int4 group, else 128 columns.
  const int group_steps = FMT == QH_FMT_INT4 ? a.w.cpg : 4;

  const size_t tstride = (size_t)a.M * a.K;  // elements between activation terms
  v4u xa[kTerms];
  WStep<FMT> ws;
  if (s0 < s1) {
    const int k = s0 * kGK + sc;
#pragma unroll
    for (int t = 0; t < kTerms; t++) xa[t] = *reinterpret_cast<const v4u*>(a.xt + t * tstride + arow + k);
    wstep_load<FMT>(a.w, brow, k, ws);
  }
  for (int st = s0; st < s1; st++) {
#pragma unroll
    for (int t = 0; t < kTerms; t++) *reinterpret_cast<v4u*>(&As[t][sr][sc]) = xa[t];
    *reinterpret_cast<v4u*>(&Bs[sr][sc]) = wstep_widen<FMT>(ws);
    __syncthreads();
    if (st + 1 < s1) {  // next step's loads in flight during this step's MFMAs
      const int k = (st + 1) * kGK + sc;
#pragma unroll
      for (int t = 0; t < kTerms; t++) xa[t] = *reinterpret_cast<const v4u*>(a.xt + t * tstride + arow + k);
      wstep_load<FMT>(a.w, brow, k, ws);
    }
    bf16x8 fa[kTerms][2], fb[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
      for (int t = 0; t < kTerms; t++)
        fa[t][i] = *reinterpret_cast<const bf16x8*>(&As[t][wm * 32 + 16 * i + fr][fk]);
      fb[i] = *reinterpret_cast<const bf16x8*>(&Bs[wn * 32 + 16 * i + fr][fk]);
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int t = 0; t < kTerms; t++)
          grp[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fa[t][i], fb[j], grp[i][j], 0, 0, 0);
    if ((st + 1) % group_steps == 0 || st + 1 == s1) {  // fold the f32 partial into the f64 total
      const int g = st / group_steps;
#pragma unroll
      for (int j = 0; j < 2; j++) {
        double sg = 1.0;
        if constexpr (FMT == QH_FMT_INT4) {
          const int n = min(n0 + wn * 32 + 16 * j + fr, a.N - 1);
          sg = a.w.scales[(size_t)n * a.w.gpr + g];
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
#pragma unroll
          for (int r = 0; r < 4; r++) acc[i][j][r] += sg * (double)grp[i][j][r];
          grp[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
    __syncthreads();
  }

  // D fragment: lane holds rows 4*(lane/16) .. +3 of column lane%16 of each tile.
  float* dst = a.out + (size_t)blockIdx.z * a.M * a.N;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int n = n0 + wn * 32 + 16 * j + fr;
    if (n >= a.N) continue;
    const float b = a.bias ? a.bias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wm * 32 + 16 * i + 4 * (lane >> 4) + r;
        if (m < a.M) dst[(size_t)m * a.N + n] = (float)(acc[i][j][r] * (double)cs[j] + (double)b);
      }
    }
  }
}

// Y = sum over splits of the partial tiles (in split order) + bias.
__global__ void k_gemm_finish(const float* __restrict__ part, int splits, const float* __restrict__ bias,
                              float* __restrict__ y, int M, int N) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)M * N;
  if (i >= total) return;
  float v = 0.f;
  for (int s = 0; s < splits; s++) v += part[(size_t)s * total + i];
  y[i] = v + (bias ? bias[i % N] : 0.f);
}

// K steps per split: enough (M/64 x N/64 x splits) tiles to cover the chip twice,
// int4 splits on group boundaries.
static int gemm_steps_per_split(const DMat& w, int M) {
  const int steps = w.cols / kGK;
  const int tiles = ((M + kGM - 1) / kGM) * ((w.rows + kGN - 1) / kGN);
  const int unit = w.format == QH_FMT_INT4 ? w.cpg : 1;
  int splits = (512 + tiles - 1) / tiles;
  splits = std::max(1, std::min(splits, steps / unit));
  int per = (steps + splits - 1) / splits;
  per = (per + unit - 1) / unit * unit;
  return per;
}

// Scratch of one launch over exactly M rows: the activation terms, then the split partials.
static size_t gemm_scratch_bytes(const DMat& w, int M) {
  const size_t split_bytes = (size_t)M * w.cols * kTerms * sizeof(uint16_t);
  const int steps = w.cols / kGK;
  const int per = gemm_steps_per_split(w, M);
  const int splits = (steps + per - 1) / per;
  const size_t part = splits > 1 ? (size_t)splits * M * w.rows * sizeof(float) : 0;
  return ((split_bytes + 255) & ~(size_t)255) + part;
}

// Scratch for every launch of 1..M rows. Not the M-row figure alone: below a 64-row tile
// boundary there are fewer tiles and so more splits, and the partials of a smaller M can
// outgrow M's own (896 x 896: 64 rows take 28 splits, 1792 partial rows; 66 rows take 14,
// 924 partial rows).
size_t matmul_prefill_scratch_bytes(const DMat& w, int M) {
  size_t most = 0;
  for (int m = 1; m <= M; m++) most = std::max(most, gemm_scratch_bytes(w, m));
  return most;
}

hipError_t launch_matmul_prefill(hipStream_t s, const DMat& w, const float* x, const float* bias,
                                 float* y, int M, void* scratch, size_t scratch_bytes) {
  if (M < 1 || gemm_scratch_bytes(w, M) > scratch_bytes) return hipErrorInvalidValue;
  const size_t nx = (size_t)M * w.cols;
  uint16_t* xt = static_cast<uint16_t*>(scratch);
  hipLaunchKernelGGL(k_split_bf16, dim3((unsigned)((nx + 255) / 256)), dim3(256), 0, s, x, xt, nx);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int steps = w.cols / kGK;
  const int per = gemm_steps_per_split(w, M);
  const int splits = (steps + per - 1) / per;
  float* part = reinterpret_cast<float*>(static_cast<char*>(scratch) + ((nx * kTerms * sizeof(uint16_t) + 255) & ~(size_t)255));
  GemmArgs a{};
  a.w = w;
  a.xt = xt;
  a.out = splits > 1 ? part : y;
  a.bias = splits > 1 ? nullptr : bias;
  a.M = M;
  a.N = w.rows;
  a.K = w.cols;
  a.steps_per_split = per;
  const dim3 grid((w.rows + kGN - 1) / kGN, (M + kGM - 1) / kGM, splits);
  if (w.format == QH_FMT_INT8) hipLaunchKernelGGL(k_gemm<QH_FMT_INT8>, grid, dim3(kBlock), 0, s, a);
  else hipLaunchKernelGGL(k_gemm<QH_FMT_INT4>, grid, dim3(kBlock), 0, s, a);
  if ((e = hipGetLastError()) != hipSuccess || splits == 1) return e;
  const size_t total = (size_t)M * w.rows;
  hipLaunchKernelGGL(k_gemm_finish, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, part, splits,
                     bias, y, M, w.rows);
  return hipGetLastError();
}

}  // namespace qh
