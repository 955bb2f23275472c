// Kernels and launchers for the standalone operator surface: matvec (f32 and
// f16 activations, single and list-driven), rmsnorm, rope, KV append,
// attention (exact order and split-K), swiglu, residual add and argmax. Each
// replaces one WGSL kernel of src/gpu/kernels.js; the decode step
// (decode.hip) is built from the same device building blocks.
#include <algorithm>

#include "attention.h"
#include "device_common.h"

namespace qh {

// ------------------------------------------------------------------ matvec --
// y[b, r] = f32(sum_c W[r, c] x[b, c] + bias[r]) for NB positions per block,
// positions b_base + blockIdx.y*NB .. +NB-1 (launches cover whole tiles only).
// x is staged in LDS as f64 when NB*cols doubles fit, else read as an f64 copy
// from global memory. Teams of TL lanes compute R consecutive rows.
template <int FMT, int R, int NB, int TL, bool X_LDS>
__global__ __launch_bounds__(kBlock) void k_matvec(DMat m, const float* __restrict__ x,
                                                   const double* __restrict__ x64,
                                                   const float* __restrict__ bias,
                                                   float* __restrict__ y, int b_base) {
  extern __shared__ double smem[];
  const int b0 = b_base + blockIdx.y * NB;
  const double* xuse;
  if constexpr (X_LDS) {
    // chunk-transposed per position, so the team's lanes read distinct LDS banks
    const float* xsrc = x + (size_t)b0 * m.cols;
    const XLayout lay = chunk_layout<FMT>(m.nchunks);
    for (int i = threadIdx.x; i < NB * m.cols; i += kBlock) {
      const int b = i / m.cols, j = i - b * m.cols;
      smem[b * m.cols + lay.pos(j)] = (double)xsrc[i];
    }
    __syncthreads();
    xuse = smem;
  } else {
    xuse = x64 + (size_t)b0 * m.cols;
  }
  using T = Teams<TL>;
  const int row0 = (blockIdx.x * T::kTeams + T::team()) * R;
  if (row0 >= m.rows) return;
  int rows[R];
#pragma unroll
  for (int i = 0; i < R; i++) rows[i] = min(row0 + i, m.rows - 1);
  double acc[NB][R];
  mv_team<FMT, R, NB, TL, X_LDS>(m, rows, xuse, m.cols, T::lane(), acc);
  if (T::lane() == 0) {
#pragma unroll
    for (int b = 0; b < NB; b++) {
#pragma unroll
      for (int i = 0; i < R; i++) {
        const int r = row0 + i;
        if (r >= m.rows) break;
        // The CPU's sum starts from the bias (src/core/ops.js:36); the f64 order only.
        const double v = bias ? acc[b][i] + (double)bias[r] : acc[b][i];
        y[(size_t)(b0 + b) * m.rows + r] = (float)v;
      }
    }
  }
}

__global__ void k_widen(const float* __restrict__ x, double* __restrict__ y, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = (double)x[i];
}

constexpr size_t kMatvecLdsBytes = 64 * 1024;

template <int NB>
static bool x_in_lds(const DMat& m) { return (size_t)NB * m.cols * sizeof(double) <= kMatvecLdsBytes; }

// `tiles` whole tiles of NB positions starting at position b_base.
template <int FMT, int NB, int TL>
static hipError_t matvec_tl(hipStream_t s, const DMat& m, const float* x, const double* x64,
                            const float* bias, float* y, int b_base, int tiles) {
  constexpr int R = 2;
  const int rows_per_block = (kBlock / TL) * R;
  const dim3 grid((m.rows + rows_per_block - 1) / rows_per_block, tiles);
  if (x_in_lds<NB>(m)) {
    hipLaunchKernelGGL((k_matvec<FMT, R, NB, TL, true>), grid, dim3(kBlock),
                       (size_t)NB * m.cols * sizeof(double), s, m, x, x64, bias, y, b_base);
  } else {
    hipLaunchKernelGGL((k_matvec<FMT, R, NB, TL, false>), grid, dim3(kBlock), 0, s, m, x, x64,
                       bias, y, b_base);
  }
  return hipGetLastError();
}

template <int FMT, int NB>
static hipError_t matvec_nb(hipStream_t s, const DMat& m, const float* x, const double* x64,
                            const float* bias, float* y, int b_base, int tiles) {
  if (team_width(m.nchunks) == 32) return matvec_tl<FMT, NB, 32>(s, m, x, x64, bias, y, b_base, tiles);
  return matvec_tl<FMT, NB, 64>(s, m, x, x64, bias, y, b_base, tiles);
}

template <int FMT>
static hipError_t matvec_fmt(hipStream_t s, const DMat& m, const float* x, const double* x64,
                             const float* bias, float* y, int seq) {
  // Tiles of 8 positions (src/gpu/model.js:133-138 batchTileFor), then 4, 2 and 1 for the
  // remainder. The tile decides only how many positions share a weight read, never how an
  // output is summed.
  hipError_t e = hipSuccess;
  int done = 0;
  if (seq >= 8) {
    if ((e = matvec_nb<FMT, 8>(s, m, x, x64, bias, y, 0, seq / 8)) != hipSuccess) return e;
    done = seq / 8 * 8;
  }
  if (seq - done >= 4) {
    if ((e = matvec_nb<FMT, 4>(s, m, x, x64, bias, y, done, 1)) != hipSuccess) return e;
    done += 4;
  }
  if (seq - done >= 2) {
    if ((e = matvec_nb<FMT, 2>(s, m, x, x64, bias, y, done, 1)) != hipSuccess) return e;
    done += 2;
  }
  if (seq - done >= 1) e = matvec_nb<FMT, 1>(s, m, x, x64, bias, y, done, 1);
  return e;
}

size_t matvec_x64_bytes(const DMat& m, int seq) {
  // Tiles whose x does not fit in LDS read an f64 copy of all positions.
  const bool any_global = !x_in_lds<1>(m) || (seq >= 2 && !x_in_lds<2>(m)) ||
                          (seq >= 4 && !x_in_lds<4>(m)) || (seq >= 8 && !x_in_lds<8>(m));
  return any_global ? (size_t)seq * m.cols * sizeof(double) : 0;
}

hipError_t launch_matvec(hipStream_t s, const DMat& m, const float* x, const float* bias, float* y,
                         int seq, double* x64_scratch) {
  const size_t need = matvec_x64_bytes(m, seq);
  double* x64 = nullptr;
  hipError_t e = hipSuccess;
  if (need) {
    x64 = x64_scratch;
    if (!x64 && (e = hipMallocAsync((void**)&x64, need, s)) != hipSuccess) return e;
    const size_t n = (size_t)seq * m.cols;
    hipLaunchKernelGGL(k_widen, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, x64, n);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  switch (m.format) {
    case QH_FMT_F16: e = matvec_fmt<QH_FMT_F16>(s, m, x, x64, bias, y, seq); break;
    case QH_FMT_INT8: e = matvec_fmt<QH_FMT_INT8>(s, m, x, x64, bias, y, seq); break;
    default: e = matvec_fmt<QH_FMT_INT4>(s, m, x, x64, bias, y, seq); break;
  }
  if (need && !x64_scratch) {
    const hipError_t f = hipFreeAsync(x64, s);
    if (e == hipSuccess) e = f;
  }
  return e;
}

// ------------------------------------------------------------ f32 matvec --
// The fast-numerics matvec of the batched prefill: y[b, r] = f32 sum of row r with
// position b's x (+ bias), summed by the f32 core exactly as the decode step's
// fused launches sum it, so a prefill tile and the same position decoded alone give
// the same bits. All NB staged positions (values + chunk sums) sit in LDS.
template <int FMT, int R, int NB, int TL>
__global__ __launch_bounds__(kBlock) void k_matvec_f32(DMat m, const float* __restrict__ x,
                                                       const float* __restrict__ bias, float* __restrict__ y,
                                                       int b_base) {
  extern __shared__ double smem[];
  float* xs = reinterpret_cast<float*>(smem);
  const int b0 = b_base + blockIdx.y * NB;
  const int per = staged_f32_floats(m.cols, m.nchunks);
  const XLayoutF lay = chunk_layout_f<FMT>(m.nchunks);
  const int n4 = m.cols >> 2;
  // Groups of the NB positions in order; a chunk's groups are G consecutive lanes
  // (G divides n4 and kBlock), so every position's chunk sums are butterflies inside
  // one wave, and the trip count is the same for every lane.
  for (int base = 0; base < NB * n4; base += kBlock) {
    const int gi = base + threadIdx.x;
    const bool valid = gi < NB * n4;
    const int b = valid ? gi / n4 : 0, g = valid ? gi - b * n4 : 0;
    v4f v = {0.f, 0.f, 0.f, 0.f};
    if (valid) v = reinterpret_cast<const v4f*>(x + (size_t)(b0 + b) * m.cols)[g];
    float* xb = xs + (size_t)b * per;
    stage_group_f32<FMT>(v, g, valid, xb, xb + m.cols, lay);
  }
  __syncthreads();
  using T = Teams<TL>;
  const int row0 = (blockIdx.x * T::kTeams + T::team()) * R;
  if (row0 >= m.rows) return;
  int rows[R];
#pragma unroll
  for (int i = 0; i < R; i++) rows[i] = min(row0 + i, m.rows - 1);
  float acc[NB][R];
  mv_team_f32<FMT, R, NB, TL>(m, rows, xs, per, T::lane(), acc);
  if (T::lane() == 0) {
#pragma unroll
    for (int b = 0; b < NB; b++) {
#pragma unroll
      for (int i = 0; i < R; i++) {
        const int r = row0 + i;
        if (r >= m.rows) break;
        y[(size_t)(b0 + b) * m.rows + r] = bias ? __fadd_rn(acc[b][i], bias[r]) : acc[b][i];
      }
    }
  }
}

template <int NB>
static bool f32_tile_fits(const DMat& m) {
  return (size_t)NB * staged_f32_floats(m.cols, m.nchunks) * sizeof(float) <= kMatvecLdsBytes;
}

template <int FMT, int NB>
static hipError_t matvec_f32_nb(hipStream_t s, const DMat& m, const float* x, const float* bias, float* y,
                                int b_base, int tiles) {
  constexpr int R = 2;
  const size_t lds = (size_t)NB * staged_f32_floats(m.cols, m.nchunks) * sizeof(float);
  if (team_width(m.nchunks) == 32) {
    const dim3 grid((m.rows + (kBlock / 32) * R - 1) / ((kBlock / 32) * R), tiles);
    hipLaunchKernelGGL((k_matvec_f32<FMT, R, NB, 32>), grid, dim3(kBlock), lds, s, m, x, bias, y, b_base);
  } else {
    const dim3 grid((m.rows + (kBlock / 64) * R - 1) / ((kBlock / 64) * R), tiles);
    hipLaunchKernelGGL((k_matvec_f32<FMT, R, NB, 64>), grid, dim3(kBlock), lds, s, m, x, bias, y, b_base);
  }
  return hipGetLastError();
}

template <int FMT>
static hipError_t matvec_f32_fmt(hipStream_t s, const DMat& m, const float* x, const float* bias, float* y,
                                 int seq) {
  // The widest tile of 8, 4, 2 or 1 positions whose staged vectors fit in LDS, then
  // narrower tiles for the remainder.
  hipError_t e = hipSuccess;
  int done = 0;
  if (seq >= 8 && f32_tile_fits<8>(m)) {
    if ((e = matvec_f32_nb<FMT, 8>(s, m, x, bias, y, 0, seq / 8)) != hipSuccess) return e;
    done = seq / 8 * 8;
  }
  if (seq - done >= 4 && f32_tile_fits<4>(m)) {
    const int tiles = (seq - done) / 4;
    if ((e = matvec_f32_nb<FMT, 4>(s, m, x, bias, y, done, tiles)) != hipSuccess) return e;
    done += tiles * 4;
  }
  if (seq - done >= 2 && f32_tile_fits<2>(m)) {
    const int tiles = (seq - done) / 2;
    if ((e = matvec_f32_nb<FMT, 2>(s, m, x, bias, y, done, tiles)) != hipSuccess) return e;
    done += tiles * 2;
  }
  if (seq - done >= 1) e = matvec_f32_nb<FMT, 1>(s, m, x, bias, y, done, seq - done);
  return e;
}

bool matvec_f32_supported(const DMat& m) { return f32_tile_fits<1>(m) && m.cols % 4 == 0; }

hipError_t launch_matvec_f32(hipStream_t s, const DMat& m, const float* x, const float* bias, float* y,
                             int seq) {
  if (!matvec_f32_supported(m)) return hipErrorInvalidValue;
  switch (m.format) {
    case QH_FMT_F16: return matvec_f32_fmt<QH_FMT_F16>(s, m, x, bias, y, seq);
    case QH_FMT_INT8: return matvec_f32_fmt<QH_FMT_INT8>(s, m, x, bias, y, seq);
    default: return matvec_f32_fmt<QH_FMT_INT4>(s, m, x, bias, y, seq);
  }
}

// ------------------------------------------- matvec with an f16 activation --
// The isolated-matvec shape: x f16, int8 weights, one output
// vector per matrix of a list. Codes are widened to exact f16 pairs and
// multiplied with v_dot2_f32_f16: code q becomes the f16 1152+q by a byte
// permute against 0x64 (1024 + the biased byte q+128) and a packed subtract of
// 1152, both exact; accumulation is f32 and the row scale multiplies the sum.
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }

__device__ __forceinline__ float dot8_int8_h(uint32_t u, const half2_t* xp, float acc) {
  const uint32_t t = u ^ 0x80808080u;
  const half2_t bias = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  const half2_t p0 = as_h2(__builtin_amdgcn_perm(0x64646464u, t, 0x04010400u)) + bias;
  const half2_t p1 = as_h2(__builtin_amdgcn_perm(0x64646464u, t, 0x04030402u)) + bias;
  acc = __builtin_amdgcn_fdot2(p0, xp[0], acc, false);
  acc = __builtin_amdgcn_fdot2(p1, xp[1], acc, false);
  return acc;
}

template <int R, int TL>
__global__ __launch_bounds__(kBlock) void k_matvec_xh_list(DMat m, int count, size_t data_stride,
                                                           size_t scale_stride,
                                                           const uint16_t* __restrict__ x,
                                                           size_t x_stride, float* __restrict__ y) {
  using T = Teams<TL>;
  constexpr int kRowsPerBlock = T::kTeams * R;
  const int blocks_per_mat = (m.rows + kRowsPerBlock - 1) / kRowsPerBlock;
  const int mat = blockIdx.x / blocks_per_mat;
  const int rb = blockIdx.x % blocks_per_mat;
  if (mat >= count) return;
  const int row0 = (rb * T::kTeams + T::team()) * R;
  if (row0 >= m.rows) return;
  const uint8_t* data = m.data + (size_t)mat * data_stride;
  const float* scales = m.scales + (size_t)mat * scale_stride;
  const half2_t* xh = reinterpret_cast<const half2_t*>(x + (size_t)mat * x_stride);
  const int tl = T::lane();

  float acc[R];
  const v4u* rp[R];
#pragma unroll
  for (int i = 0; i < R; i++) {
    acc[i] = 0.f;
    rp[i] = reinterpret_cast<const v4u*>(data + (size_t)min(row0 + i, m.rows - 1) * m.row_bytes);
  }
  for (int c = tl; c < m.nchunks; c += TL) {
    v4u w[R];
#pragma unroll
    for (int i = 0; i < R; i++) w[i] = __builtin_nontemporal_load(&rp[i][c]);
    // 16 weights per chunk: x halves 16c .. 16c+15 as 8 pairs.
    half2_t xp[8];
    const v4u xa = reinterpret_cast<const v4u*>(xh)[2 * c];
    const v4u xb = reinterpret_cast<const v4u*>(xh)[2 * c + 1];
    xp[0] = as_h2(xa.x); xp[1] = as_h2(xa.y); xp[2] = as_h2(xa.z); xp[3] = as_h2(xa.w);
    xp[4] = as_h2(xb.x); xp[5] = as_h2(xb.y); xp[6] = as_h2(xb.z); xp[7] = as_h2(xb.w);
#pragma unroll
    for (int i = 0; i < R; i++) {
      acc[i] = dot8_int8_h(w[i].x, xp + 0, acc[i]);
      acc[i] = dot8_int8_h(w[i].y, xp + 2, acc[i]);
      acc[i] = dot8_int8_h(w[i].z, xp + 4, acc[i]);
      acc[i] = dot8_int8_h(w[i].w, xp + 6, acc[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < R; i++) acc[i] = team_sum<TL>(acc[i]);
  if (tl == 0) {
#pragma unroll
    for (int i = 0; i < R; i++) {
      const int r = row0 + i;
      if (r < m.rows) y[(size_t)mat * m.rows + r] = acc[i] * scales[r];
    }
  }
}

hipError_t launch_matvec_xh_list(hipStream_t s, const DMat& m, int count, size_t data_stride,
                                 size_t scale_stride, const uint16_t* x, size_t x_stride,
                                 float* y) {
  constexpr int R = 4;
  const int tl = team_width(m.nchunks);
  const size_t rows_per_block = (size_t)(kBlock / tl) * R;
  const size_t bpm = (m.rows + rows_per_block - 1) / rows_per_block;
  if (tl == 32) {
    hipLaunchKernelGGL((k_matvec_xh_list<R, 32>), dim3(bpm * count), dim3(kBlock), 0, s, m, count,
                       data_stride, scale_stride, x, x_stride, y);
  } else {
    hipLaunchKernelGGL((k_matvec_xh_list<R, 64>), dim3(bpm * count), dim3(kBlock), 0, s, m, count,
                       data_stride, scale_stride, x, x_stride, y);
  }
  return hipGetLastError();
}

// ----------------------------------------------------------------- rmsnorm --
__global__ __launch_bounds__(kBlock) void k_rmsnorm(const float* __restrict__ x,
                                                    const float* __restrict__ gain,
                                                    float* __restrict__ y, int cols, double eps,
                                                    int vec) {
  extern __shared__ double smem[];
  __shared__ double red[kBlock / kWave];
  const size_t base = (size_t)blockIdx.x * cols;
  if (vec) stage_rmsnorm(x + base, gain, eps, cols, smem, red, kPlain);
  else stage_rmsnorm_scalar(x + base, gain, eps, cols, smem, red);
  for (int i = threadIdx.x; i < cols; i += kBlock) y[base + i] = (float)smem[i];
}

// The f32 rmsnorm of the fast decode step's staging, one row per block.
__global__ __launch_bounds__(kBlock) void k_rmsnorm_f32(const float* __restrict__ x,
                                                        const float* __restrict__ gain,
                                                        float* __restrict__ y, int cols, float eps) {
  __shared__ float red[kBlock / kWave];
  const size_t base = (size_t)blockIdx.x * cols;
  StageIn in;
  in.load(x + base, gain, cols);
  const float scale = rms_scale_f32(in, cols, eps, red);
  const int n4 = cols >> 2;
  v4f* y4 = reinterpret_cast<v4f*>(y + base);
#pragma unroll
  for (int j = 0; j < kStageVec; j++) {
    const int i = threadIdx.x + j * kBlock;
    if (i < n4) y4[i] = rms_apply_f32(in.v[j], scale, in.g[j]);
  }
}

hipError_t launch_rmsnorm(hipStream_t s, const float* x, const float* gain, float* y, int rows,
                          int cols, double eps, bool f32) {
  // The vector staging reads float4 groups: every row start and the gain 16-byte aligned.
  const int vec = (cols % 4 == 0) && ((uintptr_t)x % 16 == 0) && ((uintptr_t)gain % 16 == 0) &&
                  ((uintptr_t)y % 16 == 0) && cols <= kStageMax;
  if (f32) {
    if (!vec) return hipErrorInvalidValue;  // model shapes always stage as float4 groups
    hipLaunchKernelGGL(k_rmsnorm_f32, dim3(rows), dim3(kBlock), 0, s, x, gain, y, cols, (float)eps);
  } else {
    hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(kBlock), cols * sizeof(double), s, x, gain, y,
                       cols, eps, vec);
  }
  return hipGetLastError();
}

// -------------------------------------------------------------------- rope --
// One thread per (row, head, pair), from f32 tables, as ROPE (kernels.js:368-389).
__global__ void k_rope(float* __restrict__ v, const float* __restrict__ cos_t,
                       const float* __restrict__ sin_t, int rows, int heads, int head_dim,
                       int base_pos) {
  const int half = head_dim / 2;
  const int per_row = heads * half;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * per_row) return;
  const int row = idx / per_row, within = idx % per_row;
  const int head = within / half, j = within % half;
  const size_t at = (size_t)(base_pos + row) * half + j;
  const float c = cos_t[at], s = sin_t[at];
  const size_t base = (size_t)row * heads * head_dim + (size_t)head * head_dim + j;
  const float lo = v[base], hi = v[base + half];
  v[base] = lo * c - hi * s;
  v[base + half] = hi * c + lo * s;
}

hipError_t launch_rope(hipStream_t s, float* v, const float* cos_t, const float* sin_t, int rows,
                       int heads, int head_dim, int base_pos) {
  const int n = rows * heads * (head_dim / 2);
  hipLaunchKernelGGL(k_rope, dim3((n + 255) / 256), dim3(256), 0, s, v, cos_t, sin_t, rows, heads,
                     head_dim, base_pos);
  return hipGetLastError();
}

// --------------------------------------------------------------- KV append --
// Keys position-major [kv_heads][capacity][64], values dimension-major
// [kv_heads][64][vstride] (the layout attention.h reads).
__global__ void k_kv_append(const float* __restrict__ k, const float* __restrict__ v,
                            uint16_t* __restrict__ kc, uint16_t* __restrict__ vt, int capacity,
                            int kv_heads, int head_dim, int past, int seq) {
  const int kv_dim = kv_heads * head_dim;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= seq * kv_dim) return;
  const int t = idx / kv_dim, e = idx % kv_dim;
  const int h = e / head_dim, d = e % head_dim;
  kc[((size_t)h * capacity + past + t) * head_dim + d] = __builtin_bit_cast(uint16_t, (_Float16)k[idx]);
  vt[((size_t)h * head_dim + d) * value_stride(capacity) + past + t] =
      __builtin_bit_cast(uint16_t, (_Float16)v[idx]);
}

hipError_t launch_kv_append(hipStream_t s, const float* k, const float* v, uint16_t* kc,
                            uint16_t* vt, int capacity, int kv_heads, int head_dim, int past,
                            int seq) {
  const int n = seq * kv_heads * head_dim;
  hipLaunchKernelGGL(k_kv_append, dim3((n + 255) / 256), dim3(256), 0, s, k, v, kc, vt, capacity,
                     kv_heads, head_dim, past, seq);
  return hipGetLastError();
}

// --------------------------------------------------------------- attention --
static int score_stride(int total) { return (total + 3) & ~3; }

size_t attention_exact_floats(int seq, int heads, int past) {
  const int total = past + seq;
  return (size_t)seq * heads * (score_stride(total) + attn_spans(total));
}

hipError_t launch_attention_exact(hipStream_t s, const float* q, const uint16_t* kc,
                                  const uint16_t* vt, int capacity, float* out, int seq, int past,
                                  int heads, int kv_heads, float* scores, int* counters) {
  ExactArgs a{};
  const int total = past + seq;
  a.q = q;
  a.kc = kc;
  a.vt = vt;
  a.scores = scores;
  a.score_stride = score_stride(total);
  a.max_stride = attn_spans(total);
  a.maxes = scores + (size_t)seq * heads * a.score_stride;
  a.counters = counters;
  a.out = out;
  a.past = past;
  a.capacity = capacity;
  a.vstride = value_stride(capacity);
  a.heads = heads;
  a.kv_heads = kv_heads;
  if (total <= kPLds) {
    hipLaunchKernelGGL(k_attn_block, dim3(heads, seq), dim3(kAttnThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL(k_attn_exact, dim3(a.max_stride, heads, seq), dim3(kBlock), 0, s, a);
  }
  return hipGetLastError();
}

// Queries per launch of a long cache's 128 slots: their partials (476 KiB per query at 14
// heads) are merged into the output before the next group reuses them.
constexpr int kSplitkQueryGroup = 64;

size_t attention_partials_floats(int seq, int heads, int capacity) {
  const int rows = decode_attn_long(capacity) ? std::min(seq, kSplitkQueryGroup) : seq;
  return (size_t)rows * heads * decode_attn_slots(capacity) * kPartStride;
}

// The decode step's attention (k_attn_gqa: one block per kv head and slot, the GQA group on
// the f16 matrix cores, so each K/V chunk is read once per kv head), with the slot count the
// capacity chooses, then the slot merge: k_attn_combine for up to kLongCapacity positions,
// k_attn_merge_long past it. Every query's blocks do what a one-query launch at the same
// capacity does, so prefill rows equal decode rows bit for bit.
hipError_t launch_attention_splitk(hipStream_t s, const float* q, const uint16_t* kc,
                                   const uint16_t* vt, int capacity, float* out, int seq, int past,
                                   int heads, int kv_heads, float* partials) {
  SlotArgs a{};
  a.q = q;
  a.kc = kc;
  a.vt = vt;
  a.part = partials;
  a.past = past;
  a.capacity = capacity;
  a.vstride = value_stride(capacity);
  a.heads = heads;
  a.kv_heads = kv_heads;
  if (!decode_attn_long(capacity)) {
    hipError_t e = launch_attn_decode(s, a, seq, 1);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_combine<true>, dim3(heads, seq), dim3(kWave), 0, s, partials, out, past, heads,
                       kDecodeSlots, (size_t)0);
    return hipGetLastError();
  }
  for (int t0 = 0; t0 < seq; t0 += kSplitkQueryGroup) {
    const int n = std::min(kSplitkQueryGroup, seq - t0);
    SlotArgs b = a;
    b.q = q + (size_t)t0 * heads * kHeadDim;
    b.past = past + t0;
    hipError_t e = launch_attn_decode(s, b, n, 1, out + (size_t)t0 * heads * kHeadDim);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t launch_attention_mfma(hipStream_t s, const float* q, const uint16_t* kc, const uint16_t* vt,
                                 int capacity, float* out, int seq, int past, int heads, int kv_heads) {
  FlashArgs a{};
  a.q = q;
  a.kc = kc;
  a.vt = vt;
  a.out = out;
  a.past = past;
  a.seq = seq;
  a.capacity = capacity;
  a.vstride = value_stride(capacity);
  a.heads = heads;
  a.kv_heads = kv_heads;
  return launch_flash_prefill(s, a);
}

// Slots per head and waves per slot of the list operator. Each (cache, kv head) is one block
// of W waves unless the context is long -- a slot of up to 256 32-key steps -- or the list
// too short to give the device ~256 blocks; W gives each wave about eight steps (one wave for
// the 4 steps of 128 positions, up to 8). Measured over >= 512 MiB of caches (14 heads / 2 kv
// heads; GB/s against K/V bytes): 128 positions 1 x 1 4.2 TB/s (4 slots x 1: 2.5), 1024
// 1 x 4 5.1 (4 x 1: 4.1), 4096 1 x 4 5.1 (16 x 1: 3.2), 32768 4 x 8 4.7 (64 x 1: 2.9):
// fewer slots write and re-read fewer partials and merge in fewer terms. With one slot the
// block writes the output itself and the combine launch goes (128 positions: 4.2 -> 5.5).
struct ListPlan {
  int slots, waves;
};
static ListPlan list_plan(int ctx, int count, int kv_heads) {
  const int steps = 2 * attn_chunks(ctx);
  int slots = std::min(kOpSlots, std::max(1, steps / 256));
  while (slots < kOpSlots && slots < steps && (long long)count * kv_heads * slots < 256) slots *= 2;
  slots = slots <= 1 ? 1 : slots <= 4 ? 4 : slots <= 16 ? 16 : kOpSlots;  // the instantiated counts
  const int per = (steps + slots - 1) / slots;
  const int waves = per <= 8 ? 1 : per <= 32 ? 4 : 8;
  return {slots, waves};
}

void attention_list_plan(int ctx, int count, int kv_heads, int* slots, int* waves) {
  const ListPlan p = list_plan(ctx, count, kv_heads);
  *slots = p.slots;
  *waves = p.waves;
}

size_t attention_list_partials_floats(int count, int heads, int kv_heads, int ctx) {
  return (size_t)count * heads * list_plan(ctx, count, kv_heads).slots * kPartStride;
}

// The list runs the GQA-group MFMA form of the slots (one read of each K/V chunk per kv
// head), then the slot combine.
template <int MAXS>
static hipError_t list_t(hipStream_t s, SlotArgs a, int count, int waves, float* out) {
  a.max_slots = MAXS;
  a.list_part = (size_t)a.heads * MAXS * kPartStride;
  if (MAXS == 1) a.out = out;  // a single slot's state is the result: no partials, no combine
  const dim3 grid(a.kv_heads * MAXS, 1, count);
  if (waves == 8) hipLaunchKernelGGL((k_attn_gqa<MAXS, 8>), grid, dim3(8 * kWave), 0, s, a);
  else if (waves == 4) hipLaunchKernelGGL((k_attn_gqa<MAXS, 4>), grid, dim3(4 * kWave), 0, s, a);
  else hipLaunchKernelGGL((k_attn_gqa<MAXS, 1>), grid, dim3(kWave), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || MAXS == 1) return e;
  hipLaunchKernelGGL(k_attn_combine<true>, dim3(a.heads, 1, count), dim3(kWave), 0, s, a.part, out, a.past, a.heads, MAXS,
                     a.list_part);
  return hipGetLastError();
}

hipError_t launch_attention_splitk_list(hipStream_t s, const float* q, const uint16_t* kc, const uint16_t* vt,
                                        size_t list_k, size_t list_v, int count, int capacity, float* out,
                                        int past, int heads, int kv_heads, float* partials) {
  SlotArgs a{};
  a.q = q;
  a.kc = kc;
  a.vt = vt;
  a.part = partials;
  a.past = past;
  a.capacity = capacity;
  a.vstride = value_stride(capacity);
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.list_k = list_k;
  a.list_v = list_v;
  const ListPlan plan = list_plan(past + 1, count, kv_heads);
  switch (plan.slots) {
    case 1: return list_t<1>(s, a, count, plan.waves, out);
    case 4: return list_t<4>(s, a, count, plan.waves, out);
    case 16: return list_t<16>(s, a, count, plan.waves, out);
    default: return list_t<kOpSlots>(s, a, count, plan.waves, out);
  }
}

// ------------------------------------------------------------ swiglu / add --
// gate = silu(gate) * up with the CPU path's f64 evaluation (src/core/ops.js:81-91).
__global__ void k_swiglu(float* __restrict__ gate, const float* __restrict__ up, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const double g = gate[i];
  gate[i] = (float)(g / (1.0 + exp(-g)) * (double)up[i]);
}

__global__ void k_add(float* __restrict__ x, const float* __restrict__ delta, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  x[i] = x[i] + delta[i];
}

hipError_t launch_swiglu(hipStream_t s, float* gate, const float* up, int n) {
  hipLaunchKernelGGL(k_swiglu, dim3((n + 255) / 256), dim3(256), 0, s, gate, up, n);
  return hipGetLastError();
}
hipError_t launch_add(hipStream_t s, float* x, const float* delta, int n) {
  hipLaunchKernelGGL(k_add, dim3((n + 255) / 256), dim3(256), 0, s, x, delta, n);
  return hipGetLastError();
}

// -------------------------------------------------------------------- copy --
// A grid-stride copy: 16-byte vectors (both pointers 16-byte aligned) or bytes.
__global__ void k_copy16(v4u* __restrict__ dst, const v4u* __restrict__ src, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}
__global__ void k_copy8(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

hipError_t launch_copy(hipStream_t s, void* dst, const void* src, size_t bytes) {
  const bool vec = ((uintptr_t)dst % 16 == 0) && ((uintptr_t)src % 16 == 0) && bytes % 16 == 0;
  const size_t n = vec ? bytes / 16 : bytes;
  const unsigned blocks = (unsigned)std::min<size_t>((n + kBlock - 1) / kBlock, 8192);
  if (vec) {
    hipLaunchKernelGGL(k_copy16, dim3(blocks), dim3(kBlock), 0, s, static_cast<v4u*>(dst),
                       static_cast<const v4u*>(src), n);
  } else {
    hipLaunchKernelGGL(k_copy8, dim3(blocks), dim3(kBlock), 0, s, static_cast<uint8_t*>(dst),
                       static_cast<const uint8_t*>(src), n);
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------ argmax --
// Block partials, then the last block's reduction (atomic counter).
constexpr int kArgmaxPerThread = 16;
constexpr int kArgmaxPerBlock = kBlock * kArgmaxPerThread;

__global__ __launch_bounds__(kBlock) void k_argmax(const float* __restrict__ x, int n,
                                                   int* counter, ArgPair* partials,
                                                   int32_t* out) {
  __shared__ ArgPair red[kBlock / kWave];
  __shared__ int is_last;
  float bv = NAN;
  int bi = 0x7fffffff;
  const int start = blockIdx.x * kArgmaxPerBlock;
  const int end = min(start + kArgmaxPerBlock, n);
  for (int e = start + threadIdx.x; e < end; e += kBlock) {
    const float v = x[e];
    if (argmax_better(v, e, bv, bi)) {
      bv = v;
      bi = e;
    }
  }
  argmax_block(bv, bi, red);
  if (threadIdx.x == 0) {
    partials[blockIdx.x] = {bv, bi};
    __threadfence();
    is_last = atomicAdd(counter, 1) == (int)gridDim.x - 1;
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  bv = NAN;
  bi = 0x7fffffff;
  for (int b = threadIdx.x; b < (int)gridDim.x; b += kBlock) {
    const ArgPair p = partials[b];
    if (argmax_better(p.v, p.i, bv, bi)) {
      bv = p.v;
      bi = p.i;
    }
  }
  __syncthreads();
  argmax_block(bv, bi, red);
  if (threadIdx.x == 0) {
    // A NaN at index 0 can never be beaten by the strict '>' scan.
    *out = (x[0] != x[0]) ? 0 : bi;
    *counter = 0;
  }
}

size_t argmax_partials_bytes(int n) {
  const int blocks = (n + kArgmaxPerBlock - 1) / kArgmaxPerBlock;
  return (size_t)blocks * sizeof(ArgPair);
}

hipError_t launch_argmax(hipStream_t s, const float* v, int n, int* counter, void* partials,
                         int32_t* d_out) {
  const int blocks = (n + kArgmaxPerBlock - 1) / kArgmaxPerBlock;
  hipLaunchKernelGGL(k_argmax, dim3(blocks), dim3(kBlock), 0, s, v, n, counter,
                     static_cast<ArgPair*>(partials), d_out);
  return hipGetLastError();
}

// ------------------------------------------------------------ perplexity --
// The negative log-likelihood of *target under one position's logits, as the reference's
// perplexity page computes it (web/perplexity.html:158-166): the largest logit (a NaN is
// skipped, as `>` skips it), the f64 sum of exp(l - max) over the vocabulary, then
// -(l[target] - max - log(sum)). One block of 1024 threads; per-thread strided f64 sums
// combined in a fixed tree, so every run gives the same bits.
constexpr int kNllThreads = 1024;
__global__ __launch_bounds__(kNllThreads) void k_nll(const float* __restrict__ logits, int vocab,
                                                     const int32_t* __restrict__ target, double* __restrict__ out) {
  __shared__ float wmax[kNllThreads / kWave];
  __shared__ double wsum[kNllThreads / kWave];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  float mx = -INFINITY;
  for (int i = tid; i < vocab; i += kNllThreads) {
    const float l = logits[i];
    if (l > mx) mx = l;
  }
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const float o = __shfl_xor(mx, off);
    if (o > mx) mx = o;
  }
  if (lane == 0) wmax[wave] = mx;
  __syncthreads();
  mx = wmax[0];
#pragma unroll
  for (int w = 1; w < kNllThreads / kWave; w++)
    if (wmax[w] > mx) mx = wmax[w];
  const double m = (double)mx;
  double sum = 0.0;
  for (int i = tid; i < vocab; i += kNllThreads) sum += exp((double)logits[i] - m);
  for (int off = kWave / 2; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if (lane == 0) wsum[wave] = sum;
  __syncthreads();
  if (tid == 0) {
    double total = 0.0;
#pragma unroll
    for (int w = 0; w < kNllThreads / kWave; w++) total += wsum[w];
    *out = -((double)logits[*target] - m - log(total));
  }
}

hipError_t launch_nll(hipStream_t s, const float* logits, int vocab, const int32_t* target, double* out) {
  hipLaunchKernelGGL(k_nll, dim3(1), dim3(kNllThreads), 0, s, logits, vocab, target, out);
  return hipGetLastError();
}

}  // namespace qh

namespace qh {

// ------------------------------------------------------------ measurement --
// What bounds a batch-1 decode launch on this device, measured beside the kernels: the
// cost of a launch that does nothing, of one that reads a vector the previous launch
// wrote (every decode launch does), and the rate of a pure streaming read.
__global__ void k_probe_empty() {}

// A dependent launch: each block reads the whole `n`-float vector the previous launch
// wrote and writes its 4 entries of the next.
__global__ __launch_bounds__(kBlock) void k_probe_phase(const float* __restrict__ in, float* __restrict__ out, int n) {
  __shared__ float red[kBlock / kWave];
  float v = 0.f;
  for (int i = threadIdx.x; i < n; i += kBlock) v += in[i];
  v = team_sum<64>(v);
  if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = v;
  __syncthreads();
  const int i = blockIdx.x * 4 + threadIdx.x;
  if (threadIdx.x < 4 && i < n) out[i] = ((red[0] + red[1]) + (red[2] + red[3])) * 1e-3f + (float)threadIdx.x;
}

// Streams n16 16-byte units once (four independent loads in flight per thread per step);
// one word per block is written so the loads are kept.
__global__ __launch_bounds__(kBlock) void k_read_ceiling(const v4u* __restrict__ p, size_t n16, uint32_t* __restrict__ sink) {
  const size_t stride = (size_t)gridDim.x * kBlock;
  uint32_t acc = 0;
  size_t i = (size_t)blockIdx.x * kBlock + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const v4u a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + stride);
    const v4u c = __builtin_nontemporal_load(p + i + 2 * stride), d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= (a.x ^ b.y) ^ (c.z ^ d.w);
  }
  for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(p + i).x;
  acc = __builtin_amdgcn_readfirstlane(acc) ^ (uint32_t)team_sum<64>((float)(acc & 0xffff));
  if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

hipError_t probe_launch_floor(hipStream_t s, int kind, int blocks, int launches, float* buf, float* us_per_launch) {
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
  for (int i = 0; i < launches && e == hipSuccess; i++) {
    if (kind == 0) hipLaunchKernelGGL(k_probe_empty, dim3(blocks), dim3(kBlock), 0, s);
    else hipLaunchKernelGGL(k_probe_phase, dim3(blocks), dim3(kBlock), 0, s, buf + (i & 1) * 4096,
                            buf + ((i + 1) & 1) * 4096, kind == 1 ? 896 : 0);
    e = hipGetLastError();
  }
  const hipError_t ec = hipStreamEndCapture(s, &g);
  if (e == hipSuccess) e = ec;
  if (e == hipSuccess) e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
  if (e == hipSuccess) e = hipGraphLaunch(ge, s);  // warm
  if (e == hipSuccess) e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  const int reps = 10;
  if (e == hipSuccess) e = hipEventRecord(e0, s);
  for (int r = 0; r < reps && e == hipSuccess; r++) e = hipGraphLaunch(ge, s);
  if (e == hipSuccess) e = hipEventRecord(e1, s);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  if (ge) hipGraphExecDestroy(ge);
  if (g) hipGraphDestroy(g);
  if (e == hipSuccess) *us_per_launch = ms * 1e3f / (reps * launches);
  return e;
}

hipError_t read_ceiling(hipStream_t s, const void* p, size_t bytes, int reps, uint32_t* sink, float* ms_per_read) {
  const int blocks = 4096;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  const v4u* v = static_cast<const v4u*>(p);
  hipLaunchKernelGGL(k_read_ceiling, dim3(blocks), dim3(kBlock), 0, s, v, bytes / 16, sink);  // warm
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipEventCreate(&e0);
  if (e == hipSuccess) e = hipEventCreate(&e1);
  if (e == hipSuccess) e = hipEventRecord(e0, s);
  for (int r = 0; r < reps && e == hipSuccess; r++) {
    hipLaunchKernelGGL(k_read_ceiling, dim3(blocks), dim3(kBlock), 0, s, v, bytes / 16, sink);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipEventRecord(e1, s);
  if (e == hipSuccess) e = hipEventSynchronize(e1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  if (e == hipSuccess) *ms_per_read = ms / reps;
  return e;
}

}  // namespace qh
