// Kernels and launchers for the standalone operator surface: matvec (f32 and
// f16 activations, single and list-driven), rmsnorm, rope, KV append,
// attention, swiglu, residual add and argmax. Each replaces one WGSL kernel of
// src/gpu/kernels.js; the fused decode step (decode.hip) reuses the same
// device building blocks.
#include "attention.h"
#include "device_common.h"

namespace qh {

// ------------------------------------------------------------------ matvec --
// y[b, r] = sum_c W[r, c] x[b, c] (+ bias[r]) for NB positions per block row.
// x (and the int4 chunk sums) staged in LDS when they fit, else x read from
// global memory through the caches.
template <int FMT, int R, int NB, int TL, bool X_LDS>
__global__ __launch_bounds__(kBlock) void k_matvec(DMat m, const float* __restrict__ x,
                                                   const float* __restrict__ bias,
                                                   float* __restrict__ y, int seq) {
  extern __shared__ float smem[];
  const int b0 = blockIdx.y * NB;
  const int nb = min(NB, seq - b0);
  float* xs = smem;                                     // [NB][cols] when X_LDS
  float* xcs = smem + (X_LDS ? NB * m.cols : 0);        // [NB][nchunks] for int4
  const float* xsrc = x + (size_t)b0 * m.cols;
  if constexpr (X_LDS) {
    for (int i = threadIdx.x; i < NB * m.cols; i += kBlock) {
      xs[i] = i < nb * m.cols ? xsrc[i] : 0.f;
    }
    __syncthreads();
  }
  const float* xuse = X_LDS ? xs : xsrc;
  if constexpr (FMT == QH_FMT_INT4) {
    for (int e = threadIdx.x; e < NB * m.nchunks; e += kBlock) {
      const int b = e / m.nchunks, c = e % m.nchunks;
      float s = 0.f;
      if (b < nb) {
        const float* xc = xuse + (size_t)b * m.cols + (size_t)c * 32;
#pragma unroll 8
        for (int j = 0; j < 32; j++) s += xc[j];
      }
      xcs[e] = s;
    }
    __syncthreads();
  }
  // Positions past the end read position 0's x (never stored).
  using TM = TeamMap<TL, R>;
  const int row0 = TM::row0(blockIdx.x);
  if (row0 >= m.rows) return;
  float acc[NB][R];
  if (X_LDS || nb == NB) {
    mv_team<FMT, R, NB, TL>(m, row0, xuse, m.cols, xcs, m.nchunks, TM::lane(), acc);
  } else {
    // Tail tile reading x from global: clamp positions to stay in bounds.
    mv_team<FMT, R, NB, TL>(m, row0, xuse, 0, xcs, 0, TM::lane(), acc);
  }
  if (TM::lane() == 0) {
#pragma unroll
    for (int b = 0; b < NB; b++) {
      if (b >= nb) break;
#pragma unroll
      for (int i = 0; i < R; i++) {
        const int r = row0 + i;
        if (r >= m.rows) break;
        float v = acc[b][i];
        if constexpr (FMT == QH_FMT_INT8) v = v * m.scales[r];
        if (bias) v = v + bias[r];
        y[(size_t)(b0 + b) * m.rows + r] = v;
      }
    }
  }
}

template <int FMT, int NB, int TL>
static hipError_t matvec_tl(hipStream_t s, const DMat& m, const float* x, const float* bias,
                            float* y, int seq) {
  constexpr int R = 2;
  using TM = TeamMap<TL, R>;
  const size_t x_bytes = (size_t)NB * m.cols * sizeof(float);
  const size_t c_bytes = FMT == QH_FMT_INT4 ? (size_t)NB * m.nchunks * sizeof(float) : 0;
  const dim3 grid((m.rows + TM::kRowsPerBlock - 1) / TM::kRowsPerBlock, (seq + NB - 1) / NB);
  if (x_bytes + c_bytes <= 48 * 1024) {
    hipLaunchKernelGGL((k_matvec<FMT, R, NB, TL, true>), grid, dim3(kBlock), x_bytes + c_bytes, s,
                       m, x, bias, y, seq);
  } else {
    hipLaunchKernelGGL((k_matvec<FMT, R, NB, TL, false>), grid, dim3(kBlock), c_bytes, s, m, x,
                       bias, y, seq);
  }
  return hipGetLastError();
}

template <int FMT, int NB>
static hipError_t matvec_nb(hipStream_t s, const DMat& m, const float* x, const float* bias,
                            float* y, int seq) {
  if (team_width(m.nchunks) == 32) return matvec_tl<FMT, NB, 32>(s, m, x, bias, y, seq);
  return matvec_tl<FMT, NB, 64>(s, m, x, bias, y, seq);
}

template <int FMT>
static hipError_t matvec_fmt(hipStream_t s, const DMat& m, const float* x, const float* bias,
                             float* y, int seq) {
  // The position tile of src/gpu/model.js:133-138. It decides only how many
  // positions share a weight read, never how an output is summed.
  if (seq >= 8) return matvec_nb<FMT, 8>(s, m, x, bias, y, seq);
  if (seq >= 4) return matvec_nb<FMT, 4>(s, m, x, bias, y, seq);
  if (seq >= 2) return matvec_nb<FMT, 2>(s, m, x, bias, y, seq);
  return matvec_nb<FMT, 1>(s, m, x, bias, y, seq);
}

hipError_t launch_matvec(hipStream_t s, const DMat& m, const float* x, const float* bias, float* y,
                         int seq) {
  switch (m.format) {
    case QH_FMT_F16: return matvec_fmt<QH_FMT_F16>(s, m, x, bias, y, seq);
    case QH_FMT_INT8: return matvec_fmt<QH_FMT_INT8>(s, m, x, bias, y, seq);
    default: return matvec_fmt<QH_FMT_INT4>(s, m, x, bias, y, seq);
  }
}

// ------------------------------------------- matvec with an f16 activation --
// The isolated-matvec shape: x f16, one output vector per matrix in a list.
// Weights are widened to exact f16 pairs and multiplied with v_dot2_f32_f16:
// int8 code q becomes the f16 1152+q by a byte permute against 0x64 (1024 + the
// biased byte q+128) and a packed subtract of 1152, which is exact; int4 levels
// likewise from 1024+level minus (1024+zero). Accumulation is f32.
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

template <int FMT, int R, int TL>
__global__ __launch_bounds__(kBlock) void k_matvec_xh_list(DMat m, int count, size_t data_stride,
                                                           size_t scale_stride,
                                                           const uint16_t* __restrict__ x,
                                                           size_t x_stride, float* __restrict__ y) {
  using TM = TeamMap<TL, R>;
  const int blocks_per_mat = (m.rows + TM::kRowsPerBlock - 1) / TM::kRowsPerBlock;
  const int mat = blockIdx.x / blocks_per_mat;
  const int rb = blockIdx.x % blocks_per_mat;
  if (mat >= count) return;
  const int row0 = TM::row0(rb);
  if (row0 >= m.rows) return;
  const uint8_t* data = m.data + (size_t)mat * data_stride;
  const float* scales = m.scales + (size_t)mat * scale_stride;
  const half2_t* xh = reinterpret_cast<const half2_t*>(x + (size_t)mat * x_stride);
  const int tl = TM::lane();

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
    static_assert(FMT == QH_FMT_INT8, "f16-activation list matvec is int8");
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
  if (team_width(m.nchunks) == 32) {
    using TM = TeamMap<32, R>;
    const size_t bpm = (m.rows + TM::kRowsPerBlock - 1) / TM::kRowsPerBlock;
    hipLaunchKernelGGL((k_matvec_xh_list<QH_FMT_INT8, R, 32>), dim3(bpm * count), dim3(kBlock), 0,
                       s, m, count, data_stride, scale_stride, x, x_stride, y);
  } else {
    using TM = TeamMap<64, R>;
    const size_t bpm = (m.rows + TM::kRowsPerBlock - 1) / TM::kRowsPerBlock;
    hipLaunchKernelGGL((k_matvec_xh_list<QH_FMT_INT8, R, 64>), dim3(bpm * count), dim3(kBlock), 0,
                       s, m, count, data_stride, scale_stride, x, x_stride, y);
  }
  return hipGetLastError();
}

// ----------------------------------------------------------------- rmsnorm --
__global__ __launch_bounds__(kBlock) void k_rmsnorm(const float* __restrict__ x,
                                                    const float* __restrict__ gain,
                                                    float* __restrict__ y, int cols, double eps) {
  extern __shared__ float smem[];
  __shared__ double red[kBlock / kWave];
  const size_t base = (size_t)blockIdx.x * cols;
  stage_rmsnorm(x + base, gain, eps, cols, smem, red);
  for (int i = threadIdx.x; i < cols; i += kBlock) y[base + i] = smem[i];
}

hipError_t launch_rmsnorm(hipStream_t s, const float* x, const float* gain, float* y, int rows,
                          int cols, double eps) {
  hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(kBlock), cols * sizeof(float), s, x, gain, y,
                     cols, eps);
  return hipGetLastError();
}

// -------------------------------------------------------------------- rope --
// One thread per (row, head, pair), as ROPE (kernels.js:368-389).
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
__global__ void k_kv_append(const float* __restrict__ k, const float* __restrict__ v,
                            uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int capacity,
                            int kv_heads, int head_dim, int past, int seq) {
  const int kv_dim = kv_heads * head_dim;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= seq * kv_dim) return;
  const int t = idx / kv_dim, e = idx % kv_dim;
  const int h = e / head_dim, d = e % head_dim;
  const size_t at = ((size_t)h * capacity + past + t) * head_dim + d;
  kc[at] = __builtin_bit_cast(uint16_t, (_Float16)k[idx]);
  vc[at] = __builtin_bit_cast(uint16_t, (_Float16)v[idx]);
}

hipError_t launch_kv_append(hipStream_t s, const float* k, const float* v, uint16_t* kc,
                            uint16_t* vc, int capacity, int kv_heads, int head_dim, int past,
                            int seq) {
  const int n = seq * kv_heads * head_dim;
  hipLaunchKernelGGL(k_kv_append, dim3((n + 255) / 256), dim3(256), 0, s, k, v, kc, vc, capacity,
                     kv_heads, head_dim, past, seq);
  return hipGetLastError();
}

// --------------------------------------------------------------- attention --
static int attention_grid_splits(int max_ctx) {
  int nchunks, cps, splits;
  attn_splits(max_ctx, &nchunks, &cps, &splits);
  return splits;
}

void attn_splits_host(int ctx, int* nchunks, int* cps, int* splits) {
  attn_splits(ctx, nchunks, cps, splits);
}

size_t attention_partials_floats(int seq, int heads, int kv_heads, int capacity) {
  const int s_grid = attention_grid_splits(capacity);
  return (size_t)seq * kv_heads * s_grid * (heads / kv_heads) * kPartialStride;
}

hipError_t launch_attention(hipStream_t s, const float* q, const uint16_t* kc, const uint16_t* vc,
                            int capacity, float* out, int seq, int past, int heads, int kv_heads,
                            float* partials, int* counters) {
  AttnArgs a{};
  a.q = q;
  a.kc = const_cast<uint16_t*>(kc);
  a.vc = const_cast<uint16_t*>(vc);
  a.partials = partials;
  a.counters = counters;
  a.out = out;
  a.past = past;
  a.seq = seq;
  a.capacity = capacity;
  a.heads = heads;
  a.kv_heads = kv_heads;
  a.s_grid = attention_grid_splits(past + seq);
  hipLaunchKernelGGL((k_attention<false, false>), dim3(a.s_grid, kv_heads, seq), dim3(kBlock), 0,
                     s, a);
  return hipGetLastError();
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

// ------------------------------------------------------------------ argmax --
// Block partials then the last block's reduction (atomic counter). Scratch:
// [counter, pad to 64 B][partials: nblocks x {float value, int index}].
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

size_t argmax_scratch_bytes(int n) {
  const int blocks = (n + kArgmaxPerBlock - 1) / kArgmaxPerBlock;
  return 64 + (size_t)blocks * sizeof(ArgPair);
}

hipError_t launch_argmax(hipStream_t s, const float* v, int n, void* scratch, int32_t* d_out) {
  const int blocks = (n + kArgmaxPerBlock - 1) / kArgmaxPerBlock;
  int* counter = static_cast<int*>(scratch);
  ArgPair* partials = reinterpret_cast<ArgPair*>(static_cast<char*>(scratch) + 64);
  hipLaunchKernelGGL(k_argmax, dim3(blocks), dim3(kBlock), 0, s, v, n, counter, partials, d_out);
  return hipGetLastError();
}

}  // namespace qh
