// Causal GQA attention over an f16 head-major KV cache [kv_heads][capacity][64]
// (device code, shared by the operators and the decode step). Replaces
// ATTENTION (src/gpu/kernels.js:404-499). Query head h reads kv head
// h / (heads/kv_heads), the blocked map of src/core/attention.js:74-76.
//
// Two algorithms:
//
// Exact order (k_attn_scores + k_attn_pv), what the model path uses. It
// evaluates groupedAttention (src/core/attention.js:32-66) step for step:
// each score is a sequential f64 dot stored to f32, the softmax shifts by the
// global max and normalizes with an f64 sum (src/core/ops.js:66-78), and the
// output accumulates sequentially over positions in f32, as the reference's
// Float32Array `out += weight * value` does. Scores and maxima are computed in
// parallel over 64-position chunks; the sequential PV sum runs one lane per
// output element. The result matches the CPU to the bit apart from f64-order
// noise, so a device f16 cache and the CPU's same-f16 cache stay identical.
//
// Split-K online softmax (k_attention_splitk), for long contexts: one block
// per (query, kv head, split of chunks) stages K/V once for all the query heads
// that share it and keeps scores in LDS; the last split to finish combines.
// Exact to f32 rounding, not to the CPU's order; checked within the kernel
// tolerance.
#pragma once

#include "device_common.h"

namespace qh {

constexpr int kChunk = 64;        // positions per chunk
constexpr int kMaxSplits = 128;   // split-K: splits per (query, kv head)
constexpr int kHeadDim = 64;
constexpr int kMaxGroup = 8;      // query heads per kv head
constexpr int kPartialStride = kHeadDim + 2;  // split-K partial: m, l, acc[64]

__host__ __device__ inline int attn_chunks(int ctx) { return (ctx + kChunk - 1) / kChunk; }

// ------------------------------------------------------------ exact order --

struct ExactArgs {
  const float* q;        // [seq][heads*64], rotated
  const uint16_t* kc;    // [kv_heads][capacity][64] f16
  const uint16_t* vc;
  const int* d_pos;      // when set, past is read from the device (decode)
  float* scores;         // [seq][heads][score_stride]; the PV pass overwrites them with p
  float* maxes;          // [seq][heads][max_stride]: per-chunk maxima
  float* out;            // [seq][heads*64]
  int past, capacity, heads, kv_heads, score_stride, max_stride;
};

// grid (chunks, kv_heads, seq): scores of one 64-position chunk for the `group`
// query heads of one kv head, and their per-chunk maxima.
static __global__ __launch_bounds__(kBlock) void k_attn_scores(ExactArgs a) {
  const int c = blockIdx.x, g = blockIdx.y, t = blockIdx.z;
  const int past = a.d_pos ? *a.d_pos : a.past;
  const int pos = past + t;
  if (pos >= a.capacity) return;  // the host keeps positions inside the cache
  const int ctx = pos + 1;
  const int p0 = c * kChunk;
  if (p0 >= ctx) return;
  const int n = min(kChunk, ctx - p0);
  const int group = a.heads / a.kv_heads;
  const int tid = threadIdx.x;

  __shared__ double qs[kMaxGroup][kHeadDim];
  __shared__ __attribute__((aligned(16))) _Float16 ks[kChunk][kHeadDim + 2];
  __shared__ float sc[kMaxGroup][kChunk];
  const float* qrow = a.q + (size_t)t * a.heads * kHeadDim + (size_t)g * group * kHeadDim;
  for (int i = tid; i < group * kHeadDim; i += kBlock) qs[i / kHeadDim][i % kHeadDim] = (double)qrow[i];
  const uint16_t* kbase = a.kc + ((size_t)g * a.capacity + p0) * kHeadDim;
  for (int e = tid; e < n * 8; e += kBlock) {
    const int p = e >> 3, part = e & 7;
    const v4u kv4 = reinterpret_cast<const v4u*>(kbase + (size_t)p * kHeadDim)[part];
#pragma unroll
    for (int k = 0; k < 4; k++) *reinterpret_cast<uint32_t*>(&ks[p][part * 8 + 2 * k]) = kv4[k];
  }
  __syncthreads();
  for (int idx = tid; idx < group * kChunk; idx += kBlock) {
    const int h = idx / kChunk, p = idx % kChunk;
    float s = -INFINITY;
    if (p < n) {
      // dot += q[i] * k[i], i ascending, in f64 (each product is exact).
      double dot = 0.0;
#pragma unroll 8
      for (int j = 0; j < kHeadDim; j += 2) {
        const uint32_t kk = *reinterpret_cast<const uint32_t*>(&ks[p][j]);
        dot = fma(qs[h][j], (double)f16_lo(kk), dot);
        dot = fma(qs[h][j + 1], (double)f16_hi(kk), dot);
      }
      s = (float)(dot * 0.125);  // scale = 1/sqrt(64), exact
      a.scores[((size_t)t * a.heads + g * group + h) * a.score_stride + p0 + p] = s;
    }
    sc[h][p] = s;
  }
  __syncthreads();
  const int wave = tid / kWave, lane = tid & (kWave - 1);
  for (int h = wave; h < group; h += kBlock / kWave) {
    const float m = wave_max(sc[h][lane]);
    if (lane == 0) a.maxes[((size_t)t * a.heads + g * group + h) * a.max_stride + c] = m;
  }
}

// grid (heads, seq): softmax with the global max, then out[d] accumulated
// sequentially over positions in f32 by lane d of wave 0.
static __global__ __launch_bounds__(kBlock) void k_attn_pv(ExactArgs a) {
  const int h = blockIdx.x, t = blockIdx.y;
  const int past = a.d_pos ? *a.d_pos : a.past;
  const int pos = past + t;
  if (pos >= a.capacity) return;
  const int ctx = pos + 1;
  const int g = h / (a.heads / a.kv_heads);
  const int tid = threadIdx.x;
  __shared__ double red[kBlock / kWave];
  __shared__ float mx[kBlock / kWave];

  const size_t row = (size_t)t * a.heads + h;
  float* sc = a.scores + row * a.score_stride;
  // The global max is the max of the chunk maxima (max is order-free).
  const float* cm = a.maxes + row * a.max_stride;
  float m = -INFINITY;
  for (int c = tid; c < attn_chunks(ctx); c += kBlock) m = fmaxf(m, cm[c]);
  m = wave_max(m);
  if ((tid & (kWave - 1)) == 0) mx[tid / kWave] = m;
  __syncthreads();
  const double M = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
  // e = exp(s - max) stored f32; the sum over the unrounded e in f64; p = f32(e32 * (1/sum)).
  double sum = 0.0;
  for (int s = tid; s < ctx; s += kBlock) {
    const double e = exp((double)sc[s] - M);
    sc[s] = (float)e;
    sum += e;
  }
  sum = block_sum_f64(sum, red);
  const double inv = 1.0 / sum;
  for (int s = tid; s < ctx; s += kBlock) sc[s] = (float)((double)sc[s] * inv);
  __syncthreads();
  if (tid >= kWave) return;

  // out[d] += p[s] * v[s][d] for s ascending, rounding to f32 at every step. The
  // product is exact in the fused form, so this is the CPU's f64-sum-then-f32
  // except in double-rounding ties (probability ~2^-29 per step).
  const uint16_t* vb = a.vc + (size_t)g * a.capacity * kHeadDim + tid;
  float o = 0.f;
  constexpr int U = 16;
  int s = 0;
  for (; s + U <= ctx; s += U) {
    float pv[U];
    _Float16 vv[U];
#pragma unroll
    for (int k = 0; k < U; k++) {
      pv[k] = sc[s + k];
      vv[k] = __builtin_bit_cast(_Float16, vb[(size_t)(s + k) * kHeadDim]);
    }
#pragma unroll
    for (int k = 0; k < U; k++) o = fmaf(pv[k], (float)vv[k], o);
  }
  for (; s < ctx; s++) o = fmaf(sc[s], (float)__builtin_bit_cast(_Float16, vb[(size_t)s * kHeadDim]), o);
  a.out[(size_t)t * a.heads * kHeadDim + (size_t)h * kHeadDim + tid] = o;
}

// -------------------------------------------------------------- split-K --

struct SplitArgs {
  const float* q;        // [seq][heads*64], rotated
  const uint16_t* kc;    // [kv_heads][capacity][64] f16
  const uint16_t* vc;
  float* partials;       // [seq][kv_heads][s_grid][group][66]
  int* counters;         // [seq][kv_heads], zero between launches
  float* out;            // [seq][heads*64]
  int past, seq, capacity, heads, kv_heads, s_grid;
};

__host__ __device__ inline void attn_splits(int ctx, int* nchunks, int* cps, int* splits) {
  const int n = attn_chunks(ctx);
  const int s = n < kMaxSplits ? n : kMaxSplits;
  const int c = (n + s - 1) / s;
  *nchunks = n;
  *cps = c;
  *splits = (n + c - 1) / c;
}

// Grid width that covers every query with context <= max_ctx. The split count
// is not monotone in ctx past kMaxSplits chunks (129 chunks need 65 splits, 128
// need 128), so the bound is min(chunks, kMaxSplits), not splits(max_ctx).
__host__ __device__ inline int attn_grid_splits(int max_ctx) {
  const int n = attn_chunks(max_ctx);
  return n < kMaxSplits ? n : kMaxSplits;
}

static __global__ __launch_bounds__(kBlock) void k_attention_splitk(SplitArgs a) {
  const int split = blockIdx.x;
  const int g = blockIdx.y;
  const int t = blockIdx.z;
  const int pos = a.past + t;
  const int ctx = pos + 1;
  int nchunks, cps, nsplit;
  attn_splits(ctx, &nchunks, &cps, &nsplit);
  if (split >= nsplit || nsplit > a.s_grid) return;
  const int c0 = split * cps;
  const int c1 = min(c0 + cps, nchunks);
  const int group = a.heads / a.kv_heads;
  const int tid = threadIdx.x;

  __shared__ float qs[kMaxGroup][kHeadDim];
  __shared__ __attribute__((aligned(16))) _Float16 ks[kChunk][kHeadDim + 2];
  __shared__ __attribute__((aligned(16))) _Float16 vs[kChunk][kHeadDim];
  __shared__ float sc[kMaxGroup][kChunk];
  __shared__ float mst[kMaxGroup], lst[kMaxGroup], alpha[kMaxGroup];
  __shared__ int is_last;

  const size_t qrow = (size_t)t * a.heads * kHeadDim;
  for (int idx = tid; idx < group * kHeadDim; idx += kBlock) {
    qs[idx / kHeadDim][idx % kHeadDim] = a.q[qrow + (size_t)g * group * kHeadDim + idx];
  }
  if (tid < kMaxGroup) {
    mst[tid] = -INFINITY;
    lst[tid] = 0.f;
  }
  float acc0 = 0.f, acc1 = 0.f;  // outputs tid and tid + 256 of [group][64]
  const int o0 = tid, o1 = tid + kBlock;
  __syncthreads();

  const uint16_t* kbase = a.kc + (size_t)g * a.capacity * kHeadDim;
  const uint16_t* vbase = a.vc + (size_t)g * a.capacity * kHeadDim;
  for (int c = c0; c < c1; c++) {
    const int p0 = c * kChunk;
    const int n = min(kChunk, ctx - p0);
    for (int e = tid; e < kChunk * 8; e += kBlock) {
      const int p = e >> 3, part = e & 7;
      v4u kv4 = {0, 0, 0, 0}, vv4 = {0, 0, 0, 0};
      if (p < n) {
        kv4 = reinterpret_cast<const v4u*>(kbase + (size_t)(p0 + p) * kHeadDim)[part];
        vv4 = reinterpret_cast<const v4u*>(vbase + (size_t)(p0 + p) * kHeadDim)[part];
      }
#pragma unroll
      for (int k = 0; k < 4; k++) *reinterpret_cast<uint32_t*>(&ks[p][part * 8 + 2 * k]) = kv4[k];
      *reinterpret_cast<v4u*>(&vs[p][part * 8]) = vv4;
    }
    __syncthreads();
    for (int idx = tid; idx < group * kChunk; idx += kBlock) {
      const int h = idx / kChunk, p = idx % kChunk;
      float s = -INFINITY;
      if (p < n) {
        float d = 0.f;
#pragma unroll 8
        for (int j = 0; j < kHeadDim; j += 2) {
          const uint32_t kk = *reinterpret_cast<const uint32_t*>(&ks[p][j]);
          d = fmaf(qs[h][j], f16_lo(kk), d);
          d = fmaf(qs[h][j + 1], f16_hi(kk), d);
        }
        s = d * 0.125f;
      }
      sc[h][p] = s;
    }
    __syncthreads();
    {
      const int wave = tid / kWave, lane = tid & (kWave - 1);
      for (int h = wave; h < group; h += kBlock / kWave) {
        const float v = sc[h][lane];
        const float m_old = mst[h];
        const float m_new = fmaxf(m_old, wave_max(v));
        const float e = lane < n ? expf(v - m_new) : 0.f;
        const float sum = team_sum<64>(e);
        sc[h][lane] = e;
        if (lane == 0) {
          const float al = expf(m_old - m_new);
          alpha[h] = al;
          lst[h] = lst[h] * al + sum;
          mst[h] = m_new;
        }
      }
    }
    __syncthreads();
    if (o0 < group * kHeadDim) {
      const int h = o0 / kHeadDim, d = o0 % kHeadDim;
      float s = acc0 * alpha[h];
      for (int p = 0; p < n; p++) s = fmaf(sc[h][p], (float)vs[p][d], s);
      acc0 = s;
    }
    if (o1 < group * kHeadDim) {
      const int h = o1 / kHeadDim, d = o1 % kHeadDim;
      float s = acc1 * alpha[h];
      for (int p = 0; p < n; p++) s = fmaf(sc[h][p], (float)vs[p][d], s);
      acc1 = s;
    }
    __syncthreads();
  }

  float* pbase = a.partials + (((size_t)t * a.kv_heads + g) * a.s_grid) * group * kPartialStride;
  {
    float* mine = pbase + (size_t)split * group * kPartialStride;
    if (o0 < group * kHeadDim) {
      const int h = o0 / kHeadDim, d = o0 % kHeadDim;
      mine[h * kPartialStride + 2 + d] = acc0;
      if (d == 0) {
        mine[h * kPartialStride] = mst[h];
        mine[h * kPartialStride + 1] = lst[h];
      }
    }
    if (o1 < group * kHeadDim) {
      const int h = o1 / kHeadDim, d = o1 % kHeadDim;
      mine[h * kPartialStride + 2 + d] = acc1;
      if (d == 0) {
        mine[h * kPartialStride] = mst[h];
        mine[h * kPartialStride + 1] = lst[h];
      }
    }
  }
  __threadfence();
  __syncthreads();
  int* counter = a.counters + (size_t)t * a.kv_heads + g;
  if (tid == 0) is_last = atomicAdd(counter, 1) == nsplit - 1;
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  for (int idx = tid; idx < group * kHeadDim; idx += kBlock) {
    const int h = idx / kHeadDim, d = idx % kHeadDim;
    float M = -INFINITY;
    for (int s = 0; s < nsplit; s++) M = fmaxf(M, pbase[((size_t)s * group + h) * kPartialStride]);
    float L = 0.f, A = 0.f;
    for (int s = 0; s < nsplit; s++) {
      const float* ps = pbase + ((size_t)s * group + h) * kPartialStride;
      const float w = expf(ps[0] - M);
      L = fmaf(w, ps[1], L);
      A = fmaf(w, ps[2 + d], A);
    }
    a.out[qrow + (size_t)(g * group + h) * kHeadDim + d] = A / L;
  }
  if (tid == 0) *counter = 0;
}

}  // namespace qh
