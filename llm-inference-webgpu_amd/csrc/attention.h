// Causal GQA attention over an f16 KV cache (device code, shared by the
// operators and the decode step). Replaces ATTENTION (src/gpu/kernels.js:
// 404-499). Query head h reads kv head h / (heads/kv_heads), the blocked map of
// src/core/attention.js:74-76.
//
// Cache layout, per kv head: keys position-major [capacity][64] (a position's
// key is one 128-byte row, read whole by the lane that scores it) and values
// dimension-major [64][vstride] with vstride = capacity rounded up to 8 (one
// dimension's values over positions are contiguous, so the lane that owns
// output dimension d reads 8 positions in one 16-byte load).
//
// Two algorithms:
//
// Exact order (k_attn_block up to kPLds positions, k_attn_exact beyond), what
// the model path uses. It evaluates groupedAttention (src/core/attention.js:
// 32-66) step for step: each score is a sequential f64 dot stored to f32, the
// softmax shifts by the global max and normalizes with an f64 sum
// (src/core/ops.js:66-78), and the output accumulates sequentially over
// positions in f32, as the reference's Float32Array `out += weight * value`
// does, one lane per output dimension. k_attn_block does a (query, head) in one
// 1024-thread block; k_attn_exact scores 256 positions per block and the last
// block of a (query, head) to finish does the softmax and the PV sum. The
// result matches the CPU to the bit apart from f64-order noise, so a device f16
// cache and the CPU's same-f16 cache stay identical.
//
// Split-K online softmax (k_attention_splitk), for long contexts: one block
// per (query, kv head, split of chunks) stages K/V once for all the query heads
// that share it and keeps scores in LDS; the last split to finish combines.
// Exact to f32 rounding, not to the CPU's order; checked within the kernel
// tolerance.
#pragma once

#include "device_common.h"

namespace qh {

constexpr int kChunk = 64;        // split-K: positions per chunk
constexpr int kMaxSplits = 128;   // split-K: splits per (query, kv head)
constexpr int kHeadDim = 64;
constexpr int kMaxGroup = 8;      // query heads per kv head
constexpr int kPartialStride = kHeadDim + 2;  // split-K partial: m, l, acc[64]
constexpr int kPLds = 4096;       // exact: probabilities kept in LDS up to this context
static_assert(kSpan == kBlock, "exact attention scores one position per thread");

__host__ __device__ inline int attn_chunks(int ctx) { return (ctx + kChunk - 1) / kChunk; }

// ------------------------------------------------------------ exact order --

struct ExactArgs {
  const float* q;        // [seq][heads*64], rotated
  const uint16_t* kc;    // [kv_heads][capacity][64] f16
  const uint16_t* vt;    // [kv_heads][64][vstride] f16
  const int* d_pos;      // when set, past is read from the device (decode)
  float* scores;         // [seq][heads][score_stride], score_stride % 4 == 0
  float* maxes;          // [seq][heads][max_stride]: per-span maxima
  int* counters;         // [seq][heads]: zero between launches; the last block resets its own
  float* out;            // [seq][heads*64]
  int past, capacity, vstride, heads, kv_heads, score_stride, max_stride;
};

// The sequential PV sum reads values from LDS: the last block stages a head's
// values in chunks of kVChunk positions, double-buffered, waves 1-3 loading
// chunk k+1 while wave 0 sums chunk k. Rows are padded by 16 bytes, so the 64
// lanes (one row each) spread their 16-byte reads over all LDS banks.
constexpr int kVChunk = 512;
constexpr int kVRow = kVChunk + 8;   // f16 elements per staged row

// buf[d][0..n8) = values of dimension d at positions p0 .. p0+n8-1, n8 = n rounded
// up to 8 (the tail group stays inside the row: vstride is a multiple of 8 and
// p0 + n <= capacity). Thread t of nt loads NS 16-byte groups before storing any.
template <int NS>
__device__ __forceinline__ void stage_values(const uint16_t* __restrict__ vbase, int vstride, int p0,
                                             int n, uint16_t (*buf)[kVRow], int t, int nt) {
  const int gpr = (n + 7) >> 3;  // 16-byte groups per row
  const int items = kHeadDim * gpr;
  for (int base = 0; base < items; base += nt * NS) {
    v4u v[NS];
#pragma unroll
    for (int j = 0; j < NS; j++) {
      const int i = base + t + j * nt;
      if (i < items) {
        const int d = i / gpr, gi = i - d * gpr;
        v[j] = *reinterpret_cast<const v4u*>(vbase + (size_t)d * vstride + p0 + 8 * gi);
      }
    }
#pragma unroll
    for (int j = 0; j < NS; j++) {
      const int i = base + t + j * nt;
      if (i < items) {
        const int d = i / gpr, gi = i - d * gpr;
        *reinterpret_cast<v4u*>(&buf[d][8 * gi]) = v[j];
      }
    }
  }
}

// Eight steps of the PV sum: o += p[s] * v[s] in order, v eight f16 values.
__device__ __forceinline__ float pv8(const v4f pa, const v4f pb, const v4u v, float o) {
  o = fmaf(pa.x, f16_lo(v.x), o);
  o = fmaf(pa.y, f16_hi(v.x), o);
  o = fmaf(pa.z, f16_lo(v.y), o);
  o = fmaf(pa.w, f16_hi(v.y), o);
  o = fmaf(pb.x, f16_lo(v.z), o);
  o = fmaf(pb.y, f16_hi(v.z), o);
  o = fmaf(pb.z, f16_lo(v.w), o);
  o = fmaf(pb.w, f16_hi(v.w), o);
  return o;
}

// o += p[s] * v[s] for s < n, ascending, rounding to f32 at every step (lane d
// holds output dimension d; row = its staged values). The product is exact in
// the fused form, so each step is the CPU's f64 sum stored to f32 except in
// double-rounding ties (probability ~2^-29 per step). row is LDS (p is LDS or
// global); the reads of the next 16 positions are issued before the current 16
// are summed.
struct PvGroup {  // 16 positions: p as 4 x float4, values as 2 x 8 f16
  v4f p[4];
  v4u v[2];
};
__device__ __forceinline__ void pv_load(const v4f* pg, const v4u* vg, int grp, PvGroup& g) {
#pragma unroll
  for (int k = 0; k < 4; k++) g.p[k] = pg[4 * grp + k];
  g.v[0] = vg[2 * grp];
  g.v[1] = vg[2 * grp + 1];
}
__device__ __forceinline__ float pv_sum(const PvGroup& g, float o) {
  o = pv8(g.p[0], g.p[1], g.v[0], o);
  return pv8(g.p[2], g.p[3], g.v[1], o);
}

__device__ __forceinline__ float pv_lds(const float* __restrict__ p, const uint16_t* row, int n, float o) {
  const v4f* pg = reinterpret_cast<const v4f*>(p);
  const v4u* vg = reinterpret_cast<const v4u*>(row);
  const int groups = n >> 4;
  // Two named buffers alternate, so no register copies sit between the loads of
  // one group and the arithmetic of the other.
  PvGroup a, b;
  if (groups > 0) pv_load(pg, vg, 0, a);
  int grp = 0;
  for (; grp + 2 <= groups; grp += 2) {
    pv_load(pg, vg, grp + 1, b);
    o = pv_sum(a, o);
    if (grp + 2 < groups) pv_load(pg, vg, grp + 2, a);
    o = pv_sum(b, o);
  }
  if (grp < groups) o = pv_sum(a, o);
  for (int s = groups << 4; s < n; s++) o = fmaf(p[s], (float)__builtin_bit_cast(_Float16, row[s]), o);
  return o;
}

// ------------------------------------------------- exact order, one block --
// Contexts up to kPLds: one 512-thread block per (query, head) does it all in
// LDS -- scores one position per thread and step, softmax, and the PV sum by
// wave 0 while the other 7 waves stage the next value chunk -- with no
// cross-block synchronization. The first value chunk and the first key rows are in flight
// from the kernel's start.
constexpr int kAttnThreads = 512;
constexpr int kAttnWaves = kAttnThreads / kWave;

__device__ __forceinline__ double block_sum_f64_n(double v, double* red) {
  v = team_sum<64>(v);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  double t = 0;
#pragma unroll
  for (int w = 0; w < kAttnWaves; w++) t += red[w];
  __syncthreads();
  return t;
}

static __global__ __launch_bounds__(kAttnThreads) void k_attn_block(ExactArgs a) {
  const int h = blockIdx.x, t = blockIdx.y;
  const int past = a.d_pos ? *a.d_pos : a.past;
  const int pos = past + t;
  if (pos >= a.capacity || pos >= kPLds) return;  // the host keeps positions inside both
  const int ctx = pos + 1;
  const int g = h / (a.heads / a.kv_heads);
  const int tid = threadIdx.x;

  __shared__ double qs[kHeadDim];
  __shared__ float wred[kAttnWaves];
  __shared__ double red[kAttnWaves];
  __shared__ __attribute__((aligned(16))) float pl[kPLds];
  __shared__ __attribute__((aligned(16))) uint16_t vbuf[2][kHeadDim][kVRow];

  // First value chunk: 64 rows x up to 64 16-byte groups, 8 per thread.
  const uint16_t* vbase = a.vt + (size_t)g * kHeadDim * a.vstride;
  const int n0 = min(ctx, kVChunk);
  const int gpr0 = (n0 + 7) >> 3;
  constexpr int kPre = kHeadDim * (kVChunk / 8) / kAttnThreads;
  v4u vpre[kPre];
#pragma unroll
  for (int j = 0; j < kPre; j++) {
    const int i = tid + j * kAttnThreads;
    if (i < kHeadDim * gpr0) {
      const int d = i / gpr0, gi = i - d * gpr0;
      vpre[j] = *reinterpret_cast<const v4u*>(vbase + (size_t)d * a.vstride + 8 * gi);
    }
  }
  const uint16_t* kb = a.kc + (size_t)g * a.capacity * kHeadDim;
  v4u kr[8];
  if (tid < ctx) {
#pragma unroll
    for (int j = 0; j < 8; j++) kr[j] = reinterpret_cast<const v4u*>(kb + (size_t)tid * kHeadDim)[j];
  }
  if (tid < kHeadDim) qs[tid] = (double)a.q[((size_t)t * a.heads + h) * kHeadDim + tid];
  __syncthreads();

  // Scores: dot += q[i] * k[i], i ascending, in f64 (each product is exact), stored f32.
  float m = -INFINITY;
  for (int p = tid; p < ctx; p += kAttnThreads) {
    if (p != tid) {
#pragma unroll
      for (int j = 0; j < 8; j++) kr[j] = reinterpret_cast<const v4u*>(kb + (size_t)p * kHeadDim)[j];
    }
    double dot = 0.0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint32_t u[4] = {kr[j].x, kr[j].y, kr[j].z, kr[j].w};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        dot = fma(qs[8 * j + 2 * e], (double)f16_lo(u[e]), dot);
        dot = fma(qs[8 * j + 2 * e + 1], (double)f16_hi(u[e]), dot);
      }
    }
    const float s = (float)(dot * 0.125);  // scale = 1/sqrt(64), exact
    pl[p] = s;
    m = fmaxf(m, s);
  }
#pragma unroll
  for (int j = 0; j < kPre; j++) {
    const int i = tid + j * kAttnThreads;
    if (i < kHeadDim * gpr0) {
      const int d = i / gpr0, gi = i - d * gpr0;
      *reinterpret_cast<v4u*>(&vbuf[0][d][8 * gi]) = vpre[j];
    }
  }
  m = wave_max(m);
  if ((tid & (kWave - 1)) == 0) wred[tid / kWave] = m;
  __syncthreads();
  float mb = wred[0];
#pragma unroll
  for (int w = 1; w < kAttnWaves; w++) mb = fmaxf(mb, wred[w]);
  const double M = mb;
  // e = exp(s - max) stored f32; the sum over the unrounded e in f64; p = f32(e32 * (1/sum)).
  double sum = 0.0;
  for (int p = tid; p < ctx; p += kAttnThreads) {
    const double e = exp((double)pl[p] - M);
    pl[p] = (float)e;
    sum += e;
  }
  sum = block_sum_f64_n(sum, red);
  const double inv = 1.0 / sum;
  for (int p = tid; p < ctx; p += kAttnThreads) pl[p] = (float)((double)pl[p] * inv);
  __syncthreads();

  const int nch = (ctx + kVChunk - 1) / kVChunk;
  float o = 0.f;
  for (int k = 0; k < nch; k++) {
    const int p0 = k * kVChunk;
    if (tid < kWave) {
      o = pv_lds(pl + p0, vbuf[k & 1][tid], min(kVChunk, ctx - p0), o);
    } else if (k + 1 < nch) {
      // 448 threads x 10 groups cover a chunk's 64 x 64 groups in one pass
      stage_values<10>(vbase, a.vstride, p0 + kVChunk, min(kVChunk, ctx - p0 - kVChunk), vbuf[(k + 1) & 1],
                      tid - kWave, kAttnThreads - kWave);
    }
    __syncthreads();
  }
  if (tid < kHeadDim) a.out[((size_t)t * a.heads + h) * kHeadDim + tid] = o;
}

// grid (spans, heads, seq). Block (span, h, t) scores positions span*256 ..
// +255 of query t against head h and records the span's maximum; the last span
// block of (t, h) to finish computes the probabilities and the output.
static __global__ __launch_bounds__(kBlock) void k_attn_exact(ExactArgs a) {
  const int sp = blockIdx.x, h = blockIdx.y, t = blockIdx.z;
  const int past = a.d_pos ? *a.d_pos : a.past;
  const int pos = past + t;
  if (pos >= a.capacity) return;  // the host keeps positions inside the cache
  const int ctx = pos + 1;
  const int nspan = attn_spans(ctx);
  if (sp >= nspan) return;
  const int g = h / (a.heads / a.kv_heads);
  const int tid = threadIdx.x;
  const int p = sp * kSpan + tid;

  __shared__ double qs[kHeadDim];
  __shared__ float wmax[kBlock / kWave];
  __shared__ double red[kBlock / kWave];
  __shared__ int is_last;
  __shared__ __attribute__((aligned(16))) float pl[kPLds];
  __shared__ __attribute__((aligned(16))) uint16_t vbuf[2][kHeadDim][kVRow];

  v4u kr[8];
  if (p < ctx) {
    const v4u* kp = reinterpret_cast<const v4u*>(a.kc + ((size_t)g * a.capacity + p) * kHeadDim);
#pragma unroll
    for (int j = 0; j < 8; j++) kr[j] = kp[j];
  }
  if (tid < kHeadDim) qs[tid] = (double)a.q[((size_t)t * a.heads + h) * kHeadDim + tid];
  __syncthreads();

  const size_t row = (size_t)t * a.heads + h;
  float* sc = a.scores + row * a.score_stride;
  float s = -INFINITY;
  if (p < ctx) {
    // dot += q[i] * k[i], i ascending, in f64 (each product is exact).
    double dot = 0.0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const uint32_t u[4] = {kr[j].x, kr[j].y, kr[j].z, kr[j].w};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        dot = fma(qs[8 * j + 2 * e], (double)f16_lo(u[e]), dot);
        dot = fma(qs[8 * j + 2 * e + 1], (double)f16_hi(u[e]), dot);
      }
    }
    s = (float)(dot * 0.125);  // scale = 1/sqrt(64), exact
    sc[p] = s;
  }
  const float wm = wave_max(s);
  if ((tid & (kWave - 1)) == 0) wmax[tid / kWave] = wm;
  __syncthreads();
  if (tid == 0) {
    a.maxes[row * a.max_stride + sp] = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    __threadfence();
    is_last = atomicAdd(a.counters + row, 1) == nspan - 1;
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();

  // The first value chunk loads while the softmax runs.
  const uint16_t* vbase = a.vt + (size_t)g * kHeadDim * a.vstride;
  const int nch = (ctx + kVChunk - 1) / kVChunk;
  stage_values<16>(vbase, a.vstride, 0, min(ctx, kVChunk), vbuf[0], tid, kBlock);

  // The global max is the max of the span maxima (max is order-free).
  float m = -INFINITY;
  for (int c = tid; c < nspan; c += kBlock) m = fmaxf(m, a.maxes[row * a.max_stride + c]);
  m = wave_max(m);
  __syncthreads();
  if ((tid & (kWave - 1)) == 0) wmax[tid / kWave] = m;
  __syncthreads();
  const double M = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  // e = exp(s - max) stored f32; the sum over the unrounded e in f64; p = f32(e32 * (1/sum)).
  float* pb = ctx <= kPLds ? pl : sc;
  double sum = 0.0;
  for (int i = tid; i < ctx; i += kBlock) {
    const double e = exp((double)sc[i] - M);
    pb[i] = (float)e;
    sum += e;
  }
  sum = block_sum_f64(sum, red);
  const double inv = 1.0 / sum;
  for (int i = tid; i < ctx; i += kBlock) pb[i] = (float)((double)pb[i] * inv);
  __syncthreads();
  float o = 0.f;
  for (int k = 0; k < nch; k++) {
    const int p0 = k * kVChunk;
    if (tid < kWave) {
      // separate calls, so the LDS one compiles to LDS reads rather than flat ones
      if (ctx <= kPLds) o = pv_lds(pl + p0, vbuf[k & 1][tid], min(kVChunk, ctx - p0), o);
      else o = pv_lds(sc + p0, vbuf[k & 1][tid], min(kVChunk, ctx - p0), o);
    } else if (k + 1 < nch) {
      stage_values<16>(vbase, a.vstride, p0 + kVChunk, min(kVChunk, ctx - p0 - kVChunk), vbuf[(k + 1) & 1],
                       tid - kWave, kBlock - kWave);
    }
    __syncthreads();
  }
  if (tid < kHeadDim) a.out[row * kHeadDim + tid] = o;
  if (tid == 0) a.counters[row] = 0;
}

// -------------------------------------------------------------- split-K --

struct SplitArgs {
  const float* q;        // [seq][heads*64], rotated
  const uint16_t* kc;    // [kv_heads][capacity][64] f16
  const uint16_t* vt;    // [kv_heads][64][vstride] f16
  float* partials;       // [seq][kv_heads][s_grid][group][66]
  int* counters;         // [seq][kv_heads], zero between launches
  float* out;            // [seq][heads*64]
  int past, seq, capacity, vstride, heads, kv_heads, s_grid;
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

[[maybe_unused]] static __global__ __launch_bounds__(kBlock) void k_attention_splitk(SplitArgs a) {
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
  __shared__ _Float16 vs[kChunk][kHeadDim + 2];
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
  const uint16_t* vbase = a.vt + (size_t)g * kHeadDim * a.vstride;
  for (int c = c0; c < c1; c++) {
    const int p0 = c * kChunk;
    const int n = min(kChunk, ctx - p0);
    for (int e = tid; e < kChunk * 8; e += kBlock) {
      // keys: position p, 16-byte part; values: dimension d, 8 positions from p8
      const int p = e >> 3, part = e & 7;
      v4u kv4 = {0, 0, 0, 0}, vv4 = {0, 0, 0, 0};
      if (p < n) kv4 = reinterpret_cast<const v4u*>(kbase + (size_t)(p0 + p) * kHeadDim)[part];
      const int d = e >> 3, p8 = (e & 7) * 8;
      if (p8 < n) vv4 = *reinterpret_cast<const v4u*>(vbase + (size_t)d * a.vstride + p0 + p8);
#pragma unroll
      for (int k = 0; k < 4; k++) *reinterpret_cast<uint32_t*>(&ks[p][part * 8 + 2 * k]) = kv4[k];
      const uint32_t vu[4] = {vv4.x, vv4.y, vv4.z, vv4.w};
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const uint16_t bits = (uint16_t)(vu[k >> 1] >> (16 * (k & 1)));
        // positions past the context hold no value yet: stage zeros, as their weights are
        vs[p8 + k][d] = p8 + k < n ? __builtin_bit_cast(_Float16, bits) : (_Float16)0.f;
      }
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
