// Causal GQA attention over an f16 KV cache (device code, shared by the
// operators and the decode step). Replaces ATTENTION (src/gpu/kernels.js:
// 404-499). Query head h reads kv head h / (heads/kv_heads), the blocked map of
// src/core/attention.js:74-76.
//
// Cache layout, per kv head: keys position-major [capacity][64] (a position's
// key is one 128-byte row, read whole by the lane that scores it) and values
// dimension-major [64][vstride] with vstride = capacity rounded up to 64 (one
// dimension's values over positions are contiguous, so the lane that owns
// output dimension d reads 8 positions in one 16-byte load).
//
// Three algorithms:
//
// Exact order (k_attn_block up to kPLds positions, k_attn_exact beyond), the
// model's QH_NUMERICS_EXACT path. It evaluates groupedAttention (src/core/attention.js:
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
// Split-K online softmax with the GQA group on the matrix cores (k_attn_gqa): the
// decode step's and batched prefill's path (QH_NUMERICS_FAST), qh_attention_splitk's
// and the list operator's: one block per (query, kv head, run of 64-position
// chunks), the group's query heads as the columns of f16 MFMA products, so each K/V
// chunk is read once per kv head; the runs' partials are merged afterwards. q and p
// go in as two f16 terms each (~1e-6 of the output): exact to f32 rounding, not to
// the CPU's order, and checked within the kernel tolerance. A flash form of the same
// products (k_flash_prefill) serves the MFMA prompt path.
#pragma once

#include "device_common.h"

namespace qh {

constexpr int kChunk = 64;        // split-K: positions per chunk
constexpr int kHeadDim = 64;
constexpr int kPLds = 4096;       // exact: probabilities kept in LDS up to this context
static_assert(kSpan == kBlock, "exact attention scores one position per thread");

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
// up to 8 (the tail group stays inside the row: vstride is a multiple of 64 and
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
// Split-K online softmax. The context is cut into 64-position chunks; a "slot"
// (run) is every S-th chunk of a query's context. A slot's partial state (m, l,
// o[64]) per query head goes to `part`; a merge (k_attn_combine, k_attn_merge_long,
// or the decode o-projection's staging) combines the slots of a head:
//   M = max_s m_s,  L = sum_s l_s 2^(m_s - M),  out = sum_s o_s 2^(m_s - M) / L
// (maxima in base-2 units). f32 throughout; agrees with groupedAttention
// (src/core/attention.js:32-66) to f32 rounding. The chunks of a slot depend on the
// query's own context only, so a prefill row and the same position decoded alone
// give the same bits.
constexpr int kPartStride = 68;   // floats per slot partial: m, l, 2 pad, o[64]
constexpr int kDecodeSlots = 16;  // slots per head in the decode step (combined in staging)
constexpr int kOpSlots = 64;      // most slots per head of the list operator

__host__ __device__ inline int attn_chunks(int ctx) { return (ctx + kChunk - 1) / kChunk; }

// Slot s of a query owns chunks s, s + S, s + 2S, ... below attn_chunks(ctx)
// (S slots per query head); a slot with no chunk writes the neutral partial
// (m = -inf, l = 0, o = 0). The first chunk a slot reads does not depend on the
// context, so its loads start before the position arrives from the device.
__host__ __device__ inline int slots_used(int ctx, int max_slots) {
  const int n = attn_chunks(ctx);
  return n < max_slots ? n : max_slots;
}

struct SlotArgs {
  const float* q;        // [seq][heads*64], rotated
  const uint16_t* kc;    // [kv_heads][capacity][64] f16
  const uint16_t* vt;    // [kv_heads][64][vstride] f16
  const int* d_pos;      // when set, past is read from the device (decode)
  float* part;           // [seq][heads][max_slots][kPartStride]
  float* out;            // k_attn_gqa with one slot: the output [list][seq][heads*64] in place of partials
  int past, capacity, vstride, heads, kv_heads, max_slots;
  // A list of same-shape caches, one per blockIdx.z (0 apart from the list operator):
  // element strides between consecutive key caches, value caches, and partial sets.
  size_t list_k, list_v, list_part;
};

template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
  return fmaxf(v, dpp32<CTRL>(v));
}
// Max over a team of TL lanes (16 or 64); every lane ends with the same value.
template <int TL>
__device__ __forceinline__ float team_max(float v) {
  v = dpp_max<kDppQuadXor1>(v);
  v = dpp_max<kDppQuadXor2>(v);
  v = dpp_max<kDppHalfMirror>(v);
  v = dpp_max<kDppMirror>(v);
  if constexpr (TL >= 32) v = fmaxf(v, swz_xor16(v));
  if constexpr (TL >= 64) v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

// ------------------------------------------------ prefill on the matrix cores --
// Causal GQA attention of `seq` queries (positions past .. past+seq-1) as a flash
// attention on v_mfma_f32_16x16x32_f16: one block per (query head, 16 queries), keys
// in steps of 32 with an online softmax per query, the steps spread over the block's
// waves and their states merged at the end.
//
// Transposed products keep every operand where it is loaded: S^T = K Q^T (A = 16 key
// rows of the position-major cache, 16 bytes per lane; B = the wave's queries), then
// O^T += V^T P^T (A = 16 dimension rows of the dimension-major value cache; B = P^T).
// In the D layout lane l holds rows 4*(l/16)+r of query l%16; with the key rows of
// the two 16-key tiles interleaved (KvStep below) those are keys 8*(l/16) .. +7 over
// both tiles, exactly the B operand of the second product for query l%16 with the
// contraction in key order -- the value operand is one 16-byte run of a dimension row
// -- so P never leaves its registers, and the softmax state of a query lives in the
// four lanes that share it.
//
// Precision: q (scaled by 1/8 log2 e) and p are each split into two f16 terms
// whose sum is the f32 value to 2^-22, the f16 K/V are exact, products accumulate
// in f32: the output agrees with the split-K f32 path to ~1e-6 (not to the bit).
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kFlashQ = 16;  // queries per wave
// q is scaled by 1/sqrt(64) * log2(e) once, so scores are in base-2 units and the softmax
// weights are 2^(s - max) -- the same softmax.
constexpr float kScoreLog2 = 0.125f * 1.44269504088896340736f;

// 2^x for finite x <= 0 as v_exp_f32 of the fraction in [-0.5, 0.5] scaled by 2^rint(x):
// the hardware exp2 is taken only where it is accurate (on the whole range its error
// reached ~1e-5 of the attention output at short contexts).
__device__ __forceinline__ float exp2_reduced(float x) {
  const float n = __builtin_rintf(x);
  return __builtin_ldexpf(__builtin_amdgcn_exp2f(x - n), (int)n);
}
constexpr int kFlashK = 32;  // keys per step

struct FlashArgs {
  const float* q;        // [seq][heads*64], rotated
  const uint16_t* kc;    // [kv_heads][capacity][64] f16
  const uint16_t* vt;    // [kv_heads][64][vstride] f16
  float* out;            // [seq][heads*64]
  int past, seq, capacity, vstride, heads, kv_heads;
  int first;             // blocks of the first round: the device's compute units (launch_flash_prefill)
};

// x as hi + lo, two f16 values: hi = f16(x), lo = f16(x - hi) (x - hi is exact in f32).
// x must be one materialized f32 value (f32_pinned): left as a product, the compiler
// fuses it into both conversions (v_fma_mix*), rounding hi and lo from different values
// whose halves need not sum to either.
__device__ __forceinline__ float f32_pinned(float x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ __forceinline__ _Float16 f16_hi_part(float x) { return (_Float16)x; }
__device__ __forceinline__ _Float16 f16_lo_part(float x) { return (_Float16)(x - (float)(_Float16)x); }

// One step of 32 keys (p0 .. p0+31) for 16 query columns, shared by the flash and the
// GQA kernels: S^T = K Q^T over two 16-key tiles (8 MFMAs), the online softmax per
// query column, O^T += V^T P^T (8 MFMAs). The loads of a step go into a KvStep so a
// caller can issue the next step's loads before this step's arithmetic.
//
// Key order: row n of 16-key tile j holds key 8*(n/4) + 4j + n%4, so the score tile's D
// layout gives lane (n, g) keys 8g + 4j + r, and the eight P values of the lane are keys
// 8g .. 8g+7 in order -- the value operand of dimension 16dt + n is then one 16-byte
// run of its row (the contraction order is the same permutation for both operands).
struct KvStep {
  f16x8 k[2][2];  // key 8*(n/4) + 4j + n%4, dims 32ks + 8g .. +7
  v4u v[4];       // dimension 16dt + n: keys 8g .. 8g+7
};

__device__ __forceinline__ int kv_key_row(int j, int n) { return 8 * (n >> 2) + 4 * j + (n & 3); }

// In bounds for every p0 >= 0: key rows are clamped to the cache, value runs to the row.
__device__ __forceinline__ void kv_load(const uint16_t* kb, const uint16_t* vb, int p0, int capacity, int vstride,
                                        int n, int g, KvStep& d) {
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const uint16_t* kr = kb + (size_t)min(p0 + kv_key_row(j, n), capacity - 1) * kHeadDim;
#pragma unroll
    for (int ks = 0; ks < 2; ks++) d.k[j][ks] = *reinterpret_cast<const f16x8*>(kr + 32 * ks + 8 * g);
  }
#pragma unroll
  for (int dt = 0; dt < 4; dt++)
    d.v[dt] = *reinterpret_cast<const v4u*>(vb + (size_t)(16 * dt + n) * vstride + min(p0 + 8 * g, vstride - 8));
}

// Scores of keys >= slim (this lane's query column) are masked; values of keys >= vlim
// (uniform: keys never written for this launch may hold any bits) become zeros. A query
// column whose keys are all masked so far keeps m = -inf, l = 0 and o = 0 exactly.
__device__ __forceinline__ void kv_step(const f16x8 (&qh)[2], const f16x8 (&ql)[2], KvStep& d, int p0, int slim,
                                        int vlim, int g, float& m, float& l, f32x4 (&o)[4]) {
  f32x4 s[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(d.k[j][ks], qh[ks], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(d.k[j][ks], ql[ks], acc, 0, 0, 0);
    }
    s[j] = acc;
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      s[j][r] = p0 + 8 * g + 4 * j + r < slim ? s[j][r] : -INFINITY;
      tmax = fmaxf(tmax, s[j][r]);
    }
  tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
  tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
  const float mn = fmaxf(m, tmax);
  const float alpha = m == -INFINITY ? 0.f : exp2_reduced(m - mn);  // m finite: mn finite too
  float pv[2][4], psum = 0.f;
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      pv[j][r] = s[j][r] == -INFINITY ? 0.f : exp2_reduced(s[j][r] - mn);
      psum += pv[j][r];
    }
  psum += __shfl_xor(psum, 16);
  psum += __shfl_xor(psum, 32);
  l = fmaf(l, alpha, psum);
  m = mn;
  f16x8 ph, pl;  // contraction order: keys 8g .. 8g+7
#pragma unroll
  for (int r = 0; r < 4; r++) {
    ph[r] = f16_hi_part(pv[0][r]);
    pl[r] = f16_lo_part(pv[0][r]);
    ph[4 + r] = f16_hi_part(pv[1][r]);
    pl[4 + r] = f16_lo_part(pv[1][r]);
  }
  if (p0 + 32 > vlim) {
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const int k0 = p0 + 8 * g + 2 * w;  // keys of d.v[dt][w]: k0, k0+1
        d.v[dt][w] &= (k0 < vlim ? 0x0000ffffu : 0u) | (k0 + 1 < vlim ? 0xffff0000u : 0u);
      }
  }
#pragma unroll
  for (int dt = 0; dt < 4; dt++) {
    f32x4 c = o[dt];
#pragma unroll
    for (int r = 0; r < 4; r++) c[r] *= alpha;
    const f16x8 va = __builtin_bit_cast(f16x8, d.v[dt]);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, ph, c, 0, 0, 0);
    o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pl, c, 0, 0, 0);
  }
}

// q split into hi + lo f16 terms, scaled to base-2 score units: B of S^T = K Q^T for
// query column n, dims 32ks + 8g .. +7 (qr: the query's 64 floats).
__device__ __forceinline__ void load_query_split(const float* qr, int g, f16x8 (&qh)[2], f16x8 (&ql)[2]) {
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    const v4f x0 = *reinterpret_cast<const v4f*>(qr + 32 * ks + 8 * g);
    const v4f x1 = *reinterpret_cast<const v4f*>(qr + 32 * ks + 8 * g + 4);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float a0 = f32_pinned(x0[e] * kScoreLog2), a1 = f32_pinned(x1[e] * kScoreLog2);
      qh[ks][e] = f16_hi_part(a0);
      ql[ks][e] = f16_lo_part(a0);
      qh[ks][4 + e] = f16_hi_part(a1);
      ql[ks][4 + e] = f16_lo_part(a1);
    }
  }
}

// A (query head, 16 queries) tile is one block of kFlashWaves waves: key step i (keys
// 32i .. 32i+31, up to the tile's last key) goes to wave i % kFlashWaves, which walks its
// steps with the next one's loads in flight (two KvStep buffers); the waves' (m, l, o)
// states then merge through LDS in wave order. Step i lands on the same wave whatever
// the tile, and a key a query does not see adds exact zeros, so a query's output does
// not depend on the other queries of its tile.
constexpr int kFlashWaves = 4;

static __global__ __launch_bounds__(kWave * kFlashWaves) void k_flash_prefill(FlashArgs a) {
  __shared__ v4f sh_o[kFlashWaves][4][kWave];
  __shared__ float sh_m[kFlashWaves][kFlashQ], sh_l[kFlashWaves][kFlashQ];
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave, n = lane & 15, g = lane >> 4;
  // Block order (a bijection of the (query tile, head) pairs): a causal tile's work grows with
  // its index, and the blocks of a launch are dealt to the CUs in turn, block b and b + CUs
  // sharing a CU. So the first `first` blocks (one per CU) take the heaviest tiles, heaviest
  // first, and the rest the lightest, lightest first: a CU's two blocks then sum to about the
  // same work everywhere (in tile order, block b and b + 256 were the same tile of two heads).
  const int tiles = (a.seq + kFlashQ - 1) / kFlashQ, nb = tiles * a.heads;
  const int first = min(nb, a.first), b = blockIdx.x;
  const int k = b < first ? b : nb - 1 - (b - first);
  const int h = k % a.heads;
  const int kvh = h / (a.heads / a.kv_heads);
  const int t0 = (tiles - 1 - k / a.heads) * kFlashQ;
  const int tn = min(t0 + n, a.seq - 1);  // this lane's query; past the end, a copy of the last
  const int qpos = a.past + tn;
  const int kmax = a.past + min(t0 + kFlashQ - 1, a.seq - 1);  // the tile's last key

  f16x8 qh[2], ql[2];
  load_query_split(a.q + ((size_t)tn * a.heads + h) * kHeadDim, g, qh, ql);
  const uint16_t* kb = a.kc + (size_t)kvh * a.capacity * kHeadDim;
  const uint16_t* vb = a.vt + (size_t)kvh * kHeadDim * a.vstride;
  float m = -INFINITY, l = 0.f;
  f32x4 o[4];  // O^T: dims 16dt + 4g + r of query n
#pragma unroll
  for (int dt = 0; dt < 4; dt++) o[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};

  constexpr int kStride = kFlashWaves * kFlashK;
  const int steps = kmax / kFlashK + 1;
  int left = (steps - w + kFlashWaves - 1) / kFlashWaves;  // steps w, w + kFlashWaves, ...
  int p0 = w * kFlashK;
  KvStep A, B;
  kv_load(kb, vb, p0, a.capacity, a.vstride, n, g, A);
  while (left > 0) {
    if (left == 1) {
      kv_step(qh, ql, A, p0, qpos + 1, kmax + 1, g, m, l, o);
      break;
    }
    kv_load(kb, vb, p0 + kStride, a.capacity, a.vstride, n, g, B);
    __builtin_amdgcn_sched_barrier(0);  // the next step's loads before this step's arithmetic
    kv_step(qh, ql, A, p0, qpos + 1, kmax + 1, g, m, l, o);
    p0 += kStride;
    if (--left == 1) {
      kv_step(qh, ql, B, p0, qpos + 1, kmax + 1, g, m, l, o);
      break;
    }
    kv_load(kb, vb, p0 + kStride, a.capacity, a.vstride, n, g, A);
    __builtin_amdgcn_sched_barrier(0);
    kv_step(qh, ql, B, p0, qpos + 1, kmax + 1, g, m, l, o);
    p0 += kStride;
    --left;
  }
#pragma unroll
  for (int dt = 0; dt < 4; dt++) sh_o[w][dt][lane] = (v4f)o[dt];
  if (g == 0) {
    sh_m[w][n] = m;
    sh_l[w][n] = l;
  }
  __syncthreads();
  // Merge: wave dt writes dims 16dt + 4g .. +3 of query n (wave 0 always holds key 0).
  for (int dt = w; dt < 4; dt += kFlashWaves) {
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < kFlashWaves; v++) mx = fmaxf(mx, sh_m[v][n]);
    float lt = 0.f;
    v4f ot = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < kFlashWaves; v++) {
      const float mv = sh_m[v][n];
      const float wt = mv == -INFINITY ? 0.f : exp2_reduced(mv - mx);
      lt = fmaf(sh_l[v][n], wt, lt);
      const v4f ov = sh_o[v][dt][lane];
#pragma unroll
      for (int r = 0; r < 4; r++) ot[r] = fmaf(ov[r], wt, ot[r]);
    }
    if (t0 + n < a.seq) {
      const v4f r = {ot[0] / lt, ot[1] / lt, ot[2] / lt, ot[3] / lt};
      *reinterpret_cast<v4f*>(a.out + ((size_t)(t0 + n) * a.heads + h) * kHeadDim + 16 * dt + 4 * g) = r;
    }
  }
}

static inline hipError_t launch_flash_prefill(hipStream_t s, FlashArgs a) {
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  a.first = cus > 0 ? cus : 1;
  hipLaunchKernelGGL(k_flash_prefill, dim3((a.seq + kFlashQ - 1) / kFlashQ * a.heads), dim3(kWave * kFlashWaves), 0,
                     s, a);
  return hipGetLastError();
}

// --------------------------------------- GQA group per slot on the matrix cores --
// The split-K slots with a whole GQA group per block: the group's query
// heads are the columns of the MFMA products of the flash kernel above (heads/kv_heads
// of the 16 used, the rest repeat head 0 and are dropped), so each key/value position
// is read once for the group instead of once per query head. A slot's chunks are
// walked in steps of 32 keys -- S^T for 2 tiles of 16 keys (8 MFMAs), the online
// softmax per head column, O^T += V^T P^T (8 MFMAs). Writes (m, l, o) slot partials in
// the layout above, with the maxima in base-2 units (merged by CombineIn in
// the decode step, k_attn_combine<true> for the operators). q and p are split into
// two f16 terms as in the flash kernel (~1e-6 of the output).
// Step i of slot sl: 32 keys starting at p0 (chunk sl + (i/2)*MAXS, half i%2).
template <int MAXS>
__device__ __forceinline__ int gqa_p0(int sl, int i) {
  return (sl + (i >> 1) * MAXS) * kChunk + (i & 1) * 32;
}

// grid (kv_heads * MAXS, queries, list entries), W waves per block. Block (kv head,
// slot) walks the slot's steps with step i on wave i % W (each wave with the next
// step's loads in flight), and the waves' (m, l, o) states merge
// through LDS in wave order, as in k_flash_prefill; the merged state is the slot's
// partial. Query t (blockIdx.y) is at position past + t, and its blocks do exactly what a
// launch for that query alone does, so a batch of queries gets the bits of one-query
// launches. The decode step runs W = 4 (at contexts up to 2048 each wave has at most one
// step, so a slot costs one step's latency), the list operator W = 1 (throughput).
template <int MAXS, int W>
static __global__ __launch_bounds__(kWave * W) void k_attn_gqa(SlotArgs a) {
  __shared__ v4f sh_o[W][4][kWave];
  __shared__ float sh_m[W][16], sh_l[W][16];
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave, n = lane & 15, g = lane >> 4;
  const int group = a.heads / a.kv_heads;
  const int kvh = blockIdx.x / MAXS, sl = blockIdx.x % MAXS;
  const int t = blockIdx.y;
  const size_t z = blockIdx.z;
  const int h = kvh * group + (n < group ? n : 0);
  f16x8 qh[2], ql[2];
  load_query_split(a.q + ((size_t)t * a.heads + h) * kHeadDim, g, qh, ql);
  const uint16_t* kb = a.kc + z * a.list_k + (size_t)kvh * a.capacity * kHeadDim;
  const uint16_t* vb = a.vt + z * a.list_v + (size_t)kvh * kHeadDim * a.vstride;
  KvStep A, B;
  int i = w;
  // A step in the slot's first chunk (sl < MAXS, so below 64 MAXS positions) is loaded before
  // the position arrives; a later one only once the position says the context reaches it
  // (loading it blind would fetch rows past the context whenever it does not).
  const bool early = i < 2;
  if (early) kv_load(kb, vb, gqa_p0<MAXS>(sl, i), a.capacity, a.vstride, n, g, A);
  const int pos = (a.d_pos ? *a.d_pos : a.past) + t;
  if (pos >= a.capacity) return;  // block-uniform
  const int ctx = pos + 1, nch = attn_chunks(ctx);
  float m = -INFINITY, l = 0.f;
  f32x4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; dt++) o[dt] = (f32x4){0.f, 0.f, 0.f, 0.f};
  int steps = 0;
  if (sl < nch) {
    const int chunks = (nch - 1 - sl) / MAXS + 1;
    const int last = sl + (chunks - 1) * MAXS;
    steps = 2 * chunks - (last * kChunk + 32 >= ctx ? 1 : 0);
  }
  int left = i < steps ? (steps - 1 - i) / W + 1 : 0;
  if (!early && left > 0) kv_load(kb, vb, gqa_p0<MAXS>(sl, i), a.capacity, a.vstride, n, g, A);
  while (left > 0) {
    if (left == 1) {
      kv_step(qh, ql, A, gqa_p0<MAXS>(sl, i), ctx, ctx, g, m, l, o);
      break;
    }
    kv_load(kb, vb, gqa_p0<MAXS>(sl, i + W), a.capacity, a.vstride, n, g, B);
    __builtin_amdgcn_sched_barrier(0);
    kv_step(qh, ql, A, gqa_p0<MAXS>(sl, i), ctx, ctx, g, m, l, o);
    i += W;
    if (--left == 1) {
      kv_step(qh, ql, B, gqa_p0<MAXS>(sl, i), ctx, ctx, g, m, l, o);
      break;
    }
    kv_load(kb, vb, gqa_p0<MAXS>(sl, i + W), a.capacity, a.vstride, n, g, A);
    __builtin_amdgcn_sched_barrier(0);
    kv_step(qh, ql, B, gqa_p0<MAXS>(sl, i), ctx, ctx, g, m, l, o);
    i += W;
    --left;
  }
  float* dst = a.part + z * a.list_part + (((size_t)t * a.heads + h) * MAXS + sl) * kPartStride;
  // One slot and an output buffer: the slot's state is the result, written as o / l (what the
  // combine of a single slot computes, bit for bit) with no partials and no combine launch.
  float* res = nullptr;
  if constexpr (MAXS == 1) {
    if (a.out) res = a.out + (((size_t)z * gridDim.y + t) * a.heads + h) * kHeadDim;
  }
  if constexpr (W == 1) {  // the merge below would scale by exactly 1
    if (res) {
      if (n < group) {
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
          const v4f r4 = {o[dt][0] / l, o[dt][1] / l, o[dt][2] / l, o[dt][3] / l};
          *reinterpret_cast<v4f*>(res + 16 * dt + 4 * g) = r4;
        }
      }
      return;
    }
    if (n < group) {
#pragma unroll
      for (int dt = 0; dt < 4; dt++) *reinterpret_cast<v4f*>(dst + 4 + 16 * dt + 4 * g) = (v4f)o[dt];
      if (g == 0) {
        dst[0] = m;
        dst[1] = l;
      }
    }
    return;
  }
#pragma unroll
  for (int dt = 0; dt < 4; dt++) sh_o[w][dt][lane] = (v4f)o[dt];
  if (g == 0) {
    sh_m[w][n] = m;
    sh_l[w][n] = l;
  }
  __syncthreads();
  float mx = -INFINITY;
#pragma unroll
  for (int v = 0; v < W; v++) mx = fmaxf(mx, sh_m[v][n]);
  for (int dt = w; dt < 4; dt += W) {
    float lt = 0.f;
    v4f ot = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < W; v++) {
      const float mv = sh_m[v][n];
      const float wt = mv == -INFINITY ? 0.f : exp2_reduced(mv - mx);
      lt = fmaf(sh_l[v][n], wt, lt);
      const v4f ov = sh_o[v][dt][lane];
#pragma unroll
      for (int r = 0; r < 4; r++) ot[r] = fmaf(ov[r], wt, ot[r]);
    }
    if (res) {
      if (n < group) *reinterpret_cast<v4f*>(res + 16 * dt + 4 * g) = v4f{ot[0] / lt, ot[1] / lt, ot[2] / lt, ot[3] / lt};
    } else if (n < group) {
      *reinterpret_cast<v4f*>(dst + 4 + 16 * dt + 4 * g) = ot;
      if (dt == 0 && g == 0) {
        dst[0] = mx;
        dst[1] = lt;
      }
    }
  }
}

// Slots per head of the decode attention for a cache of `capacity` positions. Up to
// kLongCapacity: kDecodeSlots, merged in the o-projection's staging (CombineIn). Past it the
// 2 x 16 blocks of that form stream the context through 32 CUs (19 us per launch at 32k
// positions), so a long cache takes kLongSlots slots (256 blocks), merged by k_attn_merge_long
// into the attention output before an o-projection that stages it as it is: one launch more
// per layer, which costs more than it saves below ~8k positions. The choice depends on the
// capacity only, so a cache's decode step and batched prefill merge alike.
constexpr int kDecodeWaves = 4;
constexpr int kLongSlots = 128;
constexpr int kLongCapacity = 8192;
__host__ __device__ inline bool decode_attn_long(int capacity) { return capacity > kLongCapacity; }
__host__ __device__ inline int decode_attn_slots(int capacity) {
  return decode_attn_long(capacity) ? kLongSlots : kDecodeSlots;
}

// out[z][t][h*64 + d] = the merge of the kLongSlots slot partials of (query t, head h): one
// 64-lane block per (h, t, list entry z). Every load is issued before any is used (the slots
// are a compile-time count; empty slots are neutral: m = -inf, l = 0, o = 0); the weights
// 2^(m_s - M) are shared through LDS and the output sums the slots in order.
template <int MAXS>
static __global__ __launch_bounds__(kWave) void k_attn_merge_long(const float* __restrict__ part,
                                                                  float* __restrict__ out, int heads,
                                                                  size_t list_part) {
  static_assert(MAXS % kWave == 0, "whole slots per lane");
  constexpr int kPer = MAXS / kWave;
  __shared__ float wl[MAXS];
  const int h = blockIdx.x, t = blockIdx.y, d = threadIdx.x;
  const size_t z = blockIdx.z;
  const float* p = part + z * list_part + ((size_t)t * heads + h) * MAXS * kPartStride;
  float ms[kPer], ls[kPer], ov[MAXS];
#pragma unroll
  for (int k = 0; k < kPer; k++) {
    ms[k] = p[(size_t)(d + k * kWave) * kPartStride];
    ls[k] = p[(size_t)(d + k * kWave) * kPartStride + 1];
  }
#pragma unroll
  for (int s2 = 0; s2 < MAXS; s2++) ov[s2] = p[(size_t)s2 * kPartStride + 4 + d];
  float M = ms[0];
#pragma unroll
  for (int k = 1; k < kPer; k++) M = fmaxf(M, ms[k]);
  M = team_max<64>(M);  // slot 0 always holds position 0
  float L = 0.f;
#pragma unroll
  for (int k = 0; k < kPer; k++) {
    const float w = ms[k] == -INFINITY ? 0.f : exp2_reduced(ms[k] - M);
    wl[d + k * kWave] = w;
    L = fmaf(w, ls[k], L);
  }
  L = team_sum<64>(L);
  __builtin_amdgcn_wave_barrier();  // one wave: its LDS writes land before its reads
  float A = 0.f;
#pragma unroll
  for (int s2 = 0; s2 < MAXS; s2++) A = fmaf(wl[s2], ov[s2], A);
  out[((z * gridDim.y + t) * heads + h) * kHeadDim + d] = A / L;
}

// The decode step's attention over `seq` queries (grid.y) and `count` list entries (grid.z):
// k_attn_gqa with decode_attn_slots(capacity) slots per head and four waves per slot. Short
// caches leave the slot partials for the decode combine (CombineIn); long ones merge them
// into `merged` ([count][seq][heads*64]) when it is given (the cold list times the slots
// alone).
static inline hipError_t launch_attn_decode(hipStream_t s, SlotArgs a, int seq, int count,
                                            float* merged = nullptr) {
  if (!decode_attn_long(a.capacity)) {
    a.max_slots = kDecodeSlots;
    hipLaunchKernelGGL((k_attn_gqa<kDecodeSlots, kDecodeWaves>), dim3(a.kv_heads * kDecodeSlots, seq, count),
                       dim3(kDecodeWaves * kWave), 0, s, a);
    return hipGetLastError();
  }
  a.max_slots = kLongSlots;
  hipLaunchKernelGGL((k_attn_gqa<kLongSlots, kDecodeWaves>), dim3(a.kv_heads * kLongSlots, seq, count),
                     dim3(kDecodeWaves * kWave), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !merged) return e;
  hipLaunchKernelGGL(k_attn_merge_long<kLongSlots>, dim3(a.heads, seq, count), dim3(kWave), 0, s, a.part, merged,
                     a.heads, a.list_part);
  return hipGetLastError();
}

// out[t][h][d] from the slot partials of (t, h): one 64-lane block per (h, t) (and list
// entry z, whose partials are list_part floats and output seq*heads*64 floats further on).
// B2: the partials' maxima are in base-2 units (k_attn_gqa), so the slot weights are
// 2^(m_s - M); else e^(m_s - M).
template <bool B2>
static __global__ __launch_bounds__(kWave) void k_attn_combine(const float* __restrict__ part,
                                                               float* __restrict__ out, int past,
                                                               int heads, int max_slots, size_t list_part) {
  const int h = blockIdx.x, t = blockIdx.y, d = threadIdx.x;
  const size_t z = blockIdx.z;
  const int nslots = slots_used(past + t + 1, max_slots);
  const float* p = part + z * list_part + ((size_t)t * heads + h) * max_slots * kPartStride;
  out += z * (size_t)gridDim.y * heads * kHeadDim;
  float M = -INFINITY;
  for (int s = 0; s < nslots; s++) M = fmaxf(M, p[(size_t)s * kPartStride]);
  float L = 0.f, A = 0.f;
  for (int s = 0; s < nslots; s++) {
    const float ms = p[(size_t)s * kPartStride];
    const float w = B2 ? (ms == -INFINITY ? 0.f : exp2_reduced(ms - M)) : expf(ms - M);
    L = fmaf(w, p[(size_t)s * kPartStride + 1], L);
    A = fmaf(w, p[(size_t)s * kPartStride + 4 + d], A);
  }
  out[((size_t)t * heads + h) * kHeadDim + d] = A / L;
}

// The decode step's combine, run by the o-projection while it stages its input:
// xs[lay.pos(i)] = attention output i (i = h*64 + d) as f64, for a single query
// whose slot partials (kDecodeSlots <= 16 per head, empty ones neutral, written by
// k_attn_gqa with the maxima in base-2 units) are at `part`. Thread i < heads*16
// owns head h = i/16: it reads the (m, l) of slot i%16 (neutral past the slots) and
// the four output dimensions 4*(i%16) .. +3 of every slot; the 16 lanes of a head
// form one DPP team, so M, L and the slot weights 2^(m_s - M) / L stay
// inside it (shared through the wave's own LDS slice). Nothing here depends on
// the position. heads <= 16. Loads (CombineIn::load) and arithmetic are split as
// for StageIn.
constexpr int kCombineLanes = 16;  // lanes per head in the combine: four output dimensions each
struct CombineIn {
  v4f ov[kDecodeSlots];
  float mv, lv;
  __device__ __forceinline__ void load(const float* __restrict__ part, int heads) {
    static_assert(kDecodeSlots <= kCombineLanes, "one lane per slot of a head");
    const int i = threadIdx.x;
    const int h = min(i / kCombineLanes, heads - 1), k = i % kCombineLanes;
    const float* ph = part + (size_t)h * kDecodeSlots * kPartStride;
#pragma unroll
    for (int s = 0; s < kDecodeSlots; s++)
      ov[s] = *reinterpret_cast<const v4f*>(ph + (size_t)s * kPartStride + 4 + 4 * k);
    const int ks = min(k, kDecodeSlots - 1);  // lanes past the slots hold the neutral partial
    mv = ph[(size_t)ks * kPartStride];
    lv = ph[(size_t)ks * kPartStride + 1];
    if (k >= kDecodeSlots) {
      mv = -INFINITY;
      lv = 0.f;
    }
  }
};

// The merged output dimensions 4*(i%16) .. +3 of head i/16 for thread i. `wl` is
// LDS of kBlock floats.
__device__ __forceinline__ v4f attn_combine_quad(const CombineIn& in, float* wl) {
  const int i = threadIdx.x;
  const float M = team_max<16>(in.mv);  // slot 0 always holds position 0
  // maxima in base-2 units (k_attn_gqa); an empty slot (m = -inf) weighs 0
  const float w = in.mv == -INFINITY ? 0.f : exp2_reduced(in.mv - M);
  const float L = team_sum<16>(w * in.lv);
  wl[i] = w / L;
  __builtin_amdgcn_wave_barrier();
  const float* wh = wl + (i & ~(kCombineLanes - 1));
  v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < kDecodeSlots; s++) {
    const float ws = wh[s];
    acc.x = fmaf(ws, in.ov[s].x, acc.x);
    acc.y = fmaf(ws, in.ov[s].y, acc.y);
    acc.z = fmaf(ws, in.ov[s].z, acc.z);
    acc.w = fmaf(ws, in.ov[s].w, acc.w);
  }
  return acc;
}

__device__ __forceinline__ void stage_attn_combine(const CombineIn& in, int heads, double* xs, XLayout lay,
                                                   float* wl) {
  const v4f acc = attn_combine_quad(in, wl);
  const int i = threadIdx.x;
  if (i < heads * kCombineLanes) {
    const int j = (i / kCombineLanes) * kHeadDim + 4 * (i % kCombineLanes);
    xs[lay.pos(j)] = (double)acc.x;
    xs[lay.pos(j + 1)] = (double)acc.y;
    xs[lay.pos(j + 2)] = (double)acc.z;
    xs[lay.pos(j + 3)] = (double)acc.w;
  }
  __syncthreads();
}

// The same merge staged for the f32 matvec core: thread i's quad is 4-element group
// i of the attention output (i = h*16 + k holds elements 64h + 4k .. +3), stored with
// its chunk sums after the heads*64 values.
template <int FMT>
__device__ __forceinline__ void stage_attn_combine_f32(const CombineIn& in, int heads, float* xs, XLayoutF lay,
                                                       float* wl) {
  const v4f acc = attn_combine_quad(in, wl);
  const int i = threadIdx.x;
  stage_group_f32<FMT>(acc, i, i < heads * kCombineLanes, xs, xs + heads * kHeadDim, lay);
  __syncthreads();
}

}  // namespace qh
