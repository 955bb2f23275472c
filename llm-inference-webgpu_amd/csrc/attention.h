// Causal GQA attention over an f16 head-major KV cache, split-K over context
// with an online softmax (device code, shared by the operator and the fused
// decode step).
//
// Replaces ATTENTION (src/gpu/kernels.js:404-499). The reference gives each
// (position, query head) a workgroup, writes every score to a global scratch
// buffer and walks all positions with 64 of 256 threads for the PV sum. Here
// one block owns (query position, kv head, split): the K/V chunk it stages
// into LDS serves all `group` query heads that share the kv head (7 for
// Qwen2.5), and the scores never leave LDS.
//
// Structure of one query at context ctx (= its position + 1):
//   chunks of 64 positions; S = min(nchunks, kMaxSplits) splits of
//   cps = ceil(nchunks / S) consecutive chunks; each split runs the online
//   softmax over its chunks in order and writes (m, l, acc[64]) per head;
//   the last split block to finish (atomic counter) combines the splits in
//   split order. The structure depends only on ctx, so a query computed in a
//   prefill and the same query computed in decode give the same bits.
#pragma once

#include "device_common.h"

namespace qh {

constexpr int kChunk = 64;        // positions per online-softmax step
constexpr int kMaxSplits = 128;   // splits per (query, kv head)
constexpr int kHeadDim = 64;
constexpr int kMaxGroup = 8;      // query heads per kv head
constexpr int kPartialStride = kHeadDim + 2;  // m, l, acc[64]

struct AttnArgs {
  const float* q;        // [seq][heads*64]; pre-rotation when rope_q
  const float* k_new;    // fused append: this step's k [kv_heads*64], pre-rotation
  const float* v_new;    // fused append: this step's v [kv_heads*64]
  uint16_t* kc;          // [kv_heads][capacity][64] f16
  uint16_t* vc;
  const float* cos_t;    // rope tables [positions][32]
  const float* sin_t;
  const int* d_pos;      // decode: past read from the device
  float* partials;       // [seq][kv_heads][s_grid][group][66]
  int* counters;         // [seq][kv_heads], zero between launches
  float* out;            // [seq][heads*64]
  int past, seq, capacity, heads, kv_heads, s_grid;
};

__host__ __device__ inline void attn_splits(int ctx, int* nchunks, int* cps, int* splits) {
  const int n = (ctx + kChunk - 1) / kChunk;
  const int s = n < kMaxSplits ? n : kMaxSplits;
  const int c = (n + s - 1) / s;
  *nchunks = n;
  *cps = c;
  *splits = (n + c - 1) / c;
}

template <bool ROPE_Q, bool FUSED_APPEND>
__global__ __launch_bounds__(kBlock) void k_attention(AttnArgs a) {
  const int split = blockIdx.x;
  const int g = blockIdx.y;
  const int t = blockIdx.z;
  const int past = a.d_pos ? *a.d_pos : a.past;
  const int pos = past + t;
  const int ctx = pos + 1;
  int nchunks, cps, nsplit;
  attn_splits(ctx, &nchunks, &cps, &nsplit);
  if (split >= nsplit) return;
  const int c0 = split * cps;
  const int c1 = min(c0 + cps, nchunks);
  const int group = a.heads / a.kv_heads;
  const int tid = threadIdx.x;

  __shared__ float qs[kMaxGroup][kHeadDim];
  __shared__ __attribute__((aligned(16))) _Float16 ks[kChunk][kHeadDim + 2];
  __shared__ __attribute__((aligned(16))) _Float16 vs[kChunk][kHeadDim];
  __shared__ float sc[kMaxGroup][kChunk];
  __shared__ float mst[kMaxGroup], lst[kMaxGroup], alpha[kMaxGroup];
  __shared__ __attribute__((aligned(16))) _Float16 knew[kHeadDim];
  __shared__ __attribute__((aligned(16))) _Float16 vnew[kHeadDim];
  __shared__ int is_last;

  const size_t qrow = (size_t)t * a.heads * kHeadDim;
  // Query heads g*group .. g*group+group-1 share kv head g (the blocked map of
  // src/core/attention.js:74-76).
  for (int idx = tid; idx < group * kHeadDim; idx += kBlock) {
    const int h = idx / kHeadDim, j = idx % kHeadDim;
    const float* qh_ = a.q + qrow + (size_t)(g * group + h) * kHeadDim;
    if constexpr (ROPE_Q) {
      // Half-split rotation from the f32 tables, as ROPE (kernels.js:380-388).
      const int jj = j & 31;
      const float c = a.cos_t[(size_t)pos * 32 + jj], s = a.sin_t[(size_t)pos * 32 + jj];
      const float lo = qh_[jj], hi = qh_[jj + 32];
      qs[h][j] = j < 32 ? lo * c - hi * s : hi * c + lo * s;
    } else {
      qs[h][j] = qh_[j];
    }
  }
  const bool owns_new = FUSED_APPEND && c1 == nchunks;
  if constexpr (FUSED_APPEND) {
    if (owns_new && tid < kHeadDim) {
      const int j = tid, jj = j & 31;
      const float* kh = a.k_new + (size_t)g * kHeadDim;
      const float c = a.cos_t[(size_t)pos * 32 + jj], s = a.sin_t[(size_t)pos * 32 + jj];
      const float lo = kh[jj], hi = kh[jj + 32];
      const float kr = j < 32 ? lo * c - hi * s : hi * c + lo * s;
      const _Float16 kh16 = (_Float16)kr;
      const _Float16 vh16 = (_Float16)a.v_new[(size_t)g * kHeadDim + j];
      knew[j] = kh16;
      vnew[j] = vh16;
      const size_t at = ((size_t)g * a.capacity + pos) * kHeadDim + j;
      a.kc[at] = __builtin_bit_cast(uint16_t, kh16);
      a.vc[at] = __builtin_bit_cast(uint16_t, vh16);
    }
  }
  if (tid < kMaxGroup) {
    mst[tid] = -INFINITY;
    lst[tid] = 0.f;
  }
  // Each thread owns outputs idx = tid and tid + 256 of [group][64].
  float acc0 = 0.f, acc1 = 0.f;
  const int o0 = tid, o1 = tid + kBlock;
  __syncthreads();

  const uint16_t* kbase = a.kc + (size_t)g * a.capacity * kHeadDim;
  const uint16_t* vbase = a.vc + (size_t)g * a.capacity * kHeadDim;
  for (int c = c0; c < c1; c++) {
    const int p0 = c * kChunk;
    const int n = min(kChunk, ctx - p0);
    // Stage K and V rows (128 B each) with 16-byte loads.
    for (int e = tid; e < kChunk * 8; e += kBlock) {
      const int p = e >> 3, part = e & 7;
      uint4 kv4 = make_uint4(0, 0, 0, 0), vv4 = make_uint4(0, 0, 0, 0);
      if (p < n) {
        if (FUSED_APPEND && owns_new && p0 + p == pos) {
          kv4 = *reinterpret_cast<const uint4*>(&knew[part * 8]);
          vv4 = *reinterpret_cast<const uint4*>(&vnew[part * 8]);
        } else {
          kv4 = reinterpret_cast<const uint4*>(kbase + (size_t)(p0 + p) * kHeadDim)[part];
          vv4 = reinterpret_cast<const uint4*>(vbase + (size_t)(p0 + p) * kHeadDim)[part];
        }
      }
      const uint32_t kw[4] = {kv4.x, kv4.y, kv4.z, kv4.w};
#pragma unroll
      for (int k = 0; k < 4; k++) {
        *reinterpret_cast<uint32_t*>(&ks[p][part * 8 + 2 * k]) = kw[k];
      }
      *reinterpret_cast<uint4*>(&vs[p][part * 8]) = vv4;
    }
    __syncthreads();
    // Scores, scaled by 1/sqrt(64) = 1/8 (exact in f32).
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
    // Online softmax update, one wave per head.
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

  // Partial (m, l, acc) for this split.
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

  // Combine the splits in split order.
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
