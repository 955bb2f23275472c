// Device building blocks shared by every kernel: wave64 reductions on DPP and
// ds_swizzle, the weight-chunk dot products for the three weight formats, the
// row-team matvec core (streamed and register-prefetched forms), and
// block-level staging helpers.
//
// Two arithmetics. The exact one follows the reference CPU path step for step
// (src/core/ops.js: f32 storage, f64 accumulation): a weight is first
// dequantized to the f32 the reference's loader would hold -- f32(q*scale),
// f32((level-zero)*scale), or the f16 value -- and then multiplied into an f64
// accumulator, so the only difference from the CPU is the order of an f64 sum
// (~1e-16 relative), which almost never survives the final rounding to f32. The
// fast one (the f32 core below) sums in f32 as the reference's WebGPU kernels do.
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
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kBlock = 256;

// ------------------------------------------------------------- reductions --
// Butterflies inside a team of TL lanes (TL = 16, 32 or 64): steps of 1, 2, 4
// and 8 lanes on DPP (quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror), 16 on ds_swizzle, 32 on a bpermute. Each step
// adds a symmetric pair, so every lane ends with the same bits. These patterns only
// read lanes of the same row, so bound_ctrl (zero for a missing source lane) never
// applies; set, it lets the compiler fold the move into the add (v_add_f32_dpp).
template <int CTRL>
__device__ __forceinline__ float dpp32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
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
// Byte b of u as f32 (one v_cvt_f32_ubyte).
template <int B>
__device__ __forceinline__ float ubyte(uint32_t u) {
  return (float)((u >> (8 * B)) & 0xffu);
}

// acc += sum over one chunk of w[i] * x[i] in f64, sequentially in i, where w[i]
// is the f32 weight the reference loader holds:
//   f16:  the f16 value (exact in f32);
//   int8: f32(q * scale)                       (src/core/quantize.js:60-68);
//   int4: f32(f64(level - zero) * scale), low nibble = even index (:134-151).
//
// Quantized chunks take a biased-byte form when the group allows it: the codes
// are offset so every byte is a non-negative integer m, converted with one
// v_cvt_f32_ubyte, and w = fma(m, scale, -bias*scale). The bias is a power of
// two, so -bias*scale is exact and the fused multiply-add rounds the exact value
// (m - bias) * scale = (level - zero) * scale once -- the reference's weight.
// The form needs scale > 0 and finite below 2^100 (no overflow in bias*scale,
// and the sign of a zero weight is +0 as the reference's is), and for int4 an
// integer zero point in [0, 15] (what the quantizer writes, quantize.js:115),
// so (level - zero + 16) is a byte in [1, 31] and four of them take one add.
// Other groups use the reference's arithmetic directly.
//
// x is the chunk's slice of the f64 activation vector, element e at
// b[(e/2)*ps + e%2]: pairs of consecutive elements are adjacent, and pair
// strides are either 2 (plain layout) or 2*nchunks (the chunk-transposed LDS
// layout of stage_*, where the 64 lanes of a team, each on its own chunk, read
// 64 consecutive 16-byte pairs -- no LDS bank conflicts, where the plain layout
// would put a whole wave on one bank).
struct XV {
  const double* b;
  int ps;
  __device__ __forceinline__ double operator[](int e) const { return b[(e >> 1) * ps + (e & 1)]; }
};

__device__ __forceinline__ double chunk_f16(const v4u w, const XV x, double acc) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; j++) {
    acc = fma((double)f16_lo(u[j]), x[2 * j], acc);
    acc = fma((double)f16_hi(u[j]), x[2 * j + 1], acc);
  }
  return acc;
}

__device__ __forceinline__ bool scale_biasable(float s) { return s > 0.f && s <= 0x1p100f; }

__device__ __forceinline__ double chunk_int8(const v4u w, const XV x, float s,
                                             double acc) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
  if (scale_biasable(s)) {
    const float c = -128.f * s;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t m = u[j] ^ 0x80808080u;  // q + 128 in every byte
      acc = fma((double)fmaf(ubyte<0>(m), s, c), x[4 * j + 0], acc);
      acc = fma((double)fmaf(ubyte<1>(m), s, c), x[4 * j + 1], acc);
      acc = fma((double)fmaf(ubyte<2>(m), s, c), x[4 * j + 2], acc);
      acc = fma((double)fmaf(ubyte<3>(m), s, c), x[4 * j + 3], acc);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const float wf = (float)(int8_t)(uint8_t)(u[j] >> (8 * b)) * s;  // q*s is exact before rounding
        acc = fma((double)wf, x[4 * j + b], acc);
      }
    }
  }
  return acc;
}

__device__ __forceinline__ double chunk_int4(const v4u w, const XV x, float s,
                                             float z, double acc) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
  const int zi = (int)z;
  if (scale_biasable(s) && (float)zi == z && (unsigned)zi <= 15u) {
    const float c = -16.f * s;
    const uint32_t bias = (uint32_t)(16 - zi) * 0x01010101u;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t ev = (u[j] & 0x0F0F0F0Fu) + bias;         // elements 8j, 8j+2, 8j+4, 8j+6
      const uint32_t od = ((u[j] >> 4) & 0x0F0F0F0Fu) + bias;  // elements 8j+1, +3, +5, +7
      acc = fma((double)fmaf(ubyte<0>(ev), s, c), x[8 * j + 0], acc);
      acc = fma((double)fmaf(ubyte<0>(od), s, c), x[8 * j + 1], acc);
      acc = fma((double)fmaf(ubyte<1>(ev), s, c), x[8 * j + 2], acc);
      acc = fma((double)fmaf(ubyte<1>(od), s, c), x[8 * j + 3], acc);
      acc = fma((double)fmaf(ubyte<2>(ev), s, c), x[8 * j + 4], acc);
      acc = fma((double)fmaf(ubyte<2>(od), s, c), x[8 * j + 5], acc);
      acc = fma((double)fmaf(ubyte<3>(ev), s, c), x[8 * j + 6], acc);
      acc = fma((double)fmaf(ubyte<3>(od), s, c), x[8 * j + 7], acc);
    }
  } else {
    const double zd = z, sd = s;
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
      for (int n = 0; n < 8; n++) {
        const float wf = (float)(((double)((u[j] >> (4 * n)) & 0xfu) - zd) * sd);
        acc = fma((double)wf, x[8 * j + n], acc);
      }
    }
  }
  return acc;
}

// The same chunk dots for R rows at once, element-major: the R accumulation
// chains interleave (so a lone wave is not stalled on one chain's f64 latency)
// and each x element is read once for all rows. Each row's sum still runs over
// its elements in ascending order, so the results are those of chunk_*.
template <int R>
__device__ __forceinline__ void chunk_rows_f16(const v4u (&w)[R], const XV x, double (&acc)[R]) {
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const double x0 = x[2 * j], x1 = x[2 * j + 1];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = fma((double)f16_lo(w[r][j]), x0, acc[r]);
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = fma((double)f16_hi(w[r][j]), x1, acc[r]);
  }
}

template <int R>
__device__ __forceinline__ void chunk_rows_int8(const v4u (&w)[R], const XV x, const float (&s)[R],
                                                double (&acc)[R]) {
  bool fast = true;
#pragma unroll
  for (int r = 0; r < R; r++) fast = fast && scale_biasable(s[r]);
  if (fast) {
    float c[R];
#pragma unroll
    for (int r = 0; r < R; r++) c[r] = -128.f * s[r];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint32_t m[R];
#pragma unroll
      for (int r = 0; r < R; r++) m[r] = w[r][j] ^ 0x80808080u;  // q + 128 in every byte
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const double xb = x[4 * j + b];
#pragma unroll
        for (int r = 0; r < R; r++)
          acc[r] = fma((double)fmaf((float)((m[r] >> (8 * b)) & 0xffu), s[r], c[r]), xb, acc[r]);
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = chunk_int8(w[r], x, s[r], acc[r]);
  }
}

template <int R>
__device__ __forceinline__ void chunk_rows_int4(const v4u (&w)[R], const XV x, const float (&s)[R],
                                                const float (&z)[R], double (&acc)[R]) {
  bool fast = true;
  int zi[R];
#pragma unroll
  for (int r = 0; r < R; r++) {
    zi[r] = (int)z[r];
    fast = fast && scale_biasable(s[r]) && (float)zi[r] == z[r] && (unsigned)zi[r] <= 15u;
  }
  if (fast) {
    float c[R];
    uint32_t bias[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      c[r] = -16.f * s[r];
      bias[r] = (uint32_t)(16 - zi[r]) * 0x01010101u;
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint32_t ev[R], od[R];
#pragma unroll
      for (int r = 0; r < R; r++) {
        ev[r] = (w[r][j] & 0x0F0F0F0Fu) + bias[r];         // elements 8j, 8j+2, 8j+4, 8j+6
        od[r] = ((w[r][j] >> 4) & 0x0F0F0F0Fu) + bias[r];  // elements 8j+1, +3, +5, +7
      }
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const double xe = x[8 * j + 2 * b], xo = x[8 * j + 2 * b + 1];
#pragma unroll
        for (int r = 0; r < R; r++)
          acc[r] = fma((double)fmaf((float)((ev[r] >> (8 * b)) & 0xffu), s[r], c[r]), xe, acc[r]);
#pragma unroll
        for (int r = 0; r < R; r++)
          acc[r] = fma((double)fmaf((float)((od[r] >> (8 * b)) & 0xffu), s[r], c[r]), xo, acc[r]);
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = chunk_int4(w[r], x, s[r], z[r], acc[r]);
  }
}

// ------------------------------------------------------------ matvec core --
// Where element i of an f64 activation vector sits in a staged copy:
// chunk-transposed (XT) for a matrix with W = 1 << lw weights per chunk and nc
// chunks per row -- pair (i%W)/2 of every chunk together, chunk-minor -- else
// plain. XV over either layout reads the same elements in the same order.
struct XLayout {
  int lw, nc;  // plain: lw = 13 (W >= any staged length), nc = 1
  __device__ __forceinline__ int pos(int i) const {
    const int e = i & ((1 << lw) - 1);
    return (((e >> 1) * nc + (i >> lw)) << 1) | (i & 1);
  }
};
constexpr XLayout kPlain = {13, 1};
template <int FMT>
__host__ __device__ inline XLayout chunk_layout(int nchunks) {
  constexpr int lw = FMT == QH_FMT_F16 ? 3 : FMT == QH_FMT_INT8 ? 4 : 5;
  return XLayout{lw, nchunks};
}

// A team of TL lanes computes R rows (row indices in `rows`, each < m.rows) for
// NB positions. Lane `tl` handles chunks tl, tl+TL, ... of every row, so the x
// chunk it reads is reused across the R rows. x for position b is f64 at
// xs + b*xstride (LDS or global), chunk-transposed when XT. On return every
// lane of the team holds the R*NB f64 sums.
template <int FMT, int R, int NB, int TL, bool XT>
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
      const XV xc = XT ? XV{xs + (size_t)b * xstride + 2 * c, 2 * m.nchunks}
                       : XV{xs + (size_t)b * xstride + (size_t)c * W, 2};
      if constexpr (FMT == QH_FMT_F16) chunk_rows_f16<R>(w, xc, acc[b]);
      else if constexpr (FMT == QH_FMT_INT8) chunk_rows_int8<R>(w, xc, srow, acc[b]);
      else chunk_rows_int4<R>(w, xc, s, z, acc[b]);
    }
  }
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int i = 0; i < R; i++) acc[b][i] = team_sum<TL>(acc[b][i]);
}

// The same sums with a lane's whole share of R rows -- at most KC chunks per
// row -- loaded into registers first (WTile), so the loads of a work item are in
// flight together, ahead of the activation staging and of the previous item's
// arithmetic. Chunks are summed in the order mv_team sums them.
template <int FMT, int R, int KC>
struct WTile {
  v4u w[KC][R];
  float s[KC][R];  // int4: group scale of each chunk; int8: row scale in s[0]
  float z[KC][R];  // int4: group zero point
};

// Weights are streamed (non-temporal loads). STREAM_S: the scales and zero points too -- for a
// launch whose teams take one item each (the decode step's layer launches), where every
// scale line is used once per step, so streaming it leaves the caches to what is read again
// (the KV cache, the activations): decode 2183 -> 2195 tok/s. Teams walking several items
// share a scale line between consecutive items, and streaming it cost the streaming grids 1-4
// points of HBM peak.
template <int FMT, int R, int KC, int TL, bool STREAM_S = false>
__device__ __forceinline__ void wtile_load(const DMat& m, const int (&rows)[R], int tl,
                                           WTile<FMT, R, KC>& t) {
  // Unconditional loads (a lane past the row end re-reads the row's last chunk,
  // which wtile_dot skips): no branch, so no load has to wait for a merge.
  auto scale = [](const float* p) { return STREAM_S ? __builtin_nontemporal_load(p) : *p; };
#pragma unroll
  for (int k = 0; k < KC; k++) {
    const int c = min(tl + k * TL, m.nchunks - 1);
#pragma unroll
    for (int i = 0; i < R; i++) {
      const v4u* rp = reinterpret_cast<const v4u*>(m.data + (size_t)rows[i] * m.row_bytes);
      t.w[k][i] = __builtin_nontemporal_load(&rp[c]);
    }
    if constexpr (FMT == QH_FMT_INT4) {
      const int g = c / m.cpg;
#pragma unroll
      for (int i = 0; i < R; i++) {
        t.s[k][i] = scale(&m.scales[(size_t)rows[i] * m.gpr + g]);
        t.z[k][i] = scale(&m.zeros[(size_t)rows[i] * m.gpr + g]);
      }
    }
  }
  if constexpr (FMT == QH_FMT_INT8) {
#pragma unroll
    for (int i = 0; i < R; i++) t.s[0][i] = scale(&m.scales[rows[i]]);
  }
}

// A matrix's arrays as buffer resources. A load through one takes a 32-bit per-lane
// byte offset, and the hardware checks it against the array's size: a read past the
// end returns zeros instead of touching memory. (The check covers the per-lane offset
// and the instruction's immediate, not the scalar offset, so every offset here is
// per-lane and the scalar offset is 0.) The arrays must be under 4 GiB.
struct BufMat {
  __amdgpu_buffer_rsrc_t data, scales, zeros;
};
constexpr int kRawBufferWord3 = 0x00020000;  // raw (unformatted) buffer, stride 0
constexpr int kLoadNonTemporal = 2;          // the load's cache policy: streamed, not kept
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_buffer(const void* p, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)(uint32_t)bytes, kRawBufferWord3);
}
// The matrix, or `copies` copies of it laid out copy_w bytes (data) and copy_s floats
// (scales, zero points) apart.
__device__ __forceinline__ BufMat buf_mat(const DMat& m, int copies = 1, size_t copy_w = 0, size_t copy_s = 0) {
  const size_t n = (size_t)m.rows * (m.format == QH_FMT_INT4 ? m.gpr : 1);
  const size_t nw = (size_t)m.rows * m.row_bytes;
  const size_t ns = ((size_t)(copies - 1) * copy_s + n) * sizeof(float);
  BufMat b;
  b.data = raw_buffer(m.data, (size_t)(copies - 1) * copy_w + nw);
  b.scales = raw_buffer(m.scales, m.format == QH_FMT_F16 ? 0 : ns);
  b.zeros = raw_buffer(m.zeros, m.format == QH_FMT_INT4 ? ns : 0);
  return b;
}

// wtile_load through buffer resources, for rows that may lie past the matrix (a loop
// over rows that loads ahead): no clamping, 32-bit offsets, and what lies past the end
// reads as zeros (those rows' sums are never used; nor are chunks past a row's end).
// wbase / sbase: byte offsets of the matrix's data and scales inside the resources.
template <int FMT, int R, int KC, int TL>
__device__ __forceinline__ void wtile_load_buf(const DMat& m, const BufMat& b, const int (&rows)[R], int tl,
                                               int wbase, int sbase, WTile<FMT, R, KC>& t) {
#pragma unroll
  for (int k = 0; k < KC; k++) {
    const int c = tl + k * TL;
#pragma unroll
    for (int i = 0; i < R; i++)
      t.w[k][i] =
          __builtin_amdgcn_raw_buffer_load_b128(b.data, wbase + rows[i] * m.row_bytes + 16 * c, 0, kLoadNonTemporal);
    if constexpr (FMT == QH_FMT_INT4) {
      const int g = c / m.cpg;
#pragma unroll
      for (int i = 0; i < R; i++) {
        const int off = sbase + (rows[i] * m.gpr + g) * (int)sizeof(float);
        t.s[k][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(b.scales, off, 0, 0));
        t.z[k][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(b.zeros, off, 0, 0));
      }
    }
  }
  if constexpr (FMT == QH_FMT_INT8) {
#pragma unroll
    for (int i = 0; i < R; i++)
      t.s[0][i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(b.scales, sbase + rows[i] * 4, 0, 0));
  }
}

// xs is chunk-transposed (chunk_layout<FMT>(m.nchunks)).
template <int FMT, int R, int KC, int TL>
__device__ __forceinline__ void wtile_dot(const DMat& m, const WTile<FMT, R, KC>& t, const double* xs,
                                          int tl, double (&acc)[R]) {
#pragma unroll
  for (int i = 0; i < R; i++) acc[i] = 0.0;
#pragma unroll
  for (int k = 0; k < KC; k++) {
    const int c = tl + k * TL;
    if (c < m.nchunks) {
      const XV xc{xs + 2 * c, 2 * m.nchunks};
      if constexpr (FMT == QH_FMT_F16) chunk_rows_f16<R>(t.w[k], xc, acc);
      else if constexpr (FMT == QH_FMT_INT8) chunk_rows_int8<R>(t.w[k], xc, t.s[0], acc);
      else chunk_rows_int4<R>(t.w[k], xc, t.s[k], t.z[k], acc);
    }
  }
#pragma unroll
  for (int i = 0; i < R; i++) acc[i] = team_sum<TL>(acc[i]);
}

// ------------------------------------------------- f32 matvec core (FAST) --
// QH_NUMERICS_FAST sums every output in f32, as the reference's WebGPU kernels
// do (weights f16 in storage, activations f32, f32 accumulation; README.md
// "Precision is stated rather than inherited", src/gpu/kernels.js:33-79). The
// activations are the same f32 values the exact path stages; only the sums
// differ, by f32 rounding (~sqrt(n) * 2^-24 relative).
//
// Quantized chunks take the scale out of the sum: an int8 chunk contributes
// sum((q+128) x) - 128 sum(x), an int4 chunk scale * (sum(level x) - zero sum(x)),
// with the int8 codes converted by one v_cvt_f32_ubyte each (biased by an xor), so
// an int8 weight costs one conversion and one f32 fma. int4 codes need no
// conversion: a nibble masked in place in the low byte of a 16-bit half is the f16
// subnormal level * 2^-24 (odd nibbles, masked as 16*level, rescaled by the exact
// 1/16 once per chunk), which v_fma_mix_f32 reads directly; four masks and one
// shift unpack 8 levels, so 8 int4 weights cost 13 VALU ops instead of 18. The sums
// run 2^-24 below the scale of the f32 form, and scaling by a power of two commutes
// with rounding, so they carry the same bits (the scale folds 2^24 back in) while
// every partial sum stays a normal f32 (|partial| >= 2^-102, or zero).
// sum(x) over each chunk (the "chunk sum") is computed once, while staging,
// as a pairwise tree: ((x0+x1)+(x2+x3)) per 4-element group, then a butterfly
// over the chunk's groups. A row's chunk contributions are added in ascending
// chunk order per lane, then across the team by team_sum, so every path over a
// matrix (decode tile, streamed prefill tile) sums one output in one order.
//
// Staged f32 layout (XLayoutF): 4-element group g of chunk c at float offset
// 4*(g*nc + c) -- the team's lanes, each on its own chunk, read consecutive
// 16-byte slots (ds_read_b128 without bank conflicts).
struct XLayoutF {
  int lw, nc;  // W = 1 << lw elements per chunk, nc chunks per row
  __device__ __forceinline__ int pos(int i) const {
    const int e = i & ((1 << lw) - 1);
    return (((e >> 2) * nc + (i >> lw)) << 2) | (e & 3);
  }
};
template <int FMT>
__host__ __device__ inline XLayoutF chunk_layout_f(int nchunks) {
  constexpr int lw = FMT == QH_FMT_F16 ? 3 : FMT == QH_FMT_INT8 ? 4 : 5;
  return XLayoutF{lw, nchunks};
}

// Floats of LDS an f32-staged vector of `cols` values (a multiple of 4) takes: the
// values, then one chunk sum per chunk, rounded up to whole 16-byte groups.
__host__ __device__ inline int staged_f32_floats(int cols, int nchunks) { return cols + ((nchunks + 3) & ~3); }

// The chunk sum over the G lanes (G = 4-element groups per chunk: int8 4, int4 8)
// that hold one chunk's groups, from each lane's group sum; every lane of the G
// ends with the same bits (each step adds a symmetric pair).
template <int G>
__device__ __forceinline__ float chunk_group_sum(float s4) {
  static_assert(G == 4 || G == 8, "lanes per chunk");
  s4 += dpp32<kDppQuadXor1>(s4);
  s4 += dpp32<kDppQuadXor2>(s4);
  if constexpr (G == 8) s4 += dpp32<kDppHalfMirror>(s4);
  return s4;
}

// Stores 4-element group gi (value v) of an f32-staged vector and, for quantized
// formats, its chunk's sum into sxs[gi / G]. Every lane of the wave must call it
// together (the chunk sum is a cross-lane butterfly); `valid` false for lanes past
// the vector, whose groups only complete chunks that do not exist.
template <int FMT>
__device__ __forceinline__ void stage_group_f32(v4f v, int gi, bool valid, float* xs, float* sxs,
                                                XLayoutF lay) {
  if (valid) *reinterpret_cast<v4f*>(xs + lay.pos(4 * gi)) = v;
  if constexpr (FMT != QH_FMT_F16) {
    constexpr int G = Fmt<FMT>::kW / 4;
    float s4 = valid ? (v.x + v.y) + (v.z + v.w) : 0.f;
    s4 = chunk_group_sum<G>(s4);
    if (valid && (gi & (G - 1)) == 0) sxs[gi / G] = s4;
  }
}

// One staged chunk of an f32 activation in registers: its 4-element groups (read from
// p + g*gs, group g of the chunk) and, for quantized formats, its chunk sum.
template <int FMT>
struct XChunk {
  v4f g[Fmt<FMT>::kW / 4];
  float sx;
  __device__ __forceinline__ void load(const float* __restrict__ p, int gs, float chunk_sum) {
#pragma unroll
    for (int k = 0; k < Fmt<FMT>::kW / 4; k++) g[k] = *reinterpret_cast<const v4f*>(p + k * gs);
    sx = chunk_sum;
  }
};

// acc[r] += the f32 dot of chunk row w[r] with the chunk x, for R rows element-major.
// s/z: int4 group scale and zero point of each row (int8 takes its row scale after the
// team sum).
template <int FMT, int R>
__device__ __forceinline__ void chunk_rows_f32_x(const v4u (&w)[R], const XChunk<FMT>& x, const float (&s)[R],
                                                 const float (&z)[R], float (&acc)[R]) {
  const float sx = x.sx;
  if constexpr (FMT == QH_FMT_F16) {
    const v4f x0 = x.g[0];
    const v4f x1 = x.g[1];
    const float xe[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
#pragma unroll
      for (int r = 0; r < R; r++) acc[r] = fmaf(f16_lo(w[r][k]), xe[2 * k], acc[r]);
#pragma unroll
      for (int r = 0; r < R; r++) acc[r] = fmaf(f16_hi(w[r][k]), xe[2 * k + 1], acc[r]);
    }
  } else if constexpr (FMT == QH_FMT_INT8) {
    const float c0 = -128.f * sx;  // exact
    const v4f(&xg)[4] = x.g;
    float d[R];
#pragma unroll
    for (int r = 0; r < R; r++) d[r] = c0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const v4f x = xg[k];
#pragma unroll
      for (int r = 0; r < R; r++) {
        const uint32_t m = w[r][k] ^ 0x80808080u;  // q + 128 in every byte
        d[r] = fmaf(ubyte<0>(m), x.x, d[r]);
        d[r] = fmaf(ubyte<1>(m), x.y, d[r]);
        d[r] = fmaf(ubyte<2>(m), x.z, d[r]);
        d[r] = fmaf(ubyte<3>(m), x.w, d[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] += d[r];
  } else {
    // The sums below are the f32 form's sums times 2^-24 (see the f32 core's notes).
    float pe[R], po[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      pe[r] = -z[r] * sx * 0x1p-24f;
      po[r] = 0.f;
    }
    const v4f(&xg)[8] = x.g;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      // dword k holds elements 8k .. 8k+7: byte b = (element 8k+2b) | (element 8k+2b+1) << 4.
      // Halves of m0: elements 8k, 8k+4; m1: 16x 8k+1, 8k+5; m2: 8k+2, 8k+6; m3: 16x 8k+3, 8k+7.
      const v4f xa = xg[2 * k], xb = xg[2 * k + 1];
#pragma unroll
      for (int r = 0; r < R; r++) {
        const uint32_t d = w[r][k], d8 = d >> 8;
        const uint32_t m0 = d & 0x000F000Fu, m1 = d & 0x00F000F0u;
        const uint32_t m2 = d8 & 0x000F000Fu, m3 = d8 & 0x00F000F0u;
        pe[r] = fmaf(f16_lo(m0), xa.x, pe[r]);
        po[r] = fmaf(f16_lo(m1), xa.y, po[r]);
        pe[r] = fmaf(f16_lo(m2), xa.z, pe[r]);
        po[r] = fmaf(f16_lo(m3), xa.w, po[r]);
        pe[r] = fmaf(f16_hi(m0), xb.x, pe[r]);
        po[r] = fmaf(f16_hi(m1), xb.y, po[r]);
        pe[r] = fmaf(f16_hi(m2), xb.z, pe[r]);
        po[r] = fmaf(f16_hi(m3), xb.w, po[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = fmaf(s[r] * 0x1p24f, fmaf(po[r], 0.0625f, pe[r]), acc[r]);
  }
}

// The same with the chunk read from LDS (group g at p + g*gs, all read before any
// arithmetic) and its chunk sum sx.
template <int FMT, int R>
__device__ __forceinline__ void chunk_rows_f32(const v4u (&w)[R], const float* __restrict__ p, int gs,
                                               const float (&s)[R], const float (&z)[R], float sx,
                                               float (&acc)[R]) {
  XChunk<FMT> x;
  x.load(p, gs, sx);
  chunk_rows_f32_x<FMT, R>(w, x, s, z, acc);
}

// a * b rounded on its own: never fused into a multiply-add with the operation that
// consumes it (HIP's __fmul_rn is a plain, contractible multiply).
__device__ __forceinline__ float mul_rounded(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

// The output of a team-summed f32 row: int8 applies the row scale, rounded before
// any later add (the decode epilogue and the prefill's separate residual add see the
// same value).
template <int FMT>
__device__ __forceinline__ float row_out_f32(float sum, float srow) {
  if constexpr (FMT == QH_FMT_INT8) return mul_rounded(srow, sum);
  else return sum;
}

// wtile_dot in f32: xs is staged by stage_group_f32 (values, then chunk sums at
// xs + m.cols). Returns the team sums with the int8 row scale applied.
template <int FMT, int R, int KC, int TL>
__device__ __forceinline__ void wtile_dot_f32(const DMat& m, const WTile<FMT, R, KC>& t, const float* xs,
                                              int tl, float (&acc)[R]) {
  const float* sxs = xs + m.cols;
#pragma unroll
  for (int i = 0; i < R; i++) acc[i] = 0.f;
#pragma unroll
  for (int k = 0; k < KC; k++) {
    const int c = tl + k * TL;
    if (c < m.nchunks) {
      const float sx = FMT == QH_FMT_F16 ? 0.f : sxs[c];
      chunk_rows_f32<FMT, R>(t.w[k], xs + 4 * c, 4 * m.nchunks, t.s[k], t.z[k], sx, acc);
    }
  }
#pragma unroll
  for (int i = 0; i < R; i++) acc[i] = row_out_f32<FMT>(team_sum<TL>(acc[i]), t.s[0][i]);
}

// wtile_dot_f32 for one chunk per lane (KC = 1) whose staged chunk is already in
// registers (x: chunk tl, read once by a team that sums many items against it).
template <int FMT, int R, int TL>
__device__ __forceinline__ void wtile_dot_f32_x(const DMat& m, const WTile<FMT, R, 1>& t, const XChunk<FMT>& x,
                                                int tl, float (&acc)[R]) {
#pragma unroll
  for (int i = 0; i < R; i++) acc[i] = 0.f;
  if (tl < m.nchunks) chunk_rows_f32_x<FMT, R>(t.w[0], x, t.s[0], t.z[0], acc);
#pragma unroll
  for (int i = 0; i < R; i++) acc[i] = row_out_f32<FMT>(team_sum<TL>(acc[i]), t.s[0][i]);
}

// mv_team in f32 over NB positions staged at xs + b*xstride (each a stage_group_f32
// vector: values, then chunk sums at + m.cols).
template <int FMT, int R, int NB, int TL>
__device__ __forceinline__ void mv_team_f32(const DMat& m, const int (&rows)[R], const float* xs, int xstride,
                                            int tl, float (&acc)[NB][R]) {
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int i = 0; i < R; i++) acc[b][i] = 0.f;
  const v4u* rp[R];
#pragma unroll
  for (int i = 0; i < R; i++) rp[i] = reinterpret_cast<const v4u*>(m.data + (size_t)rows[i] * m.row_bytes);
  float srow[R] = {};
  if constexpr (FMT == QH_FMT_INT8) {
#pragma unroll
    for (int i = 0; i < R; i++) srow[i] = m.scales[rows[i]];
  }
  for (int c = tl; c < m.nchunks; c += TL) {
    v4u w[R];
#pragma unroll
    for (int i = 0; i < R; i++) w[i] = __builtin_nontemporal_load(&rp[i][c]);
    float s[R] = {}, z[R] = {};
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
      const float* xb = xs + (size_t)b * xstride;
      const float sx = FMT == QH_FMT_F16 ? 0.f : xb[m.cols + c];
      chunk_rows_f32<FMT, R>(w, xb + 4 * c, 4 * m.nchunks, s, z, sx, acc[b]);
    }
  }
#pragma unroll
  for (int b = 0; b < NB; b++)
#pragma unroll
    for (int i = 0; i < R; i++) acc[b][i] = row_out_f32<FMT>(team_sum<TL>(acc[b][i]), srow[i]);
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
// Vectors of up to kStageMax f32 values are staged with every load of a thread
// issued before any is used: thread t owns the float4 groups t, t+kBlock, ...
constexpr int kStageVec = 8;                           // float4 groups per thread
constexpr int kStageMax = kStageVec * 4 * kBlock;      // 8192 values

// Staging is split into the loads (StageIn::load) and the arithmetic
// (stage_*_finish), so a kernel can issue its activation loads before its weight
// loads: vector loads return in issue order, and waiting for an activation that
// was issued after the weights would wait for the weights too.
struct StageIn {
  v4f v[kStageVec], g[kStageVec];
  // x (and gain, when given) for n values; n a multiple of 4 and at most kStageMax,
  // both 16-byte aligned.
  __device__ __forceinline__ void load(const float* __restrict__ x, const float* __restrict__ gain, int n) {
    const int n4 = n >> 2;
#pragma unroll
    for (int j = 0; j < kStageVec; j++) {
      const int i = threadIdx.x + j * kBlock;
      if (i < n4) {
        v[j] = reinterpret_cast<const v4f*>(x)[i];
        if (gain) g[j] = reinterpret_cast<const v4f*>(gain)[i];
      }
    }
  }
  // The gain alone; x follows from load_bf16 once its row is known.
  __device__ __forceinline__ void load_gain(const float* __restrict__ gain, int n) {
    const int n4 = n >> 2;
#pragma unroll
    for (int j = 0; j < kStageVec; j++) {
      const int i = threadIdx.x + j * kBlock;
      if (i < n4) g[j] = reinterpret_cast<const v4f*>(gain)[i];
    }
  }
  // x = the bf16 values of `row` widened exactly (row 8-byte aligned).
  __device__ __forceinline__ void load_bf16(const uint16_t* __restrict__ row, int n) {
    const int n4 = n >> 2;
#pragma unroll
    for (int j = 0; j < kStageVec; j++) {
      const int i = threadIdx.x + j * kBlock;
      if (i < n4) {
        const uint2 u = reinterpret_cast<const uint2*>(row)[i];  // little-endian: element 4i in u.x's low half
        v[j] = v4f{__builtin_bit_cast(float, u.x << 16), __builtin_bit_cast(float, u.x & 0xffff0000u),
                   __builtin_bit_cast(float, u.y << 16), __builtin_bit_cast(float, u.y & 0xffff0000u)};
      }
    }
  }
  // x[0 .. n-1] = the staged values.
  __device__ __forceinline__ void store(float* __restrict__ x, int n) const {
    const int n4 = n >> 2;
#pragma unroll
    for (int j = 0; j < kStageVec; j++) {
      const int i = threadIdx.x + j * kBlock;
      if (i < n4) reinterpret_cast<v4f*>(x)[i] = v[j];
    }
  }
};

// xs = x / sqrt(mean(x^2) + eps) * gain as f64 values of the f32 result, with
// the statistic and the products in f64 as src/core/ops.js:17-24 evaluates
// them, so the normalized vector is the CPU's up to the order of the f64 sum.
// `in` holds x and gain (StageIn::load); element i goes to xs[lay.pos(i)].
__device__ __forceinline__ void stage_rmsnorm_finish(const StageIn& in, double eps, int cols, double* xs,
                                                     double* red, XLayout lay) {
  const int n4 = cols >> 2;
  double ss = 0;
#pragma unroll
  for (int j = 0; j < kStageVec; j++) {
    if (threadIdx.x + j * kBlock < n4) {
#pragma unroll
      for (int e = 0; e < 4; e++) ss = fma((double)in.v[j][e], (double)in.v[j][e], ss);  // v*v exact in f64
    }
  }
  ss = block_sum_f64(ss, red);
  const double scale = 1.0 / sqrt(ss / cols + eps);
#pragma unroll
  for (int j = 0; j < kStageVec; j++) {
    const int i = threadIdx.x + j * kBlock;
    if (i < n4) {
#pragma unroll
      for (int e = 0; e < 4; e++)
        xs[lay.pos(4 * i + e)] = (double)(float)((double)in.v[j][e] * scale * (double)in.g[j][e]);
    }
  }
  __syncthreads();
}

__device__ __forceinline__ void stage_rmsnorm(const float* __restrict__ x,
                                              const float* __restrict__ gain, double eps, int cols,
                                              double* xs, double* red, XLayout lay) {
  StageIn in;
  in.load(x, gain, cols);
  stage_rmsnorm_finish(in, eps, cols, xs, red, lay);
}

// stage_rmsnorm for any cols and alignment, one element per thread and step.
__device__ __forceinline__ void stage_rmsnorm_scalar(const float* __restrict__ x,
                                                     const float* __restrict__ gain, double eps,
                                                     int cols, double* xs, double* red) {
  double ss = 0;
  for (int i = threadIdx.x; i < cols; i += kBlock) {
    const double v = x[i];
    xs[i] = v;
    ss = fma(v, v, ss);
  }
  ss = block_sum_f64(ss, red);
  const double scale = 1.0 / sqrt(ss / cols + eps);
  for (int i = threadIdx.x; i < cols; i += kBlock) xs[i] = (double)(float)(xs[i] * scale * (double)gain[i]);
  __syncthreads();
}

// xs = (double)x for an f32 vector (same bounds and layout as stage_rmsnorm).
__device__ __forceinline__ void stage_copy_finish(const StageIn& in, int n, double* xs, XLayout lay) {
  const int n4 = n >> 2;
#pragma unroll
  for (int j = 0; j < kStageVec; j++) {
    const int i = threadIdx.x + j * kBlock;
    if (i < n4) {
#pragma unroll
      for (int e = 0; e < 4; e++) xs[lay.pos(4 * i + e)] = (double)in.v[j][e];
    }
  }
  __syncthreads();
}

// rmsnorm in f32 for fast numerics, the WGSL RMSNORM's arithmetic
// (src/gpu/kernels.js:300-341): an f32 sum of squares, scale = inverseSqrt(sum / cols
// + eps), y = x * scale * gain. Both the decode staging and the prefill's rmsnorm
// launch evaluate it with the same thread-to-element map (StageIn), so they agree
// bit for bit.
//
// Sum over the block in f32, fixed order; `red` (kBlock/kWave floats of LDS) must not
// be reused before the caller's next barrier.
__device__ __forceinline__ float block_sum_f32(float v, float* red) {
  v = team_sum<64>(v);
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kBlock / kWave; w++) t += red[w];
  return t;
}

__device__ __forceinline__ float rms_scale_f32(const StageIn& in, int cols, float eps, float* red) {
  const int n4 = cols >> 2;
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kStageVec; j++) {
    if (threadIdx.x + j * kBlock < n4) {
#pragma unroll
      for (int e = 0; e < 4; e++) ss = fmaf(in.v[j][e], in.v[j][e], ss);
    }
  }
  ss = block_sum_f32(ss, red);
  return __builtin_amdgcn_rsqf(ss / (float)cols + eps);
}

__device__ __forceinline__ v4f rms_apply_f32(v4f v, float scale, v4f g) {
  v4f y;
#pragma unroll
  for (int e = 0; e < 4; e++) y[e] = mul_rounded(mul_rounded(v[e], scale), g[e]);
  return y;
}

// The staging above for the f32 core: the f32 rmsnorm, stored by stage_group_f32
// with the chunk sums after the `cols` values.
template <int FMT>
__device__ __forceinline__ void stage_rmsnorm_finish_f32(const StageIn& in, float eps, int cols, float* xs,
                                                         float* red, XLayoutF lay) {
  const int n4 = cols >> 2;
  const float scale = rms_scale_f32(in, cols, eps, red);
#pragma unroll
  for (int j = 0; j < kStageVec; j++) {
    if (j * kBlock < n4) {  // uniform over the block
      const int i = threadIdx.x + j * kBlock;
      const bool valid = i < n4;
      v4f v = {0.f, 0.f, 0.f, 0.f};
      if (valid) v = rms_apply_f32(in.v[j], scale, in.g[j]);
      stage_group_f32<FMT>(v, i, valid, xs, xs + cols, lay);
    }
  }
  __syncthreads();
}

template <int FMT>
__device__ __forceinline__ void stage_copy_finish_f32(const StageIn& in, int n, float* xs, XLayoutF lay) {
  const int n4 = n >> 2;
#pragma unroll
  for (int j = 0; j < kStageVec; j++) {
    if (j * kBlock < n4) {
      const int i = threadIdx.x + j * kBlock;
      const bool valid = i < n4;
      const v4f zero = {0.f, 0.f, 0.f, 0.f};
      stage_group_f32<FMT>(valid ? in.v[j] : zero, i, valid, xs, xs + n, lay);
    }
  }
  __syncthreads();
}

// silu(g) * u in f32 for the reference's WGSL SWIGLU (src/gpu/kernels.js:502-514), g / (1 + e^-g)
// * up: WGSL bounds exp and division by a few ulps rather than rounding them correctly, and here
// e^-g is the hardware exp2 of a fraction in [-0.5, 0.5] scaled by 2^rint (the range where
// v_exp_f32 is accurate to about an ulp) and the division the hardware reciprocal -- ~9 VALU
// instructions against ~30 for a correctly rounded expf and division, a few ulps from them. A
// large negative g gives e = inf and -0; a non-finite g or u gives a non-finite value.
__device__ __forceinline__ float swiglu_f32(float g, float u) {
  const float t = -g * 1.44269504088896340736f;
  const float n = __builtin_rintf(t);
  const float e = __builtin_ldexpf(__builtin_amdgcn_exp2f(t - n), (int)n);
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
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
