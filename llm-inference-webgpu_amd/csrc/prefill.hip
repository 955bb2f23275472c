// Batched-prefill contraction on the matrix cores: Y[M, N] = X[M, K] . W^T for
// int8 (per-row scale) and int4 (per-group scale and zero point) weights in the
// reference quantizer's layout (src/core/quantize.js:36-151). The reference has no
// GEMM: its prefill reads each weight once per <= 8 positions (batchedMatvec,
// src/gpu/kernels.js:232-290); this is the M = 512 contraction that replaces it.
//
// Arithmetic: integers on v_mfma_i32_16x16x64_i8. A weight code is already a small
// integer: int8 q in [-127, 127], int4 (level - zero) in [-15, 15]. Each activation
// row is made one too, once per contraction by the row kernel that produces it (k_rows:
// the previous contraction's split sum, residual add, rmsnorm or swiglu, then the
// digits): with s = max|x_row| / 127, every x
// becomes the fixed-point integer X = rint(x * 2^16 / s), |X| <= 127 * 2^16, an
// absolute error of at most s * 2^-17 = max|x_row| * 2^-17 / 127 (the row's largest
// value keeps 24 significant bits, as in f32), stored as three balanced base-256
// digits X = d0 + 256 d1 + 65536 d2, each an int8. The three digit planes go through
// the int8 MFMA against the raw codes, so every product and every sum is exact in
// int32 (|d q| <= 128 * 127, times at most 2^17 columns, stays below 2^31), and the
// digits are recombined in f64 (S0 + 256 S1 + 65536 S2, exact) only at the end: for
// int8 once per output, for int4 once per group, scaled by the group's scale into an
// f64 running total. The output is that total times s * 2^-16 (and the int8 row
// scale), rounded once to f32.
//
// Tiling. A block of four waves computes 64 positions x 128 weight rows, each wave
// owning 16 positions (1 x 8 MFMA tiles of 16 x 16), stepping K by 64. The weight tile
// (128 x 64 codes, int4 expanded to int8) is staged in one of two LDS buffers, one
// barrier per step; each wave loads its three digit fragments (one contiguous 1 KB run
// per digit in the step-major digit layout) straight from global memory, three steps ahead. A step is 24 MFMAs per wave
// against 8 LDS fragment reads and no per-element vector arithmetic for int8 weights.
// Long K is split over gridDim.z; partial tiles are summed in a fixed order by
// k_gemm_finish.
#include <algorithm>
#include <type_traits>
#include <utility>

#include "device_common.h"

namespace qh {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGM = 64, kGN = 128, kGK = 64;
constexpr int kDigits = 3;                    // base-256 digits of an activation
constexpr int kGemmWaves = 4;                 // waves per block, 16 positions each
constexpr int kGemmThreads = kGemmWaves * kWave;
constexpr int kNT = kGN / 16;                 // 16-column MFMA tiles per wave
constexpr int kGRow = kGK + 16;               // bytes per LDS row: 64 + 16 of padding
constexpr int kStages = 3;                    // K steps of global loads in flight

// K rounded up to whole steps: the digit planes are that wide, zeros past K.
__host__ __device__ inline int padded_k(int K) { return (K + kGK - 1) / kGK * kGK; }

// Digit planes, step-major: for each K step of 64 columns, the three digits, each M rows
// rounded up to whole 16-row tiles (Mp); within a tile the 16-byte runs are in MFMA lane
// order -- run g (columns 16g .. 16g+15 of the step) of row r at (16 g + r) * 16 -- so a
// wave's fragment of one digit for one step is one contiguous 1 KB load, lane l taking row
// l % 16, columns 16 (l / 16) .. +15. Rows past M within the last tile are never written
// (only outputs of those rows read them, and those are dropped).
__host__ __device__ inline int digit_rows(int M) { return (M + 15) & ~15; }
__host__ __device__ inline size_t digit_offset(int Mp, int step, int d, int m, int b) {
  return ((size_t)(step * kDigits + d) * Mp + (m & ~15)) * kGK + (b >> 4) * 256 + (m & 15) * 16 + (b & 15);
}

// ------------------------------------------------------------ activation digits --
// The larger magnitude, NaN kept once met.
__device__ __forceinline__ float peak_of(float p, float v) { return (v > p || v != v) ? v : p; }

// One row kernel in front of every contraction (one block per row m, rows of n <= 8192
// values): the row is the sum of `splits` partial rows (+ bias) -- a previous contraction's
// split-K output, summed in the order k_gemm_finish sums it -- or, for ROW_SWIGLU,
// silu(g) * u of such a row of interleaved gate|up pairs (no bias, no residual); optionally
// added into the residual stream `resid` (f32, as the batched path's add); for ROW_RMSNORM normalized
// as the f32 rmsnorm does; and, when `digits` is set, written as the digit planes of the
// next contraction: s = max|y| / 127, X = rint(y * 2^16 / s) in three balanced base-256
// digits (step-major, digit_offset), zeros past n, and the row factor s * 2^-16 (NaN for a
// row holding an infinity or a NaN, whose digits are zero).
//
// Every load is issued before any is used, from a clamped address (a lane past the row re-reads
// its last group and masks it out): a load behind a branch, or inside a loop whose count is
// only known at run time, makes the compiler wait for each in turn. J = float4 groups per
// thread (rows of up to 1024 J values); the splits are read U at a time (four for the split
// contractions' rows; the gate|up contraction is not split) and added in order.
//
// Rows are dealt to blocks so that the 16 rows of a digit tile run on one XCD (workgroups go to
// the 8 XCDs round-robin by linear id): a 128-byte line of a digit plane holds 16 bytes of each
// of 8 rows, and one L2 then merges the line's parts instead of eight L2s each writing one back.
// Needs M to be a multiple of 128; otherwise block b handles row b.
__device__ __forceinline__ int row_of_block(int b, int M) {
  if (M % 128) return b;
  const int xcd = b & 7, r = b >> 3;
  return 16 * (xcd + 8 * (r >> 4)) + (r & 15);
}

template <int OP, int J>
__global__ __launch_bounds__(kBlock) void k_rows(RowArgs a) {
  __shared__ float red[kBlock / kWave];
  constexpr int W = OP == ROW_SWIGLU ? 2 : 1;  // float4 loads per group and split
  constexpr int U = OP == ROW_SWIGLU ? 1 : 4;  // splits read together
  const int m = row_of_block(blockIdx.x, a.M), tid = threadIdx.x;
  const int n4 = a.n / 4;
  const int in_len = W * a.n;
  const size_t plane_in = (size_t)a.M * in_len;
  const float* in_row = a.in + (size_t)m * in_len;
  int idx[J];
  bool ok[J];
#pragma unroll
  for (int j = 0; j < J; j++) {
    ok[j] = tid + j * kBlock < n4;
    idx[j] = min(tid + j * kBlock, n4 - 1);
  }
  // Residual, gain and bias first (read from the row itself where there is none).
  float* resid_row = a.resid ? a.resid + (size_t)m * a.n : nullptr;
  const float* rsrc = a.resid ? resid_row : in_row;
  const float* gsrc = OP == ROW_RMSNORM ? a.gain : in_row;
  const float* bsrc = a.bias ? a.bias : in_row;
  // (the swiglu row has neither: launch_rows refuses one with a residual or bias)
  constexpr bool kAdds = OP != ROW_SWIGLU;
  v4f res[J], gain[J], bias[J][W];
#pragma unroll
  for (int j = 0; j < J; j++) {
    if constexpr (kAdds) res[j] = *reinterpret_cast<const v4f*>(rsrc + 4 * idx[j]);
    if constexpr (OP == ROW_RMSNORM) gain[j] = *reinterpret_cast<const v4f*>(gsrc + 4 * idx[j]);
    if constexpr (kAdds) {
#pragma unroll
      for (int w = 0; w < W; w++) bias[j][w] = *reinterpret_cast<const v4f*>(bsrc + 4 * (W * idx[j] + w));
    }
  }
  v4f sum[J][W];
#pragma unroll
  for (int j = 0; j < J; j++)
#pragma unroll
    for (int w = 0; w < W; w++) sum[j][w] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int sp0 = 0; sp0 < a.splits; sp0 += U) {
    v4f t[U][J][W];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const float* src = in_row + (size_t)min(sp0 + u, a.splits - 1) * plane_in;
#pragma unroll
      for (int j = 0; j < J; j++)
#pragma unroll
        for (int w = 0; w < W; w++) t[u][j][w] = *reinterpret_cast<const v4f*>(src + 4 * (W * idx[j] + w));
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (sp0 + u < a.splits) {  // block-uniform
#pragma unroll
        for (int j = 0; j < J; j++)
#pragma unroll
          for (int w = 0; w < W; w++) sum[j][w] += t[u][j][w];
      }
    }
  }
  v4f v[J];
#pragma unroll
  for (int j = 0; j < J; j++) {
    if (kAdds && a.bias) {
#pragma unroll
      for (int w = 0; w < W; w++) sum[j][w] += bias[j][w];
    }
    if constexpr (OP == ROW_SWIGLU)
      v[j] = v4f{swiglu_f32(sum[j][0][0], sum[j][0][1]), swiglu_f32(sum[j][0][2], sum[j][0][3]),
                 swiglu_f32(sum[j][1][0], sum[j][1][1]), swiglu_f32(sum[j][1][2], sum[j][1][3])};
    else
      v[j] = sum[j][0];
    if (kAdds && a.resid) {
      v[j] = res[j] + v[j];
      if (ok[j]) *reinterpret_cast<v4f*>(resid_row + 4 * idx[j]) = v[j];
    }
    if (!ok[j]) v[j] = v4f{0.f, 0.f, 0.f, 0.f};
  }
  if constexpr (OP == ROW_RMSNORM) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < J; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) ss = fmaf(v[j][e], v[j][e], ss);
    ss = block_sum_f32(ss, red);
    const float scale = __builtin_amdgcn_rsqf(ss / (float)a.n + a.eps);
    __syncthreads();  // red is reused below
#pragma unroll
    for (int j = 0; j < J; j++)
      if (ok[j]) v[j] = rms_apply_f32(v[j], scale, gain[j]);
  }
  if (!a.digits) return;
  float peak = 0.f;
#pragma unroll
  for (int j = 0; j < J; j++)
#pragma unroll
    for (int e = 0; e < 4; e++) peak = peak_of(peak, fabsf(v[j][e]));
  for (int off = kWave / 2; off > 0; off >>= 1) peak = peak_of(peak, __shfl_xor(peak, off));
  if ((tid & (kWave - 1)) == 0) red[tid / kWave] = peak;
  __syncthreads();
  peak = 0.f;
#pragma unroll
  for (int w = 0; w < kBlock / kWave; w++) peak = peak_of(peak, red[w]);
  const bool finite = peak <= 3.402823466e38f;
  const double s = (double)peak / 127.0;
  const double inv = finite && peak > 0.f ? 65536.0 / s : 0.0;
  if (tid == 0) a.row_factor[m] = finite ? s / 65536.0 : (double)NAN;
  const int Mp = digit_rows(a.M);
#pragma unroll
  for (int j = 0; j < J; j++) {
    const int i4 = tid + j * kBlock;
    if (4 * i4 >= a.Kp) break;
    uint32_t w[kDigits] = {0, 0, 0};
    if (i4 < n4 && inv != 0.0) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        int q = (int)rint((double)v[j][e] * inv);  // |q| <= 127 * 2^16
#pragma unroll
        for (int d = 0; d < kDigits; d++) {
          const int dig = (int)(int8_t)(uint8_t)(q & 0xff);  // balanced: [-128, 127]
          w[d] |= (uint32_t)(uint8_t)dig << (8 * e);
          q = (q - dig) >> 8;
        }
      }
    }
#pragma unroll
    for (int d = 0; d < kDigits; d++)
      *reinterpret_cast<uint32_t*>(a.digits + digit_offset(Mp, i4 >> 4, d, m, (4 * i4) & (kGK - 1))) = w[d];
  }
}

template <int OP>
static hipError_t launch_rows_op(hipStream_t s, const RowArgs& a) {
  const int groups = (a.n / 4 + kBlock - 1) / kBlock;  // float4 groups per thread
  if (groups <= 1) hipLaunchKernelGGL((k_rows<OP, 1>), dim3(a.M), dim3(kBlock), 0, s, a);
  else if (groups <= 2) hipLaunchKernelGGL((k_rows<OP, 2>), dim3(a.M), dim3(kBlock), 0, s, a);
  else if (groups <= 4) hipLaunchKernelGGL((k_rows<OP, 4>), dim3(a.M), dim3(kBlock), 0, s, a);
  else if (groups <= 5) hipLaunchKernelGGL((k_rows<OP, 5>), dim3(a.M), dim3(kBlock), 0, s, a);
  else hipLaunchKernelGGL((k_rows<OP, 8>), dim3(a.M), dim3(kBlock), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_rows(hipStream_t s, int op, const RowArgs& a) {
  if (a.n % 4 || a.n > 8192 || a.splits < 1 || (a.digits && a.Kp != padded_k(a.n))) return hipErrorInvalidValue;
  if (op == ROW_SWIGLU && (a.bias || a.resid)) return hipErrorInvalidValue;
  switch (op) {
    case ROW_PLAIN: return launch_rows_op<ROW_PLAIN>(s, a);
    case ROW_RMSNORM: return launch_rows_op<ROW_RMSNORM>(s, a);
    case ROW_SWIGLU: return launch_rows_op<ROW_SWIGLU>(s, a);
    default: return hipErrorInvalidValue;
  }
}

// ------------------------------------------------------------------ weight tile --
// Thirty-two codes of one step for one thread: row n, columns k .. k+31, as int8.
template <int FMT>
struct WRaw {
  v4u q[2];     // int8: 32 codes; int4: q[0] = 32 nibbles
  float zero;   // int4: the group's zero point
  float scale;  // int4: the step's group scale of weight row n0 + tid % 128
};

// Past K (the second half of a last 64-column step) the thread loads columns K - 32 ..
// K - 1 again: the digit planes are zeros there, so those codes add nothing. Every thread
// loads, with nothing done to the registers until their step: a branch around the loads,
// or a select right after them, would make the waits before each step cover the loads
// of the steps prefetched behind it as well.
template <int FMT>
__device__ __forceinline__ void wraw_load(const DMat& w, int n, int k, int K, WRaw<FMT>& r) {
  const int kk = min(k, K - 32);
  const uint8_t* row = w.data + (size_t)n * w.row_bytes;
  if constexpr (FMT == QH_FMT_INT8) {
    r.q[0] = *reinterpret_cast<const v4u*>(row + kk);
    r.q[1] = *reinterpret_cast<const v4u*>(row + kk + 16);
  } else {
    r.q[0] = *reinterpret_cast<const v4u*>(row + kk / 2);
    r.zero = w.zeros[(size_t)n * w.gpr + kk / (w.cpg * 32)];
  }
}

// Bytewise a + b (mod 256 in each byte, no carry between bytes).
__device__ __forceinline__ uint32_t add_bytes(uint32_t a, uint32_t b) {
  return ((a & 0x7f7f7f7fu) + (b & 0x7f7f7f7fu)) ^ ((a ^ b) & 0x80808080u);
}

// The thirty-two codes as int8 bytes, in column order (int4: level - zero; the low
// nibble of a byte is the even column).
template <int FMT>
__device__ __forceinline__ void wraw_bytes(const WRaw<FMT>& r, v4u (&o)[2]) {
  if constexpr (FMT == QH_FMT_INT8) {
    o[0] = r.q[0];
    o[1] = r.q[1];
  } else {
    // the zero point is an integer in [0, 15] (src/core/quantize.js:115)
    const uint32_t nz = (uint32_t)((256 - (int)r.zero) & 0xff) * 0x01010101u;  // -zero in every byte
    uint32_t b[8];
    const uint32_t src[4] = {r.q[0].x, r.q[0].y, r.q[0].z, r.q[0].w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t lo = src[i] & 0x0f0f0f0fu, hi = (src[i] >> 4) & 0x0f0f0f0fu;  // even, odd columns
      // interleave: bytes lo0 hi0 lo1 hi1 | lo2 hi2 lo3 hi3
      b[2 * i] = add_bytes(__builtin_amdgcn_perm(hi, lo, 0x05010400u), nz);
      b[2 * i + 1] = add_bytes(__builtin_amdgcn_perm(hi, lo, 0x07030602u), nz);
    }
    o[0] = v4u{b[0], b[1], b[2], b[3]};
    o[1] = v4u{b[4], b[5], b[6], b[7]};
  }
}

struct GemmArgs {
  DMat w;                    // int8 | int4, rows = N, cols = K
  const int8_t* digits;      // step-major digit planes (digit_offset), Kp columns
  const double* row_factor;  // [M]
  float* out;                // splits == 1: Y [M][N]; else partials [splits][M][N]
  const float* bias;         // [N] or NULL (splits == 1 only)
  int M, N, K, Kp;
  int steps_per_split;       // K steps (of 64) per gridDim.z slice
};

// Steps st + U of a group, each from register set U (a compile-time index, so the sets
// stay in registers), up to step s1.
template <typename F, int... U>
__device__ __forceinline__ void step_group(F& step, int st, int s1, std::integer_sequence<int, U...>) {
  ((st + U < s1 ? (step(std::integral_constant<int, U>{}, st + U), 0) : 0), ...);
}

template <int FMT>
__global__ __launch_bounds__(kGemmThreads) void k_gemm(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][kGN][kGRow];
  __shared__ float Ss[2][kGN];  // int4: the step's group scales of the tile's weight rows
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  const int m0 = blockIdx.y * kGM, n0 = blockIdx.x * kGN;
  const int s0 = blockIdx.z * a.steps_per_split;
  const int s1 = min(s0 + a.steps_per_split, a.Kp / kGK);
  const int fr = lane & 15, fg = lane >> 4;  // fragment row (or column) and 16-byte k group
  const int mw = m0 + 16 * wave;             // this wave's first position
  const bool active = mw < a.M;              // wave-uniform: rows past M are not computed

  // A fragments: this wave's 16-row tile (clamped to the last; results past M are
  // discarded), lane row fr, bytes 16*fg .. +15 of each step, one 1 KB load per digit.
  const int Mp = digit_rows(a.M);
  const int8_t* ar = a.digits + (size_t)min(mw, Mp - 16) * kGK + 16 * lane;
  const size_t dplane = (size_t)Mp * kGK;  // one digit of one step
  // Weight staging: thread t stages row t/2 of the tile, columns 32*(t%2) .. +31.
  const int br = tid >> 1, bk = 32 * (tid & 1);
  const int brow = min(n0 + br, a.N - 1);

  v4i acc[kDigits][kNT];
  double tot[kNT][4];
#pragma unroll
  for (int j = 0; j < kNT; j++) {
#pragma unroll
    for (int d = 0; d < kDigits; d++) acc[d][j] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int r = 0; r < 4; r++) tot[j][r] = 0.0;
  }
  // int4: steps per group (a group is a multiple of 64 columns on this path).
  const int group_steps = FMT == QH_FMT_INT4 ? a.w.cpg / 2 : 1;

  v4i xa[kStages][kDigits];
  WRaw<FMT> wr[kStages];
  // Loads are unconditional, so the register sets rotate in place and no wait covers more
  // than the step being consumed: a step past the split's last re-reads that last one
  // (never used), and waves past M read the clamped row.
  auto issue = [&](int st, v4i (&x)[kDigits], WRaw<FMT>& w) {
    const int k = min(st, s1 - 1) * kGK;
#pragma unroll
    for (int d = 0; d < kDigits; d++) x[d] = *reinterpret_cast<const v4i*>(ar + (size_t)(k / kGK * kDigits + d) * dplane);
    wraw_load<FMT>(a.w, brow, k + bk, a.K, w);
    if constexpr (FMT == QH_FMT_INT4)
      w.scale = a.w.scales[(size_t)min(n0 + (tid & (kGN - 1)), a.N - 1) * a.w.gpr + min(st, s1 - 1) / group_steps];
  };
#pragma unroll
  for (int u = 0; u < kStages; u++) issue(s0 + u, xa[u], wr[u]);
  // One K step from register set U; the loop below runs whole groups of kStages steps (no
  // exit inside a group, so every set is reloaded in place) and then the remainder.
  auto step = [&](auto U, int st) {
    constexpr int u = decltype(U)::value;
    const int buf = (st - s0) & 1;
    {
      v4u wb[2];
      wraw_bytes<FMT>(wr[u], wb);
      *reinterpret_cast<v4u*>(&Bs[buf][br][bk]) = wb[0];
      *reinterpret_cast<v4u*>(&Bs[buf][br][bk + 16]) = wb[1];
      if constexpr (FMT == QH_FMT_INT4)
        if (tid < kGN) Ss[buf][tid] = wr[u].scale;
    }
    // One barrier per step: Bs[buf] is complete, and every wave has finished reading it
    // two steps ago (each wave reads a buffer before it arrives at the next barrier).
    __syncthreads();
    if (active) {
      v4i fb[kNT];
#pragma unroll
      for (int j = 0; j < kNT; j++) fb[j] = *reinterpret_cast<const v4i*>(&Bs[buf][16 * j + fr][16 * fg]);
#pragma unroll
      for (int d = 0; d < kDigits; d++)
#pragma unroll
        for (int j = 0; j < kNT; j++)
          acc[d][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[u][d], fb[j], acc[d][j], 0, 0, 0);
      if constexpr (FMT == QH_FMT_INT4) {
        if ((st + 1) % group_steps == 0) {  // the group's exact sum, scaled into the total
#pragma unroll
          for (int j = 0; j < kNT; j++) {
            const double sg = Ss[buf][16 * j + fr];
#pragma unroll
            for (int r = 0; r < 4; r++)
              tot[j][r] += sg * ((double)acc[2][j][r] * 65536.0 + (double)acc[1][j][r] * 256.0 +
                                 (double)acc[0][j][r]);
#pragma unroll
            for (int d = 0; d < kDigits; d++) acc[d][j] = v4i{0, 0, 0, 0};
          }
        }
      }
    }
    // The set's next loads, issued once its digits are in the MFMAs: they land in the same
    // registers kStages steps ahead of their use.
    issue(st + kStages, xa[u], wr[u]);
  };
  int st = s0;
  for (; st + kStages <= s1; st += kStages) step_group(step, st, s1, std::make_integer_sequence<int, kStages>{});
  step_group(step, st, s1, std::make_integer_sequence<int, kStages - 1>{});
  if (!active) return;

  // D fragment: lane holds rows 4*fg .. +3 of column fr of each tile.
  float* dst = a.out + (size_t)blockIdx.z * a.M * a.N;
  double rf[4];
#pragma unroll
  for (int r = 0; r < 4; r++) rf[r] = a.row_factor[min(mw + 4 * fg + r, a.M - 1)];
#pragma unroll
  for (int j = 0; j < kNT; j++) {
    const int n = n0 + 16 * j + fr;
    if (n >= a.N) continue;
    const double cs = FMT == QH_FMT_INT8 ? (double)a.w.scales[n] : 1.0;
    const double b = a.bias ? (double)a.bias[n] : 0.0;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = mw + 4 * fg + r;
      double v;
      if constexpr (FMT == QH_FMT_INT8)
        v = (double)acc[2][j][r] * 65536.0 + (double)acc[1][j][r] * 256.0 + (double)acc[0][j][r];
      else
        v = tot[j][r];
      if (m < a.M) dst[(size_t)m * a.N + n] = (float)(v * rf[r] * cs + b);
    }
  }
}

// The int8 contraction with whole weight lines: a stage of 128 columns (two MFMA K steps)
// per barrier, so a weight row's 128 bytes of the stage are one cache line, read by eight
// consecutive lanes -- a wave's load instruction covers 8 whole lines instead of 32 halves
// (the per-CU rate of line requests, not bytes, bounds this kernel). Same block tile,
// fragments and exact integer sums as k_gemm<int8>, so a split's outputs are the same bits.
constexpr int kSK = 2 * kGK;        // columns staged per barrier
constexpr int kSRow = kSK + 16;     // bytes per LDS row: 128 + 16 of padding (rows 36 banks apart)
constexpr int kSStages = 2;         // stages of global loads in flight
constexpr int kSLoads = kGN * kSK / 16 / kGemmThreads;  // 16-byte weight loads per thread per stage

__global__ __launch_bounds__(kGemmThreads) void k_gemm8w(GemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t Bs[2][kGN][kSRow];
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
  // Tile of this block. Workgroups are dealt to the 8 XCDs (8 separate L2s) round-robin by
  // linear id. With K split (gridDim.z > 1) and (position tiles x splits) a multiple of 8,
  // the ids are remapped so that the X weight tiles of one (position tile, split) run on one
  // XCD and an XCD's groups share a split: each L2 then holds one K slice of the weights and
  // a few position tiles' digits (~2 MB for down at M = 512) instead of all of both.
  int bx = blockIdx.x, by = blockIdx.y, bz = blockIdx.z;
  {
    const int X = gridDim.x, Y = gridDim.y, Z = gridDim.z;
    if (Z > 1 && (Y * Z) % 8 == 0) {
      const int b = blockIdx.x + X * (blockIdx.y + Y * blockIdx.z);
      const int xcd = b & 7, r = b >> 3;
      const int gi = xcd + 8 * (r / X);  // (position tile, split) group, = xcd mod 8
      bx = r % X;
      bz = gi % Z;
      by = gi / Z;
    }
  }
  const int m0 = by * kGM, n0 = bx * kGN;
  const int s0 = bz * a.steps_per_split;  // even: splits fall on stage boundaries
  const int s1 = min(s0 + a.steps_per_split, a.Kp / kGK);
  const int g0 = s0 / 2, g1 = (s1 + 1) / 2;       // stages; the last may hold one step
  const int fr = lane & 15, fg = lane >> 4;
  const int mw = m0 + 16 * wave;
  const bool active = mw < a.M;

  const int Mp = digit_rows(a.M);
  const int8_t* ar = a.digits + (size_t)min(mw, Mp - 16) * kGK + 16 * lane;
  const size_t dplane = (size_t)Mp * kGK;
  // Weight staging: load i of thread t is row 32 i + t / 8 of the tile, bytes 16 (t % 8) ..
  // +15 of the stage (rows past N re-read the last row; their outputs are dropped).
  const int wrow = tid >> 3, wcol = 16 * (tid & 7);
  const uint8_t* wsrc[kSLoads];
#pragma unroll
  for (int i = 0; i < kSLoads; i++)
    wsrc[i] = a.w.data + (size_t)min(n0 + 32 * i + wrow, a.N - 1) * a.w.row_bytes;

  // The epilogue's factors, loaded before the K loop so that no memory round trip is left
  // behind it: the four rows' factors, and each tile column's row scale and bias.
  double rf[4];
#pragma unroll
  for (int r = 0; r < 4; r++) rf[r] = a.row_factor[min(mw + 4 * fg + r, a.M - 1)];
  // Unconditional loads (a branch around one makes the compiler wait for each in turn):
  // without a bias the scales are read in its place and multiplied by zero.
  const float* bsrc = a.bias ? a.bias : a.w.scales;
  const float bmul = a.bias ? 1.f : 0.f;
  float cs[kNT], bias[kNT];
#pragma unroll
  for (int j = 0; j < kNT; j++) {
    const int n = min(n0 + 16 * j + fr, a.N - 1);
    cs[j] = a.w.scales[n];
    bias[j] = bsrc[n];
  }

  v4i acc[kDigits][kNT];
#pragma unroll
  for (int j = 0; j < kNT; j++)
#pragma unroll
    for (int d = 0; d < kDigits; d++) acc[d][j] = v4i{0, 0, 0, 0};

  v4i xa[kSStages][2][kDigits];
  v4u wv[kSStages][kSLoads];
  // Unconditional, clamped loads: a stage past the split's last re-reads that last one (never
  // used); a step past s1 re-reads step s1 - 1 (its MFMAs are skipped); weight columns past
  // K re-read columns K - 16 .. K - 1, which meet zero digits.
  auto issue = [&](int g, v4i (&x)[2][kDigits], v4u (&w)[kSLoads]) {
    const int gg = min(g, g1 - 1);
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int st = min(2 * gg + h, s1 - 1);
#pragma unroll
      for (int d = 0; d < kDigits; d++) x[h][d] = *reinterpret_cast<const v4i*>(ar + (size_t)(st * kDigits + d) * dplane);
    }
    const int col = min(gg * kSK + wcol, a.K - 16);
#pragma unroll
    for (int i = 0; i < kSLoads; i++) w[i] = *reinterpret_cast<const v4u*>(wsrc[i] + col);
  };
#pragma unroll
  for (int u = 0; u < kSStages; u++) issue(g0 + u, xa[u], wv[u]);
  auto stage = [&](auto U, int g) {
    constexpr int u = decltype(U)::value;
    const int buf = (g - g0) & 1;
#pragma unroll
    for (int i = 0; i < kSLoads; i++) *reinterpret_cast<v4u*>(&Bs[buf][32 * i + wrow][wcol]) = wv[u][i];
    // One barrier per stage: Bs[buf] is complete, and every wave finished reading it two
    // stages ago (each wave reads a buffer before it arrives at the next barrier).
    __syncthreads();
    if (active) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        if (2 * g + h < s1) {  // block-uniform
          v4i fb[kNT];
#pragma unroll
          for (int j = 0; j < kNT; j++) fb[j] = *reinterpret_cast<const v4i*>(&Bs[buf][16 * j + fr][kGK * h + 16 * fg]);
#pragma unroll
          for (int d = 0; d < kDigits; d++)
#pragma unroll
            for (int j = 0; j < kNT; j++)
              acc[d][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[u][h][d], fb[j], acc[d][j], 0, 0, 0);
        }
      }
    }
    issue(g + kSStages, xa[u], wv[u]);
  };
  int g = g0;
  for (; g + kSStages <= g1; g += kSStages) step_group(stage, g, g1, std::make_integer_sequence<int, kSStages>{});
  step_group(stage, g, g1, std::make_integer_sequence<int, kSStages - 1>{});
  if (!active) return;

  float* dst = a.out + (size_t)bz * a.M * a.N;
#pragma unroll
  for (int j = 0; j < kNT; j++) {
    const int n = n0 + 16 * j + fr;
    if (n >= a.N) continue;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = mw + 4 * fg + r;
      const double v = (double)acc[2][j][r] * 65536.0 + (double)acc[1][j][r] * 256.0 + (double)acc[0][j][r];
      if (m < a.M) dst[(size_t)m * a.N + n] = (float)(v * rf[r] * (double)cs[j] + (double)(bias[j] * bmul));
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

// int8, or int4 in groups of a multiple of 64 columns (a step never spans two scales); K up
// to 2^17 keeps every int32 sum exact.
bool matmul_prefill_supported(const DMat& w) {
  return (w.format == QH_FMT_INT8 || (w.format == QH_FMT_INT4 && w.cpg % 2 == 0)) && w.cols <= (1 << 17);
}

// K steps per split: as many splits as keep (M/64 x N/128 x splits) blocks within one per
// CU, int4 splits on group boundaries. A CU holding two blocks runs each at well under half
// speed (its L2 load rate is the bound), and every split adds an M x N partial that the
// consumer row kernel reads back: 512-token prefill 3.6 ms at two blocks per CU, 3.4 ms at one.
// int8 splits fall on whole 128-column stages (k_gemm8w).
static int gemm_steps_per_split(const DMat& w, int M) {
  const int steps = padded_k(w.cols) / kGK;
  const int tiles = ((M + kGM - 1) / kGM) * ((w.rows + kGN - 1) / kGN);
  const int unit = w.format == QH_FMT_INT4 ? w.cpg / 2 : kSK / kGK;
  int splits = 256 / tiles;
  splits = std::max(1, std::min(splits, steps / unit));
  int per = (steps + splits - 1) / splits;
  per = (per + unit - 1) / unit * unit;
  return per;
}

static int gemm_splits(const DMat& w, int M) {
  const int steps = padded_k(w.cols) / kGK;
  const int per = gemm_steps_per_split(w, M);
  return (steps + per - 1) / per;
}

static size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

size_t digits_bytes(int M, int K) { return round256((size_t)kDigits * digit_rows(M) * padded_k(K)); }
int digits_width(int K) { return padded_k(K); }

// Split partials of every launch of 1..M rows. Not the M-row figure alone: below a 64-row
// tile boundary there are fewer tiles and so more splits, and the partials of a smaller M
// can outgrow M's own. The split count depends on m only through its 64-row tiles, so within
// each band of 64 rows the largest m holds the most: one evaluation per band (this runs on
// the host before every batched forward).
size_t gemm_partials_bytes(const DMat& w, int M) {
  size_t most = 0;
  for (int hi = std::min(M, kGM); hi >= 1; hi = hi == M ? 0 : std::min(M, hi + kGM)) {
    const int splits = gemm_splits(w, hi);
    if (splits > 1) most = std::max(most, (size_t)splits * hi * w.rows * sizeof(float));
  }
  return most;
}

hipError_t launch_gemm_digits(hipStream_t s, const DMat& w, const int8_t* digits, const double* row_factor, int M,
                              const float* bias, float* y, float* part, size_t part_bytes, int* splits_out) {
  if (M < 1 || !matmul_prefill_supported(w)) return hipErrorInvalidValue;
  const int Kp = padded_k(w.cols);
  const int splits = gemm_splits(w, M);
  if (splits > 1 && (size_t)splits * M * w.rows * sizeof(float) > part_bytes) return hipErrorInvalidValue;
  GemmArgs a{};
  a.w = w;
  a.digits = digits;
  a.row_factor = row_factor;
  a.out = splits > 1 ? part : y;
  a.bias = splits > 1 ? nullptr : bias;
  a.M = M;
  a.N = w.rows;
  a.K = w.cols;
  a.Kp = Kp;
  a.steps_per_split = gemm_steps_per_split(w, M);
  const dim3 grid((w.rows + kGN - 1) / kGN, (M + kGM - 1) / kGM, splits);
  if (w.format == QH_FMT_INT8) hipLaunchKernelGGL(k_gemm8w, grid, dim3(kGemmThreads), 0, s, a);
  else hipLaunchKernelGGL(k_gemm<QH_FMT_INT4>, grid, dim3(kGemmThreads), 0, s, a);
  *splits_out = splits;
  return hipGetLastError();
}

// The whole standalone contraction: the row kernel's digits of x, the GEMM, the split sum.
size_t matmul_prefill_scratch_bytes(const DMat& w, int M) {
  return digits_bytes(M, w.cols) + round256((size_t)M * sizeof(double)) + gemm_partials_bytes(w, M);
}

hipError_t launch_matmul_prefill(hipStream_t s, const DMat& w, const float* x, const float* bias,
                                 float* y, int M, void* scratch, size_t scratch_bytes) {
  if (M < 1 || !matmul_prefill_supported(w) || w.cols > 8192 || matmul_prefill_scratch_bytes(w, M) > scratch_bytes)
    return hipErrorInvalidValue;
  char* p = static_cast<char*>(scratch);
  const size_t db = digits_bytes(M, w.cols), rb = round256((size_t)M * sizeof(double));
  RowArgs r{};
  r.in = x;
  r.splits = 1;
  r.M = M;
  r.n = w.cols;
  r.Kp = padded_k(w.cols);
  r.digits = reinterpret_cast<int8_t*>(p);
  r.row_factor = reinterpret_cast<double*>(p + db);
  hipError_t e = launch_rows(s, ROW_PLAIN, r);
  if (e != hipSuccess) return e;
  float* part = reinterpret_cast<float*>(p + db + rb);
  int splits = 1;
  e = launch_gemm_digits(s, w, r.digits, r.row_factor, M, bias, y, part, scratch_bytes - db - rb, &splits);
  if (e != hipSuccess || splits == 1) return e;
  const size_t total = (size_t)M * w.rows;
  hipLaunchKernelGGL(k_gemm_finish, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, part, splits,
                     bias, y, M, w.rows);
  return hipGetLastError();
}

}  // namespace qh
