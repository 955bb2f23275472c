// The batched prefill forward: GpuModel.#forward (src/gpu/model.js:240-402) over
// `seq` positions at once, each weight read once per 8-position tile
// (QH_MATMUL_BATCHED, the reference's batchedMatvec, src/gpu/kernels.js:232-290,
// selected by src/gpu/model.js:297-306) or once per prefill on the matrix cores
// (QH_MATMUL_MFMA, prefill.hip).
//
// Per layer, over all positions: rmsnorm -> q|k|v matmul + bias -> rope (f64) with
// the f16 K/V append -> attention (QH_MATMUL_BATCHED: the decode step's algorithm
// for the model's numerics, one query per position; QH_MATMUL_MFMA: flash attention
// on the matrix cores) -> o matmul, residual add -> rmsnorm -> gate|up
// matmul -> swiglu -> down matmul, residual add. The last position's row then goes
// through the decode step's own output head and pick.
//
// QH_MATMUL_BATCHED sums every output exactly as the decode step does (same
// matvec summation order, same rope, attention and merge arithmetic, same f32
// residual adds), so a prefill and the same positions decoded one by one give
// the same bits -- the reference's prefill == incremental decode property
// (README.md:256-272, web/model.html:169-198). QH_MATMUL_MFMA is held to a stated
// tolerance instead.
#include "attention.h"
#include "device_common.h"
#include "model_dev.h"

namespace qh {

// Rows of q|k|v at positions past+t -- each the sum of `splits` partial rows (planes of
// seq rows apart, in k_gemm_finish's order) plus `bias` when given, else the row itself
// (bias included) -- with q and k heads rotated as the decode step's QKV epilogue does
// (rope_pair over f64 angles), q to `q`, k and v to the f16 caches.
// grid (ceil(items / 256), seq).
// Columns col[0..N) of a row summed over `splits` partial rows (`plane` floats apart) in split
// order, + bias. Every load is issued before any is used -- the splits four at a time from
// clamped indices, the bias (or the row itself where there is none) up front -- since a load
// inside a loop of run-time count, or behind a branch, makes the compiler wait for each in turn.
template <int N>
__device__ __forceinline__ void split_sum_cols(const float* row, size_t plane, int splits, const float* bias,
                                               const int (&col)[N], float (&v)[N]) {
  const float* bsrc = bias ? bias : row;
  float b[N];
#pragma unroll
  for (int k = 0; k < N; k++) {
    b[k] = bsrc[col[k]];
    v[k] = 0.f;
  }
  for (int sp0 = 0; sp0 < splits; sp0 += 4) {
    float x[4][N];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const float* src = row + (size_t)min(sp0 + u, splits - 1) * plane;
#pragma unroll
      for (int k = 0; k < N; k++) x[u][k] = src[col[k]];
    }
#pragma unroll
    for (int u = 0; u < 4; u++)
      if (sp0 + u < splits) {
#pragma unroll
        for (int k = 0; k < N; k++) v[k] += x[u][k];
      }
  }
  if (bias) {
#pragma unroll
    for (int k = 0; k < N; k++) v[k] += b[k];
  }
}

__global__ void k_rope_kv(const float* __restrict__ qkv, int splits, const float* __restrict__ bias,
                          float* __restrict__ q, uint16_t* __restrict__ kc, uint16_t* __restrict__ vt,
                          const double* __restrict__ rope_cos, const double* __restrict__ rope_sin, int past,
                          int heads, int kv_heads, int capacity, int vstride) {
  const int t = blockIdx.y, pos = past + t;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int hidden = heads * kHeadDim, kvd = kv_heads * kHeadDim;
  const int width = hidden + 2 * kvd;
  const size_t plane = (size_t)gridDim.y * width;
  const float* row = qkv + (size_t)t * width;
  const int rope_pairs = (heads + kv_heads) * 32;
  if (i < rope_pairs) {
    const int head = i / 32, j = i % 32;
    const int base = head < heads ? head * kHeadDim : hidden + (head - heads) * kHeadDim;
    const double cs = rope_cos[(size_t)pos * 32 + j], sn = rope_sin[(size_t)pos * 32 + j];
    const int col[2] = {base + j, base + j + 32};
    float x[2], lo, hi;
    split_sum_cols<2>(row, plane, splits, bias, col, x);
    rope_pair(x[0], x[1], cs, sn, &lo, &hi);
    if (head < heads) {
      q[(size_t)t * hidden + head * kHeadDim + j] = lo;
      q[(size_t)t * hidden + head * kHeadDim + j + 32] = hi;
    } else {
      uint16_t* k = kc + ((size_t)(head - heads) * capacity + pos) * kHeadDim;
      k[j] = __builtin_bit_cast(uint16_t, (_Float16)lo);
      k[j + 32] = __builtin_bit_cast(uint16_t, (_Float16)hi);
    }
  } else if (i < rope_pairs + kvd) {
    const int e = i - rope_pairs;  // kv head e/64, dimension e%64
    const int col[1] = {hidden + kvd + e};
    float x[1];
    split_sum_cols<1>(row, plane, splits, bias, col, x);
    vt[(size_t)e * vstride + pos] = __builtin_bit_cast(uint16_t, (_Float16)x[0]);
  }
}

// The decode step's slot merge for every query: out [seq][heads*64]. grid (seq).
__global__ __launch_bounds__(kBlock) void k_attn_merge_rows(const float* __restrict__ part, int heads,
                                                            float* __restrict__ out) {
  __shared__ float wl[kBlock];
  const int t = blockIdx.x;
  CombineIn in;
  in.load(part + (size_t)t * heads * kDecodeSlots * kPartStride, heads);
  const v4f acc = attn_combine_quad(in, wl);
  const int i = threadIdx.x;
  if (i < heads * kCombineLanes) {
    float* o = out + (size_t)t * heads * kHeadDim + (i / kCombineLanes) * kHeadDim + 4 * (i % kCombineLanes);
    o[0] = acc.x;
    o[1] = acc.y;
    o[2] = acc.z;
    o[3] = acc.w;
  }
}

// h[t][j] = silu(g) * u over interleaved gate|up rows (g = gu[t][2j], u = gu[t][2j+1]), as
// the decode step's SWIGLU epilogue evaluates it: in f64 (src/core/ops.js:81-91), or in
// f32 for fast numerics (F32).
template <bool F32>
__global__ void k_swiglu_pairs(const float* __restrict__ gu, float* __restrict__ h, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  if constexpr (F32) {
    h[i] = swiglu_f32(gu[2 * i], gu[2 * i + 1]);
  } else {
    const double g = gu[2 * i], u = gu[2 * i + 1];
    h[i] = (float)(g / (1.0 + exp(-g)) * u);
  }
}

// rows [seq][hidden] = bf16 embedding rows of tokens[past .. past+seq-1], widened exactly.
__global__ void k_embed_rows(const uint16_t* __restrict__ embed, const int* __restrict__ tokens, int past,
                             int hidden, int vocab, float* __restrict__ rows) {
  const int t = blockIdx.x;
  int tok = tokens[past + t];
  tok = (tok < 0 || tok >= vocab) ? 0 : tok;  // ids are validated on the host
  const uint16_t* src = embed + (size_t)tok * hidden;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x)
    rows[(size_t)t * hidden + i] = __builtin_bit_cast(float, (uint32_t)src[i] << 16);
}

int prefill_chunk(const ModelDev& m, const CacheDev& c) {
  int p = c.capacity < kPrefillChunk ? c.capacity : kPrefillChunk;
  if (m.numerics == QH_NUMERICS_EXACT && c.capacity > kPLds) {
    // exact attention past kPLds keeps every query's scores: bound them to 64M floats
    const size_t per = (size_t)m.heads * (c.score_stride + attn_spans(c.capacity));
    const size_t fit = ((size_t)64 << 20) / per;
    p = (int)std::max<size_t>(1, std::min<size_t>(p, fit));
  }
  return p;
}

// Every layer matrix contracts on the matrix cores (the fused layer loop below).
static bool all_mfma(const ModelDev& m) {
  for (int L = 0; L < m.layers; L++) {
    const LayerDev& l = m.layers_host[L];
    for (const DMat* w : {&l.qkv, &l.o, &l.gu, &l.down})
      if (!matmul_prefill_supported(*w)) return false;
  }
  return m.hidden <= 8192 && m.intermediate <= 8192;
}

// The fused layer loop's part of the scratch: digit planes of the widest row, row factors,
// then the largest split partials of any matrix at any length up to P.
static size_t mfma_digit_region(const ModelDev& m, size_t P) {
  return digits_bytes((int)P, std::max(m.hidden, m.intermediate)) + ((P * sizeof(double) + 255) & ~(size_t)255);
}

PrefillBytes prefill_bytes(const ModelDev& m, const CacheDev& c, int matmul) {
  const size_t P = prefill_chunk(m, c);
  const size_t d = m.hidden, kv = (size_t)m.kv_heads * m.head_dim, f = m.intermediate;
  PrefillBytes b{};
  b.floats = P * (5 * d + (d + 2 * kv) + 3 * f);
  if (m.numerics == QH_NUMERICS_FAST) b.floats += P * m.heads * kDecodeSlots * kPartStride;
  else if (c.capacity > kPLds) b.floats += P * m.heads * (c.score_stride + attn_spans(c.capacity));
  b.counters = m.numerics == QH_NUMERICS_EXACT ? P * m.heads : 0;
  size_t scratch = 0;
  for (int L = 0; L < m.layers; L++) {
    const LayerDev& l = m.layers_host[L];
    for (const DMat* w : {&l.qkv, &l.o, &l.gu, &l.down}) {
      if (m.numerics == QH_NUMERICS_EXACT) scratch = std::max(scratch, matvec_x64_bytes(*w, (int)P));
      if (matmul == QH_MATMUL_MFMA && matmul_prefill_supported(*w))
        scratch = std::max(scratch, matmul_prefill_scratch_bytes(*w, (int)P));
    }
  }
  if (matmul == QH_MATMUL_MFMA && all_mfma(m)) {
    size_t parts = 0;
    for (int L = 0; L < m.layers; L++) {
      const LayerDev& l = m.layers_host[L];
      for (const DMat* w : {&l.qkv, &l.o, &l.gu, &l.down}) parts = std::max(parts, gemm_partials_bytes(*w, (int)P));
    }
    scratch = std::max(scratch, mfma_digit_region(m, P) + parts);
  }
  b.scratch = scratch;
  return b;
}

// The matrix-core layers. Each contraction reads the digit planes its producer wrote
// (launch_rows), and its split partials are summed by its consumer -- rope and the KV
// write for q|k|v, the residual add + next rmsnorm for o and down, swiglu for gate|up --
// so a layer is ten launches: 4 contractions, rope, attention, 4 row kernels.
static hipError_t prefill_layers_mfma(hipStream_t s, const ModelDev& m, const CacheDev& c, const PrefillDev& p,
                                      int past, int seq) {
  const int d = m.hidden, f = m.intermediate;
  const size_t P = p.positions;
  char* base = static_cast<char*>(p.scratch);
  int8_t* digits = reinterpret_cast<int8_t*>(base);
  double* rowf = reinterpret_cast<double*>(base + digits_bytes((int)P, std::max(d, f)));
  float* part = reinterpret_cast<float*>(base + mfma_digit_region(m, P));
  const size_t part_bytes = p.scratch_bytes - mfma_digit_region(m, P);
  struct Out {
    const float* p;
    int splits;
    const float* bias;
  };
  auto gemm = [&](const DMat& w, const float* bias, float* y, Out* o) {
    int splits = 1;
    const hipError_t e = launch_gemm_digits(s, w, digits, rowf, seq, bias, y, part, part_bytes, &splits);
    *o = Out{splits > 1 ? part : y, splits, splits > 1 ? bias : nullptr};
    return e;
  };
  auto rows = [&](int op, const Out& in, float* resid, const float* gain, int n, bool want_digits) {
    RowArgs r{};
    r.in = in.p;
    r.splits = in.splits;
    r.bias = in.bias;
    r.resid = resid;
    r.gain = gain;
    r.eps = (float)m.eps;
    r.M = seq;
    r.n = n;
    r.Kp = digits_width(n);
    r.digits = want_digits ? digits : nullptr;
    r.row_factor = rowf;
    return launch_rows(s, op, r);
  };
  hipError_t e;
  if ((e = rows(ROW_RMSNORM, Out{p.X, 1, nullptr}, nullptr, m.layers_host[0].in_norm, d, true)) != hipSuccess)
    return e;
  for (int L = 0; L < m.layers; L++) {
    const LayerDev& l = m.layers_host[L];
    uint16_t* kc = c.kv + (size_t)L * c.layer_elems;
    uint16_t* vt = kc + c.key_elems;
    Out o;
    if ((e = gemm(l.qkv, l.qkv_bias, p.QKV, &o)) != hipSuccess) return e;
    const int items = (m.heads + m.kv_heads) * 32 + m.kv_heads * m.head_dim;
    hipLaunchKernelGGL(k_rope_kv, dim3((items + 255) / 256, seq), dim3(256), 0, s, o.p, o.splits, o.bias, p.Q, kc,
                       vt, m.rope_cos, m.rope_sin, past, m.heads, m.kv_heads, c.capacity, c.vstride);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    FlashArgs a{};
    a.q = p.Q;
    a.kc = kc;
    a.vt = vt;
    a.out = p.ATT;
    a.past = past;
    a.seq = seq;
    a.capacity = c.capacity;
    a.vstride = c.vstride;
    a.heads = m.heads;
    a.kv_heads = m.kv_heads;
    if ((e = launch_flash_prefill(s, a)) != hipSuccess) return e;
    if ((e = rows(ROW_PLAIN, Out{p.ATT, 1, nullptr}, nullptr, nullptr, d, true)) != hipSuccess) return e;
    if ((e = gemm(l.o, nullptr, p.Y, &o)) != hipSuccess) return e;
    if ((e = rows(ROW_RMSNORM, o, p.X, l.post_norm, d, true)) != hipSuccess) return e;
    if ((e = gemm(l.gu, nullptr, p.GU, &o)) != hipSuccess) return e;
    if ((e = rows(ROW_SWIGLU, o, nullptr, nullptr, f, true)) != hipSuccess) return e;
    if ((e = gemm(l.down, nullptr, p.Y, &o)) != hipSuccess) return e;
    if (L + 1 < m.layers) e = rows(ROW_RMSNORM, o, p.X, m.layers_host[L + 1].in_norm, d, true);
    else e = rows(ROW_PLAIN, o, p.X, nullptr, d, false);  // the last residual add; the head follows
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// The layer's matmul: MFMA (int8/int4 weights), or the batched matvec tiles summing as
// the decode step does for the model's numerics.
static hipError_t matmul(hipStream_t s, const ModelDev& m, int mode, const DMat& w, const float* x,
                         const float* bias, float* y, int seq, const PrefillDev& p) {
  if (mode == QH_MATMUL_MFMA && matmul_prefill_supported(w))
    return launch_matmul_prefill(s, w, x, bias, y, seq, p.scratch, p.scratch_bytes);
  if (m.numerics == QH_NUMERICS_FAST) return launch_matvec_f32(s, w, x, bias, y, seq);
  return launch_matvec(s, w, x, bias, y, seq, static_cast<double*>(p.scratch));
}

hipError_t enqueue_prefill_layers(hipStream_t s, const ModelDev& m, const CacheDev& c, const PrefillDev& p,
                                  int mode, int past, int seq) {
  if (mode == QH_MATMUL_MFMA && all_mfma(m)) return prefill_layers_mfma(s, m, c, p, past, seq);
  hipError_t e;
  const int d = m.hidden, kvd = m.kv_heads * m.head_dim, f = m.intermediate;
  const size_t n = (size_t)seq * d;
  for (int L = 0; L < m.layers; L++) {
    const LayerDev& l = m.layers_host[L];
    uint16_t* kc = c.kv + (size_t)L * c.layer_elems;
    uint16_t* vt = kc + c.key_elems;
    if ((e = launch_rmsnorm(s, p.X, l.in_norm, p.XN, seq, d, m.eps, m.numerics == QH_NUMERICS_FAST)) != hipSuccess) return e;
    if ((e = matmul(s, m, mode, l.qkv, p.XN, l.qkv_bias, p.QKV, seq, p)) != hipSuccess) return e;
    const int items = (m.heads + m.kv_heads) * 32 + kvd;
    hipLaunchKernelGGL(k_rope_kv, dim3((items + 255) / 256, seq), dim3(256), 0, s, p.QKV, 1, nullptr, p.Q, kc, vt,
                       m.rope_cos, m.rope_sin, past, m.heads, m.kv_heads, c.capacity, c.vstride);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (mode == QH_MATMUL_MFMA) {
      // the matrix-core prefill: flash attention on MFMA (held to the MFMA tolerance)
      FlashArgs a{};
      a.q = p.Q;
      a.kc = kc;
      a.vt = vt;
      a.out = p.ATT;
      a.past = past;
      a.seq = seq;
      a.capacity = c.capacity;
      a.vstride = c.vstride;
      a.heads = m.heads;
      a.kv_heads = m.kv_heads;
      if ((e = launch_flash_prefill(s, a)) != hipSuccess) return e;
    } else if (m.numerics == QH_NUMERICS_FAST) {
      SlotArgs a{};
      a.q = p.Q;
      a.kc = kc;
      a.vt = vt;
      a.part = p.part;
      a.past = past;
      a.capacity = c.capacity;
      a.vstride = c.vstride;
      a.heads = m.heads;
      a.kv_heads = m.kv_heads;
      if (!decode_attn_long(c.capacity)) {
        if ((e = launch_attn_decode(s, a, seq, 1)) != hipSuccess) return e;
        hipLaunchKernelGGL(k_attn_merge_rows, dim3(seq), dim3(kBlock), 0, s, p.part, m.heads, p.ATT);
      } else {
        // a long cache's kLongSlots partials per query, a share of the rows at a time so that
        // they fit the workspace sized for kDecodeSlots (each query's result is its own)
        const int share = std::max(1, (int)p.positions * kDecodeSlots / kLongSlots);
        for (int t0 = 0; t0 < seq; t0 += share) {
          SlotArgs b = a;
          b.q = p.Q + (size_t)t0 * m.heads * kHeadDim;
          b.past = past + t0;
          if ((e = launch_attn_decode(s, b, std::min(share, seq - t0), 1, p.ATT + (size_t)t0 * m.heads * kHeadDim)) !=
              hipSuccess)
            return e;
        }
      }
    } else {
      ExactArgs a{};
      a.q = p.Q;
      a.kc = kc;
      a.vt = vt;
      a.scores = p.scores;
      a.score_stride = c.score_stride;
      a.max_stride = attn_spans(c.capacity);
      a.maxes = p.scores + (size_t)seq * m.heads * c.score_stride;
      a.counters = p.counters;
      a.out = p.ATT;
      a.past = past;
      a.capacity = c.capacity;
      a.vstride = c.vstride;
      a.heads = m.heads;
      a.kv_heads = m.kv_heads;
      // the kernel the decode step picks for this cache (the same arithmetic per query)
      if (c.capacity <= kPLds) {
        hipLaunchKernelGGL(k_attn_block, dim3(m.heads, seq), dim3(kAttnThreads), 0, s, a);
      } else {
        hipLaunchKernelGGL(k_attn_exact, dim3(attn_spans(c.capacity), m.heads, seq), dim3(kBlock), 0, s, a);
      }
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = matmul(s, m, mode, l.o, p.ATT, nullptr, p.Y, seq, p)) != hipSuccess) return e;
    if ((e = launch_add(s, p.X, p.Y, (int)n)) != hipSuccess) return e;
    if ((e = launch_rmsnorm(s, p.X, l.post_norm, p.XN, seq, d, m.eps, m.numerics == QH_NUMERICS_FAST)) != hipSuccess) return e;
    if ((e = matmul(s, m, mode, l.gu, p.XN, nullptr, p.GU, seq, p)) != hipSuccess) return e;
    const size_t nh = (size_t)seq * f;
    if (m.numerics == QH_NUMERICS_FAST)
      hipLaunchKernelGGL(k_swiglu_pairs<true>, dim3((unsigned)((nh + 255) / 256)), dim3(256), 0, s, p.GU, p.H, nh);
    else
      hipLaunchKernelGGL(k_swiglu_pairs<false>, dim3((unsigned)((nh + 255) / 256)), dim3(256), 0, s, p.GU, p.H, nh);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = matmul(s, m, mode, l.down, p.H, nullptr, p.Y, seq, p)) != hipSuccess) return e;
    if ((e = launch_add(s, p.X, p.Y, (int)n)) != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t enqueue_embed_rows(hipStream_t s, const ModelDev& m, const CacheDev& c, const PrefillDev& p, int past,
                              int seq) {
  hipLaunchKernelGGL(k_embed_rows, dim3(seq), dim3(256), 0, s, m.embed, c.tokens, past, m.hidden, m.vocab, p.X);
  return hipGetLastError();
}

}  // namespace qh
