// The fused decode step: the whole of GpuModel.#forward for one position
// (src/gpu/model.js:240-402) as 5 launches per layer plus the gather and the
// output head, instead of the reference's ~15 dispatches and 2 copies per
// layer. Every launch reads its position from device memory, so the same
// launches can be captured once in a hipGraph and replayed every token.
//
// Per layer:
//   1. rmsnorm(x) -> fused q|k|v matvec (+bias)               k_fused<RMSNORM, BIAS>
//   2. rope(q,k) -> f16 KV append -> split-K GQA attention     k_attention<rope, append>
//   3. o-proj matvec, residual add into x                      k_fused<COPY, RESIDUAL>
//   4. rmsnorm(x) -> interleaved gate|up matvec -> swiglu      k_fused<RMSNORM, SWIGLU>
//   5. down matvec, residual add into x                        k_fused<COPY, RESIDUAL>
// then rmsnorm -> lm_head -> logits and argmax; the last block to finish
// writes the token (the reference reads back 151,936 logits and scans them on
// the host, src/gpu/model.js:372-382, web/bench.html:129-131) and advances
// the position.
#include "attention.h"
#include "device_common.h"
#include "model_dev.h"

namespace qh {

enum { PRO_RMSNORM = 0, PRO_COPY = 1 };
enum { EPI_BIAS = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2, EPI_LOGITS = 3 };

struct FusedArgs {
  DMat w;
  const float* in;      // rmsnorm input, or the vector to stage as-is
  const float* gain;    // rmsnorm gain
  double eps;
  const float* bias;    // EPI_BIAS
  float* out;           // EPI_BIAS / EPI_SWIGLU / EPI_LOGITS output; EPI_RESIDUAL target
  int ntiles;           // row tiles; blocks loop over them
  // EPI_LOGITS: argmax partials and the decode state it advances.
  ArgPair* partials;
  int* counter;
  int* state;           // [0] position, [1] forced length
  int* tokens;          // [capacity + 1]
  int* pred;            // [capacity]
  int capacity;
};

template <int FMT, int R, int TL, int PRO, int EPI>
__global__ __launch_bounds__(kBlock) void k_fused(FusedArgs a) {
  extern __shared__ float smem[];
  __shared__ double red[kBlock / kWave];
  __shared__ ArgPair tbest[kBlock / TL];
  __shared__ ArgPair wred[kBlock / kWave];
  __shared__ int is_last;
  float* xs = smem;
  float* xcs = smem + a.w.cols;
  if constexpr (PRO == PRO_RMSNORM) stage_rmsnorm(a.in, a.gain, a.eps, a.w.cols, xs, red);
  else stage_copy(a.in, a.w.cols, xs);
  if constexpr (FMT == QH_FMT_INT4) stage_chunk_sums(xs, a.w.cols, xcs);

  using TM = TeamMap<TL, R>;
  const int lane = TM::lane();
  float bv = NAN;
  int bi = 0x7fffffff;
  for (int tile = blockIdx.x; tile < a.ntiles; tile += gridDim.x) {
    const int row0 = TM::row0(tile);
    if (row0 >= a.w.rows) continue;
    float acc[1][R];
    mv_team<FMT, R, 1, TL>(a.w, row0, xs, 0, xcs, 0, lane, acc);
    if (lane != 0) continue;
    float v[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
      v[i] = acc[0][i];
      if constexpr (FMT == QH_FMT_INT8) v[i] = v[i] * a.w.scales[min(row0 + i, a.w.rows - 1)];
    }
#pragma unroll
    for (int i = 0; i < R; i++) {
      const int r = row0 + i;
      if (r >= a.w.rows) break;
      if constexpr (EPI == EPI_BIAS) a.out[r] = v[i] + a.bias[r];
      if constexpr (EPI == EPI_RESIDUAL) a.out[r] = a.out[r] + v[i];
      if constexpr (EPI == EPI_LOGITS) {
        a.out[r] = v[i];
        if (argmax_better(v[i], r, bv, bi)) {
          bv = v[i];
          bi = r;
        }
      }
      if constexpr (EPI == EPI_SWIGLU) {
        // Rows (2j, 2j+1) are gate row j and up row j: h[j] = silu(g) * u, evaluated
        // in f64 like the CPU path (src/core/ops.js:81-91).
        if ((i & 1) == 0 && r + 1 < a.w.rows) {
          const double g = v[i];
          a.out[r >> 1] = (float)(g / (1.0 + exp(-g)) * (double)v[i + 1]);
        }
      }
    }
  }
  if constexpr (EPI == EPI_LOGITS) {
    if (lane == 0) tbest[TM::team()] = {bv, bi};
    __syncthreads();
    if (threadIdx.x == 0) {
      float v = NAN;
      int i = 0x7fffffff;
      for (int t = 0; t < TM::kTeams; t++) {
        if (argmax_better(tbest[t].v, tbest[t].i, v, i)) {
          v = tbest[t].v;
          i = tbest[t].i;
        }
      }
      a.partials[blockIdx.x] = {v, i};
      __threadfence();
      is_last = atomicAdd(a.counter, 1) == (int)gridDim.x - 1;
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    float v = NAN;
    int i = 0x7fffffff;
    for (int b = threadIdx.x; b < (int)gridDim.x; b += kBlock) {
      const ArgPair p = a.partials[b];
      if (argmax_better(p.v, p.i, v, i)) {
        v = p.v;
        i = p.i;
      }
    }
    argmax_block(v, i, wred);
    if (threadIdx.x == 0) {
      const int tok = (a.out[0] != a.out[0]) ? 0 : i;
      const int pos = a.state[0];
      if (pos < a.capacity) a.pred[pos] = tok;
      if (pos + 1 >= a.state[1] && pos + 1 <= a.capacity) a.tokens[pos + 1] = tok;
      a.state[0] = pos + 1;
      *a.counter = 0;
    }
  }
}

// x = the bf16 embedding row of the token at the current position, widened exactly.
__global__ void k_embed(const uint16_t* __restrict__ embed, const int* __restrict__ tokens,
                        const int* __restrict__ state, int hidden, int vocab, float* __restrict__ x) {
  int tok = tokens[state[0]];
  tok = (tok < 0 || tok >= vocab) ? 0 : tok;  // ids are validated on the host
  const uint16_t* row = embed + (size_t)tok * hidden;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
    x[i] = __builtin_bit_cast(float, (uint32_t)row[i] << 16);
  }
}

__global__ void k_advance(int* state) {
  if (threadIdx.x == 0) state[0] = state[0] + 1;
}

constexpr int kLmRows = 4;        // rows per team in the output head
constexpr int kLmMaxBlocks = 1024;

template <int FMT, int TL, int R, int PRO, int EPI>
static hipError_t fused_t(hipStream_t s, FusedArgs a, int max_blocks) {
  using TM = TeamMap<TL, R>;
  a.ntiles = (a.w.rows + TM::kRowsPerBlock - 1) / TM::kRowsPerBlock;
  const int blocks = a.ntiles < max_blocks ? a.ntiles : max_blocks;
  const size_t lds = (size_t)(a.w.cols + a.w.cols / 32) * sizeof(float);
  hipLaunchKernelGGL((k_fused<FMT, R, TL, PRO, EPI>), dim3(blocks), dim3(kBlock), lds, s, a);
  return hipGetLastError();
}

template <int R, int PRO, int EPI>
static hipError_t fused(hipStream_t s, const FusedArgs& a, int max_blocks = 1 << 30) {
  const bool wide = team_width(a.w.nchunks) == 64;
  switch (a.w.format) {
    case QH_FMT_F16:
      return wide ? fused_t<QH_FMT_F16, 64, R, PRO, EPI>(s, a, max_blocks)
                  : fused_t<QH_FMT_F16, 32, R, PRO, EPI>(s, a, max_blocks);
    case QH_FMT_INT8:
      return wide ? fused_t<QH_FMT_INT8, 64, R, PRO, EPI>(s, a, max_blocks)
                  : fused_t<QH_FMT_INT8, 32, R, PRO, EPI>(s, a, max_blocks);
    default:
      return wide ? fused_t<QH_FMT_INT4, 64, R, PRO, EPI>(s, a, max_blocks)
                  : fused_t<QH_FMT_INT4, 32, R, PRO, EPI>(s, a, max_blocks);
  }
}

int lm_head_blocks(const ModelDev& m) {
  const int tl = team_width(m.lm_head.nchunks);
  const int rows_per_block = (kBlock / tl) * kLmRows;
  const int tiles = (m.vocab + rows_per_block - 1) / rows_per_block;
  return tiles < kLmMaxBlocks ? tiles : kLmMaxBlocks;
}

size_t lm_partials_bytes(const ModelDev& m) { return (size_t)lm_head_blocks(m) * sizeof(ArgPair); }

static int attention_grid(int capacity) {
  int nchunks, cps, splits;
  attn_splits(capacity, &nchunks, &cps, &splits);
  return splits;
}

hipError_t enqueue_step(hipStream_t s, const ModelDev& m, const CacheDev& c, StepInput in,
                        bool logits) {
  hipError_t e;
  if (in == STEP_GATHER) {
    hipLaunchKernelGGL(k_embed, dim3(1), dim3(kBlock), 0, s, m.embed, c.tokens, c.state, m.hidden,
                       m.vocab, c.x);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  const int kv_dim = m.kv_heads * m.head_dim;
  const size_t kv_layer = (size_t)m.kv_heads * c.capacity * m.head_dim;
  for (int L = 0; L < m.layers; L++) {
    const LayerDev& l = m.layers_host[L];
    uint16_t* kc = c.kv + (size_t)L * 2 * kv_layer;
    uint16_t* vc = kc + kv_layer;

    FusedArgs f{};
    f.eps = m.eps;
    f.w = l.qkv;
    f.in = c.x;
    f.gain = l.in_norm;
    f.bias = l.qkv_bias;
    f.out = c.qkv;
    if ((e = fused<2, PRO_RMSNORM, EPI_BIAS>(s, f)) != hipSuccess) return e;

    AttnArgs a{};
    a.q = c.qkv;
    a.k_new = c.qkv + m.hidden;
    a.v_new = c.qkv + m.hidden + kv_dim;
    a.kc = kc;
    a.vc = vc;
    a.cos_t = m.rope_cos;
    a.sin_t = m.rope_sin;
    a.d_pos = c.state;
    a.partials = c.attn_partials;
    a.counters = c.attn_counters;
    a.out = c.attn;
    a.seq = 1;
    a.capacity = c.capacity;
    a.heads = m.heads;
    a.kv_heads = m.kv_heads;
    a.s_grid = attention_grid(c.capacity);
    hipLaunchKernelGGL((k_attention<true, true>), dim3(a.s_grid, m.kv_heads, 1), dim3(kBlock), 0,
                       s, a);
    if ((e = hipGetLastError()) != hipSuccess) return e;

    f = FusedArgs{};
    f.w = l.o;
    f.in = c.attn;
    f.out = c.x;
    if ((e = fused<2, PRO_COPY, EPI_RESIDUAL>(s, f)) != hipSuccess) return e;

    f = FusedArgs{};
    f.eps = m.eps;
    f.w = l.gu;
    f.in = c.x;
    f.gain = l.post_norm;
    f.out = c.h;
    if ((e = fused<2, PRO_RMSNORM, EPI_SWIGLU>(s, f)) != hipSuccess) return e;

    f = FusedArgs{};
    f.w = l.down;
    f.in = c.h;
    f.out = c.x;
    if ((e = fused<2, PRO_COPY, EPI_RESIDUAL>(s, f)) != hipSuccess) return e;
  }
  if (!logits) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, c.state);
    return hipGetLastError();
  }
  FusedArgs f{};
  f.eps = m.eps;
  f.w = m.lm_head;
  f.in = c.x;
  f.gain = m.final_norm;
  f.out = c.logits;
  f.partials = static_cast<ArgPair*>(c.lm_partials);
  f.counter = c.lm_counter;
  f.state = c.state;
  f.tokens = c.tokens;
  f.pred = c.pred;
  f.capacity = c.capacity;
  return fused<kLmRows, PRO_RMSNORM, EPI_LOGITS>(s, f, kLmMaxBlocks);
}

}  // namespace qh
