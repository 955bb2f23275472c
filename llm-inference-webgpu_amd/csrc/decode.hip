// The fused decode step: the whole of GpuModel.#forward for one position
// (src/gpu/model.js:240-402) as 5 launches per layer plus the output head and
// the pick, instead of the reference's ~15 dispatches and 2 copies per layer.
// Every launch reads its position from device memory, so the same launches are
// captured once in a hipGraph and replayed every token.
//
// Per layer (the order of src/cpu/model.js:89-143):
//   1. rmsnorm(x) -> q|k|v matvec + bias -> rope (f64) -> q, f16 K/V append
//   2. attention: QH_NUMERICS_FAST, split-K slot partials (a block of four waves
//      per kv head and run of 64-position chunks, the GQA group's query heads as
//      f16 MFMA columns); QH_NUMERICS_EXACT, per head in the CPU's order (f64
//      dots, global-max softmax, sequential PV sum)
//   3. [FAST: merge the attention slots while staging] o-proj matvec, residual add into x
//   4. rmsnorm(x) -> gate|up matvec -> swiglu (f64)
//   5. down matvec, residual add into x
// then rmsnorm -> lm_head -> logits and per-block argmax partials, and the pick,
// which chooses the token (the reference reads back 151,936 logits and scans
// them on the host, src/gpu/model.js:372-382, web/bench.html:129-131),
// advances the position and gathers the next position's embedding.
//
// A matvec launch is latency-bound at these sizes (a layer's int4 weights are
// 7.5 MB), so each team issues the loads of its whole share of the weights
// (WTile) before the block stages its activation vector, and a team with more
// than one work item loads the next item's weights before the current item's
// arithmetic.
#include <algorithm>
#include <type_traits>

#include "attention.h"
#include "device_common.h"
#include "model_dev.h"

namespace qh {

// PRO_PICK: rmsnorm of the embedding row of the token that the previous step's head picked
// (the pick of k_pick, made in the prologue of the step's first launch).
enum { PRO_RMSNORM = 0, PRO_COPY = 1, PRO_COMBINE = 2, PRO_PICK = 3 };
enum { EPI_QKV = 0, EPI_RESIDUAL = 1, EPI_SWIGLU = 2, EPI_LOGITS = 3 };

struct FusedArgs {
  DMat w;
  const float* in;      // rmsnorm input, or the vector to stage as-is
  const float* gain;    // rmsnorm gain
  double eps;
  float* out;           // EPI_QKV: q [hidden]; EPI_SWIGLU: h; EPI_LOGITS: logits; EPI_RESIDUAL: x
  int items;            // work items; teams stride over them
  // EPI_QKV
  const float* bias;    // [hidden + 2*kv_dim]
  const double* rope_cos;  // [positions][32] f64
  const double* rope_sin;
  uint16_t* kc;         // this layer's keys [kv_heads][capacity][64]
  uint16_t* vt;         // this layer's values [kv_heads][64][vstride]
  int vstride;
  int heads, kv_heads;
  // EPI_QKV: the decode state
  int* state;           // [0] position, [1] forced length
  int capacity;
  // EPI_LOGITS
  ArgPair* partials;     // [blocks]: each block's best (value, index)
  int* advance;          // the decode state whose position the step's head advances, or null
  // PRO_PICK: the previous step's head partials and first logit, the step's tokens and
  // predictions, the embedding, and x (written by block 0: the residual the layer adds to)
  const ArgPair* pick_parts;
  int pick_nparts;
  const float* pick_logits;
  int* tokens;
  int* pred;
  int vocab;
  const uint16_t* embed;
  float* x;
  int f32;              // fast numerics: the f32 matvec core
  // PRO_COMBINE: `in` holds the attention slot partials of the current position
  // A list of list_count copies of the weights, one per blockIdx.y (the launch timed over a
  // working set past the last-level cache): copy z reads w.data + z * list_w bytes and its
  // scales / zero points + z * list_s floats, and writes out + z * list_out floats (and its
  // argmax partials + z * list_part). 0: the one matrix of the decode step.
  int list_count;
  size_t list_w, list_s, list_out, list_part;
  size_t list_k, list_v;  // EPI_QKV: f16 elements between consecutive copies' key / value append targets
  // A flat list (the grouped loop only; grid.y 1): the items of all list_count copies in
  // one sequence, item g being item g % items of copy g / items, and each block walks
  // list_flat consecutive ones of it (a whole number of groups of every team). 0: one
  // copy per blockIdx.y.
  int list_flat;
};

// Rows of work item `it`. QKV: R/2 consecutive rope pairs (j, j+32) of one q or k
// head, or R consecutive v rows. SWIGLU: gate and up rows (2j, 2j+1) pairwise.
// Otherwise R consecutive rows, clamped to the matrix.
template <int R>
__device__ __forceinline__ int qkv_rope_items(const FusedArgs& a) {
  return (a.heads + a.kv_heads) * 32 / (R / 2);
}
template <int EPI, int R, bool CLAMP = true>
__device__ __forceinline__ void item_rows(const FusedArgs& a, int it, int (&rows)[R]) {
  if constexpr (EPI == EPI_QKV) {
    static_assert(R == 2 || R == 4, "qkv items are one or two rope pairs");
    constexpr int P = R / 2;  // divides 32, so an item's pairs share one head
    const int hidden = a.heads * kHeadDim, kvd = a.kv_heads * kHeadDim;
    if (it < qkv_rope_items<R>(a)) {
      const int head = it * P / 32, j = it * P % 32;  // heads 0..heads-1 are q, then k heads
      const int base = head < a.heads ? head * kHeadDim : hidden + (head - a.heads) * kHeadDim;
#pragma unroll
      for (int k = 0; k < P; k++) {
        rows[2 * k] = base + j + k;
        rows[2 * k + 1] = base + j + k + 32;
      }
    } else {
      const int v = it - qkv_rope_items<R>(a);
#pragma unroll
      for (int i = 0; i < R; i++) rows[i] = hidden + kvd + R * v + i;
    }
  } else {
#pragma unroll
    for (int i = 0; i < R; i++) rows[i] = CLAMP ? min(it * R + i, a.w.rows - 1) : it * R + i;
  }
}

// Operands of an item's epilogue that do not depend on its sums, loaded with its
// weights: QKV the rows' biases and the rope angles of its pairs at the current
// position; RESIDUAL the rows' residual inputs.
template <int EPI, int R>
struct EpiIn {
  static constexpr int kPairs = R / 2 > 0 ? R / 2 : 1;
  float bias[R];
  double cs[kPairs], sn[kPairs];
  float res[R];
};

template <int EPI, int R>
__device__ __forceinline__ void epi_load(const FusedArgs& a, int it, int pos, const int (&rows)[R],
                                         EpiIn<EPI, R>& e) {
  if constexpr (EPI == EPI_QKV) {
#pragma unroll
    for (int i = 0; i < R; i++) e.bias[i] = a.bias[rows[i]];
    const int j = it * (R / 2) & 31;  // the first rope pair of a q/k item (unused by v items)
#pragma unroll
    for (int k = 0; k < R / 2; k++) {
      e.cs[k] = a.rope_cos[(size_t)pos * 32 + j + k];
      e.sn[k] = a.rope_sin[(size_t)pos * 32 + j + k];
    }
  }
  if constexpr (EPI == EPI_RESIDUAL) {
#pragma unroll
    for (int i = 0; i < R; i++) e.res[i] = a.out[rows[i]];
  }
}

// Lane 0 of the team that summed item `it` (acc = the R row sums) stores it.
// acc is f64 (exact numerics) or f32 (fast numerics, int8 row scale applied).
template <int R, int EPI, typename Acc>
__device__ __forceinline__ void epilogue(const FusedArgs& a, int it, int pos, const int (&rows)[R],
                                         const Acc (&acc)[R], const EpiIn<EPI, R>& e, float& bv,
                                         int& bi) {
  constexpr bool kF32 = std::is_same<Acc, float>::value;
  if constexpr (EPI == EPI_QKV) {
    // q/k/v = f32(sum + bias) (the bias is where the CPU's f64 sum starts; f32: one add).
    float v[R];
#pragma unroll
    for (int i = 0; i < R; i++)
      v[i] = kF32 ? __fadd_rn((float)acc[i], e.bias[i]) : (float)((double)acc[i] + (double)e.bias[i]);
    const int hidden = a.heads * kHeadDim, kvd = a.kv_heads * kHeadDim;
    if (pos >= a.capacity) return;  // the host keeps positions inside the cache
    if (it < qkv_rope_items<R>(a)) {
      const int head = it * (R / 2) / 32, j0 = it * (R / 2) % 32;
#pragma unroll
      for (int k = 0; k < R / 2; k++) {
        const int j = j0 + k;
        float lo, hi;
        rope_pair(v[2 * k], v[2 * k + 1], e.cs[k], e.sn[k], &lo, &hi);
        if (head < a.heads) {
          a.out[head * kHeadDim + j] = lo;
          a.out[head * kHeadDim + j + 32] = hi;
        } else {
          uint16_t* kr = a.kc + ((size_t)(head - a.heads) * a.capacity + pos) * kHeadDim;
          kr[j] = __builtin_bit_cast(uint16_t, (_Float16)lo);
          kr[j + 32] = __builtin_bit_cast(uint16_t, (_Float16)hi);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < R; i++) {
        const int el = rows[i] - hidden - kvd;  // kv head el/64, dimension el%64
        a.vt[(size_t)el * a.vstride + pos] = __builtin_bit_cast(uint16_t, (_Float16)v[i]);
      }
    }
  }
  if constexpr (EPI == EPI_RESIDUAL) {
#pragma unroll
    for (int i = 0; i < R; i++) {
      const int r = it * R + i;
      if (r < a.w.rows) a.out[r] = __fadd_rn(e.res[i], (float)acc[i]);
    }
  }
  if constexpr (EPI == EPI_SWIGLU) {
    // h[j] = silu(g) * u over the f32 gate and up outputs, in f64 (src/core/ops.js:81-91),
    // or in f32 (fast numerics, the WGSL kernel's evaluation).
#pragma unroll
    for (int i = 0; i < R; i += 2) {
      const int r = it * R + i;
      if (r + 1 < a.w.rows) {
        if constexpr (kF32) {
          a.out[r >> 1] = swiglu_f32((float)acc[i], (float)acc[i + 1]);
        } else {
          const double g = (float)acc[i];
          const double u = (float)acc[i + 1];
          a.out[r >> 1] = (float)(g / (1.0 + exp(-g)) * u);
        }
      }
    }
  }
  if constexpr (EPI == EPI_LOGITS) {
#pragma unroll
    for (int i = 0; i < R; i++) {
      const int r = it * R + i;
      if (r >= a.w.rows) break;
      const float v = (float)acc[i];
      a.out[r] = v;
      if (argmax_better(v, r, bv, bi)) {
        bv = v;
        bi = r;
      }
    }
  }
}

// One work item's loads (rows, weights, epilogue operands) for item min(it, last):
// past the end a team re-reads the last item, unconditionally, so no load waits
// on a branch.
template <int FMT, int TL, int R, int KC, int EPI>
struct Item {
  int rows[R];
  WTile<FMT, R, KC> w;
  EpiIn<EPI, R> e;
  // EPI_OPS: also the epilogue operands (the one-item form; the loop form loads them per
  // group, see k_fused). STREAM_S: scales and zero points streamed (wtile_load).
  template <bool EPI_OPS, bool STREAM_S = false>
  __device__ __forceinline__ void load(const FusedArgs& a, int it, int pos, int lane) {
    const int i = min(it, a.items - 1);
    item_rows<EPI, R>(a, i, rows);
    wtile_load<FMT, R, KC, TL, STREAM_S>(a.w, rows, lane, w);
    if constexpr (EPI_OPS) epi_load<EPI, R>(a, i, pos, rows, e);
  }
  // The weights of item `it`, which may lie past the last item (CLAMP off: rows past the
  // matrix read as zeros through the buffer resources).
  __device__ __forceinline__ void load_buf(const FusedArgs& a, const BufMat& b, int it, int lane, int wbase,
                                           int sbase) {
    item_rows<EPI, R, false>(a, it, rows);
    wtile_load_buf<FMT, R, KC, TL>(a.w, b, rows, lane, wbase, sbase, w);
  }
};

constexpr int kLmRows = 4;          // rows per team in the output head
constexpr int kLmMaxBlocks = 1024;  // the head's blocks (see fused_blocks)
constexpr int kPickLoads = 4;       // partial loads per thread of a pick
static_assert(kLmMaxBlocks <= kPickLoads * kBlock, "one round of partial loads");

// The pick that ends a step with logits, from its output head's block partials: the token is
// the best of them (lowest index among equal maxima, NaN logits -> 0, the reference's
// host-side scan of src/gpu/model.js:372-382). The head has advanced the position to
// q = state[0], so the pick is the prediction at q - 1 (recorded in pred) and, from the
// forced length on, the token at q; the next input is the caller's token at q below the
// forced length, else the pick. Block-wide: every thread of the block takes part.
struct Pick {
  ArgPair part[kPickLoads];
  int q, forced, given;
  float first;
  // Every load that does not depend on the argmax: all the partials at once (from clamped
  // indices -- a repeated pair does not change the best), the position, the forced length,
  // the caller's token at q and the first logit.
  __device__ __forceinline__ void load(const ArgPair* __restrict__ parts, int nparts, const float* __restrict__ logits,
                                       const int* state, const int* tokens, int capacity) {
#pragma unroll
    for (int k = 0; k < kPickLoads; k++) part[k] = parts[min((int)threadIdx.x + k * kBlock, nparts - 1)];
    q = state[0];
    forced = state[1];
    given = tokens[min(q, capacity)];
    first = logits[0];
  }
  // The next input token, known to every thread after one barrier (`red`: a pair per wave,
  // each thread reducing the waves' bests); `record`: this block writes pred and tokens.
  __device__ __forceinline__ int finish(ArgPair* red, bool record, int* pred, int* tokens, int capacity,
                                        int vocab) const {
    float v = part[0].v;
    int i = part[0].i;
#pragma unroll
    for (int k = 1; k < kPickLoads; k++) {
      if (argmax_better(part[k].v, part[k].i, v, i)) {
        v = part[k].v;
        i = part[k].i;
      }
    }
    argmax_wave(v, i);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = {v, i};
    __syncthreads();
    v = red[0].v;
    i = red[0].i;
#pragma unroll
    for (int w = 1; w < kBlock / kWave; w++) {
      if (argmax_better(red[w].v, red[w].i, v, i)) {
        v = red[w].v;
        i = red[w].i;
      }
    }
    const int tok = (first != first) ? 0 : i;
    if (record && threadIdx.x == 0) {
      if (q >= 1 && q - 1 < capacity) pred[q - 1] = tok;
      if (q >= forced && q <= capacity) tokens[q] = tok;
    }
    const bool caller = q < forced && q <= capacity;
    const int t = caller ? given : tok;
    return (t < 0 || t >= vocab) ? 0 : t;  // ids are validated on the host
  }
};

// How a team walks its items (k_fused's LOOP): one item; a ring of two buffers over
// all of them, each item's epilogue on lane 0; groups of kLoopGroup items whose
// epilogues run together.
enum { LOOP_ONE = 0, LOOP_RING = 1, LOOP_GROUP = 2 };
constexpr int kLoopBuffers = 2;     // item buffers of a group (loads kLoopBuffers - 1 items ahead)
constexpr int kLoopGroup = 8;       // items of a team per straight-line group

// LOOP_ONE: one item per team, its epilogue on lane 0 with operands loaded alongside
// its weights. LOOP_RING (the output head; streaming grids of rows with little
// epilogue work): two named item buffers alternate, so the next item's loads are in
// flight during this one's arithmetic, each epilogue on lane 0. LOOP_GROUP (streaming
// grids whose epilogues cost more): groups of kLoopGroup items, each group
// straight-line code with a ring of kLoopBuffers buffers whose loads are issued and
// consumed inside it (loads left in flight across a loop's back edge land in registers
// that the loop header reassigns, and the compiler then waits for all of them there);
// the group's epilogues run together at its end: lane 0 leaves each item's row sums
// in LDS and lane j of the team runs item j's epilogue, its operands loaded at the
// group's start -- one pass of epilogue instructions and one load per operand for
// kLoopGroup items. F32: the fast-numerics core (f32 staging with chunk sums, f32
// sums); else f64 as the CPU path sums.
template <int FMT, int TL, int R, int KC, int PRO, int EPI, int LOOP, bool F32>
__global__ __launch_bounds__(kBlock) void k_fused(FusedArgs a) {
  constexpr int NBUF = LOOP == LOOP_GROUP ? kLoopBuffers : LOOP == LOOP_RING ? 2 : 1;
  extern __shared__ double smem[];
  __shared__ double red[kBlock / kWave];
  constexpr bool kGroup = LOOP == LOOP_GROUP;
  constexpr int kBestPerTeam = kGroup ? kLoopGroup : 1;  // lanes of a team that track a best logit
  __shared__ ArgPair tbest[kBlock / TL * kBestPerTeam];
  __shared__ typename std::conditional<F32, float, double>::type
      gsum[kGroup ? kBlock / TL : 1][kGroup ? kLoopGroup : 1][R];
  __shared__ float wl[PRO == PRO_COMBINE ? kBlock : 1];
  __shared__ ArgPair pick_red[PRO == PRO_PICK ? kBlock / kWave : 1];
  using Acc = typename std::conditional<F32, float, double>::type;
  using T = Teams<TL>;
  if (blockIdx.y) {  // a copy of a weight list (block-uniform; never in the decode step)
    const size_t z = blockIdx.y;
    a.w.data += z * a.list_w;
    if (a.w.scales) a.w.scales += z * a.list_s;
    if (a.w.zeros) a.w.zeros += z * a.list_s;
    a.out += z * a.list_out;
    if (a.partials) a.partials += z * a.list_part;
    if (a.kc) a.kc += z * a.list_k;
    if (a.vt) a.vt += z * a.list_v;
  }
  const int lane = T::lane();
  const int stride = gridDim.x * T::kTeams;
  int it = blockIdx.x * T::kTeams + T::team();
  int pos = 0;
  if constexpr (EPI == EPI_QKV) pos = a.state[0];
  if constexpr (EPI == EPI_LOGITS) {
    // The step's head moves the position on (no block of this launch reads it).
    if (a.advance && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) a.advance[0] = a.advance[0] + 1;
  }

  // Loads in this order: the activations (the previous launch's output), then this
  // team's first item -- vector loads return in issue order, so the staging below
  // waits for the activations only, while the weights are still in flight.
  // PRO_PICK: the pick's loads, then the weights, then its token's row once the partials
  // are reduced (the row's wait then covers the weights too, issued a round trip earlier).
  using Pro = typename std::conditional<PRO == PRO_COMBINE, CombineIn, StageIn>::type;
  Pro pin;
  [[maybe_unused]] Pick pk;
  if constexpr (PRO == PRO_COMBINE) {
    pin.load(a.in, a.heads);
  } else if constexpr (PRO == PRO_PICK) {
    pk.load(a.pick_parts, a.pick_nparts, a.pick_logits, a.state, a.tokens, a.capacity);
    pin.load_gain(a.gain, a.w.cols);
  } else {
    pin.load(a.in, PRO == PRO_RMSNORM ? a.gain : nullptr, a.w.cols);
  }
  Item<FMT, TL, R, KC, EPI> ring[NBUF];
  if constexpr (!kGroup) ring[0].template load<true, LOOP == LOOP_ONE>(a, it, pos, lane);
  if constexpr (PRO == PRO_PICK) {
    const bool first_block = blockIdx.x == 0 && blockIdx.y == 0;
    const int t = pk.finish(pick_red, first_block, a.pred, a.tokens, a.capacity, a.vocab);
    pin.load_bf16(a.embed + (size_t)t * a.w.cols, a.w.cols);
    if (first_block) pin.store(a.x, a.w.cols);
  }
  constexpr bool kNorm = PRO == PRO_RMSNORM || PRO == PRO_PICK;
  if constexpr (F32) {
    float* xs = reinterpret_cast<float*>(smem);
    const XLayoutF lay = chunk_layout_f<FMT>(a.w.nchunks);
    if constexpr (kNorm)
      stage_rmsnorm_finish_f32<FMT>(pin, (float)a.eps, a.w.cols, xs, reinterpret_cast<float*>(red), lay);
    else if constexpr (PRO == PRO_COMBINE) stage_attn_combine_f32<FMT>(pin, a.heads, xs, lay, wl);
    else stage_copy_finish_f32<FMT>(pin, a.w.cols, xs, lay);
  } else {
    double* xs = smem;
    const XLayout lay = chunk_layout<FMT>(a.w.nchunks);
    if constexpr (kNorm) stage_rmsnorm_finish(pin, a.eps, a.w.cols, xs, red, lay);
    else if constexpr (PRO == PRO_COMBINE) stage_attn_combine(pin, a.heads, xs, lay, wl);
    else stage_copy_finish(pin, a.w.cols, xs, lay);
  }

  auto dot = [&](const WTile<FMT, R, KC>& w, Acc (&acc)[R]) {
    if constexpr (F32) wtile_dot_f32<FMT, R, KC, TL>(a.w, w, reinterpret_cast<const float*>(smem), lane, acc);
    else wtile_dot<FMT, R, KC, TL>(a.w, w, smem, lane, acc);
  };
  // The grouped loop with one chunk per lane (f32 core) sums every item against the same
  // staged chunk, so the lane reads it into registers once.
  constexpr bool kXReg = kGroup && F32 && KC == 1;
  [[maybe_unused]] XChunk<FMT> xr;
  if constexpr (kXReg) {
    const float* xs = reinterpret_cast<const float*>(smem);
    const int c = min(lane, a.w.nchunks - 1);
    xr.load(xs + 4 * c, 4 * a.w.nchunks, FMT == QH_FMT_F16 ? 0.f : xs[a.w.cols + c]);
  }
  float bv = NAN;
  int bi = 0x7fffffff;
  Acc acc[R];
  if constexpr (LOOP == LOOP_ONE) {
    if (it < a.items) {
      dot(ring[0].w, acc);
      if (lane == 0) epilogue<R, EPI, Acc>(a, it, pos, ring[0].rows, acc, ring[0].e, bv, bi);
    }
  } else if constexpr (LOOP == LOOP_RING) {
    while (it < a.items) {
      ring[1].template load<true>(a, it + stride, pos, lane);
      __builtin_amdgcn_sched_barrier(0);
      dot(ring[0].w, acc);
      if (lane == 0) epilogue<R, EPI, Acc>(a, it, pos, ring[0].rows, acc, ring[0].e, bv, bi);
      it += stride;
      if (it >= a.items) break;
      ring[0].template load<true>(a, it + stride, pos, lane);
      __builtin_amdgcn_sched_barrier(0);
      dot(ring[1].w, acc);
      if (lane == 0) epilogue<R, EPI, Acc>(a, it, pos, ring[1].rows, acc, ring[1].e, bv, bi);
      it += stride;
    }
  } else {
    constexpr int kPastEnd = 0x7fff0000;  // a byte offset past any flat list
    // The team's items are g0, g0 + gs, ... below gend: items of this block's copy, or
    // of a flat list (the block's share of it; item g is item g % items of copy
    // g / items). Item j of a group (g0 + j*gs) lives in ring[j % NBUF]; past the end
    // its loads read zeros or unused rows and the arithmetic is skipped. Lane j <
    // kLoopGroup of the team runs item j's epilogue (gl: the lanes past the group
    // repeat its last).
    const int team = T::team(), gl = min(lane, kLoopGroup - 1);
    const bool flat = a.list_flat > 0;
    int g0 = it, gs = stride, gend = a.items;
    BufMat bm;
    if (flat) {
      const int total = a.items * a.list_count;
      g0 = blockIdx.x * a.list_flat + team;
      gs = T::kTeams;
      gend = min(total, (blockIdx.x + 1) * a.list_flat);
      bm = buf_mat(a.w, a.list_count, a.list_w, a.list_s);
    } else {
      bm = buf_mat(a.w);
    }
    // (copy, item) of sequence entry g; of g0 + d from g0's by carrying into the next copies
    auto split = [&](int g, int& z, int& l) {
      z = flat ? g / a.items : 0;
      l = g - z * a.items;
    };
    for (; g0 < gend; g0 += kLoopGroup * gs) {
      int z0, l0;
      split(g0, z0, l0);
      auto step = [&](int d, int& z, int& l) {
        z = z0;
        l = l0 + d;
        if (flat)
          while (l >= a.items) {
            l -= a.items;
            z++;
          }
      };
      int ze, le;
      split(min(g0 + gl * gs, gend - 1), ze, le);
      FusedArgs ae = a;  // this lane's epilogue item's copy
      ae.out = a.out + (size_t)ze * a.list_out;
      if (a.kc) ae.kc = a.kc + (size_t)ze * a.list_k;
      if (a.vt) ae.vt = a.vt + (size_t)ze * a.list_v;
      int erows[R];
      EpiIn<EPI, R> e;
      item_rows<EPI, R>(ae, le, erows);
      epi_load<EPI, R>(ae, le, pos, erows, e);
      auto load = [&](Item<FMT, TL, R, KC, EPI>& item, int j) {
        int z, l;
        step(j * gs, z, l);
        // past the block's share of a flat list: offsets beyond the resources, which read
        // zeros without touching memory (the list is under 2 GiB)
        const bool live = !flat || g0 + j * gs < gend;
        item.load_buf(a, bm, live ? l : 0, lane, live ? z * (int)a.list_w : kPastEnd,
                      live ? z * (int)a.list_s * (int)sizeof(float) : kPastEnd);
      };
#pragma unroll
      for (int j = 0; j + 1 < NBUF; j++) load(ring[j], j);
#pragma unroll
      for (int j = 0; j < kLoopGroup; j++) {
        constexpr int kAhead = NBUF - 1;
        if (j + kAhead < kLoopGroup) load(ring[(j + kAhead) % NBUF], j + kAhead);
        __builtin_amdgcn_sched_barrier(0);
        if (g0 + j * gs < gend) {  // uniform over the team (the butterfly in dot)
          if constexpr (kXReg) wtile_dot_f32_x<FMT, R, TL>(a.w, ring[j % NBUF].w, xr, lane, acc);
          else dot(ring[j % NBUF].w, acc);
          if (lane == 0) {
#pragma unroll
            for (int i = 0; i < R; i++) gsum[team][j][i] = acc[i];
          }
        }
      }
      __builtin_amdgcn_wave_barrier();  // a team is inside one wave: lane 0's LDS stores land first
      if (lane < kLoopGroup && g0 + gl * gs < gend) {
        Acc sums[R];
#pragma unroll
        for (int i = 0; i < R; i++) sums[i] = gsum[team][lane][i];
        epilogue<R, EPI, Acc>(ae, le, pos, erows, sums, e, bv, bi);
      }
      __builtin_amdgcn_wave_barrier();  // read before the next group's stores
    }
  }
  if constexpr (EPI == EPI_LOGITS) {
    // Each tracking lane's best (argmax_better is a total order, so the merge order
    // does not change the result).
    if (lane < kBestPerTeam) tbest[T::team() * kBestPerTeam + lane] = {bv, bi};
    __syncthreads();
    if (threadIdx.x == 0) {
      float v = NAN;
      int i = 0x7fffffff;
      for (int t = 0; t < T::kTeams * kBestPerTeam; t++) {
        if (argmax_better(tbest[t].v, tbest[t].i, v, i)) {
          v = tbest[t].v;
          i = tbest[t].i;
        }
      }
      a.partials[blockIdx.x] = {v, i};  // reduced by k_pick, the next launch
    }
  }
}

// The pick ending a step whose next step does not make it in its first launch (a decode
// call's last step, a prefill with logits, a scored position): the Pick above, and x becomes
// the embedding of the next input token.
__global__ __launch_bounds__(kBlock) void k_pick(const ArgPair* __restrict__ partials, int nparts,
                                                 const float* __restrict__ logits, const int* state,
                                                 int* tokens, int* pred, int capacity,
                                                 const uint16_t* __restrict__ embed, int hidden,
                                                 int vocab, float* __restrict__ x) {
  __shared__ ArgPair wred[kBlock / kWave];
  Pick pk;
  pk.load(partials, nparts, logits, state, tokens, capacity);
  const int t = pk.finish(wred, true, pred, tokens, capacity, vocab);
  const uint16_t* row = embed + (size_t)t * hidden;
  for (int k = threadIdx.x; k < hidden; k += kBlock) x[k] = __builtin_bit_cast(float, (uint32_t)row[k] << 16);
}

// x = the bf16 embedding row of the token at the current position, widened exactly.
__global__ void k_embed(const uint16_t* __restrict__ embed, const int* __restrict__ tokens,
                        const int* __restrict__ state, int capacity, int hidden, int vocab,
                        float* __restrict__ x) {
  const int pos = state[0];
  if (pos < 0 || pos > capacity) return;  // the host keeps positions inside the cache
  int tok = tokens[pos];
  tok = (tok < 0 || tok >= vocab) ? 0 : tok;  // ids are validated on the host
  const uint16_t* row = embed + (size_t)tok * hidden;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
    x[i] = __builtin_bit_cast(float, (uint32_t)row[i] << 16);
  }
}

__global__ void k_advance(int* state) {
  if (threadIdx.x == 0) state[0] = state[0] + 1;
}


// Chunks per lane a kernel is built for: the smallest instantiated count that
// covers ceil(nchunks / TL).
static int kc_for(int nchunks) {
  const int tl = team_width(nchunks);
  const int need = (nchunks + tl - 1) / tl;
  for (int kc : {1, 2, 3, 5, 8, 16})
    if (need <= kc) return kc;
  return 0;
}

// One item per team, or for more items than max_blocks' teams (the output head) max_blocks blocks
// whose teams take every stride-th item: floor or ceil(items / teams) each, so each CU's blocks
// (1024 = four per CU) stream nearly the same number of rows (950 blocks of equal counts left a
// quarter of the CUs with three blocks where the rest had four).
static int fused_blocks(int items, int teams, int max_blocks) {
  const int blocks = (items + teams - 1) / teams;
  return blocks > max_blocks ? max_blocks : blocks;
}

// Which forms of k_fused a launch site can use, so each site instantiates only those:
// GRID_ONE, one item per team (the decode step's layer launches: their grid always covers
// the items); GRID_RING and GRID_GROUP, teams walking several items in that loop form
// (streaming grids); GRID_ANY, one item per team or the ring, whichever the grid needs
// (the output head).
enum { GRID_ONE = 0, GRID_RING = 1, GRID_GROUP = 2, GRID_ANY = 3 };

template <int FMT, int TL, int R, int KC, int PRO, int EPI, int GRID, bool F32>
static hipError_t fused_l(hipStream_t s, FusedArgs a, int items, int max_blocks) {
  using T = Teams<TL>;
  a.items = items;
  a.list_flat = 0;
  if constexpr (GRID == GRID_GROUP) {
    if (a.list_count > 1 && (size_t)a.list_count * a.list_w < ((size_t)1 << 31) &&
        (size_t)a.list_count * a.list_s * sizeof(float) < ((size_t)1 << 31)) {
      // A weight list on the grouped loop runs flat: as many blocks as the device holds at
      // once share all the copies' items equally (one block per copy leaves the copies'
      // blocks outnumbering the resident slots by a fraction, and the last round runs on
      // part of the device).
      const size_t lds = F32 ? (size_t)staged_f32_floats(a.w.cols, a.w.nchunks) * sizeof(float)
                             : (size_t)a.w.cols * sizeof(double);
      auto kernel = k_fused<FMT, TL, R, KC, PRO, EPI, LOOP_GROUP, F32>;
      int dev = 0, cus = 0, per_cu = 0;
      hipError_t e = hipGetDevice(&dev);
      if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
      if (e == hipSuccess) e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kBlock, lds);
      if (e != hipSuccess) return e;
      const size_t total = (size_t)items * a.list_count, teams = T::kTeams;
      const size_t resident = std::max(1, cus * per_cu);
      const size_t per = ((total + resident - 1) / resident + teams - 1) / teams * teams;
      a.list_flat = (int)per;
      hipLaunchKernelGGL(kernel, dim3((total + per - 1) / per, 1), dim3(kBlock), lds, s, a);
      return hipGetLastError();
    }
  }
  const int blocks = fused_blocks(items, T::kTeams, max_blocks);
  const size_t lds = F32 ? (size_t)staged_f32_floats(a.w.cols, a.w.nchunks) * sizeof(float)
                         : (size_t)a.w.cols * sizeof(double);
  const dim3 grid(blocks, a.list_count > 1 ? a.list_count : 1);
  const bool one = (size_t)blocks * T::kTeams >= (size_t)items;
  // the grouped loop addresses the matrix through 32-bit buffer offsets
  if (GRID == GRID_GROUP && (size_t)a.w.rows * a.w.row_bytes >= ((size_t)1 << 31)) return hipErrorInvalidValue;
  if constexpr (GRID == GRID_ONE) {
    if (!one) return hipErrorInvalidValue;
  }
  constexpr int kLoop = GRID == GRID_GROUP ? LOOP_GROUP : LOOP_RING;
  if constexpr (GRID == GRID_ONE) {
    hipLaunchKernelGGL((k_fused<FMT, TL, R, KC, PRO, EPI, LOOP_ONE, F32>), grid, dim3(kBlock), lds, s, a);
  } else if constexpr (GRID == GRID_ANY) {
    if (one) hipLaunchKernelGGL((k_fused<FMT, TL, R, KC, PRO, EPI, LOOP_ONE, F32>), grid, dim3(kBlock), lds, s, a);
    else hipLaunchKernelGGL((k_fused<FMT, TL, R, KC, PRO, EPI, LOOP_RING, F32>), grid, dim3(kBlock), lds, s, a);
  } else {
    hipLaunchKernelGGL((k_fused<FMT, TL, R, KC, PRO, EPI, kLoop, F32>), grid, dim3(kBlock), lds, s, a);
  }
  return hipGetLastError();
}

template <int FMT, int TL, int R, int KC, int PRO, int EPI, int GRID>
static hipError_t fused_t(hipStream_t s, const FusedArgs& a, int items, int max_blocks) {
  if (a.f32) return fused_l<FMT, TL, R, KC, PRO, EPI, GRID, true>(s, a, items, max_blocks);
  return fused_l<FMT, TL, R, KC, PRO, EPI, GRID, false>(s, a, items, max_blocks);
}

template <int FMT, int R, int PRO, int EPI, int GRID>
static hipError_t fused_f(hipStream_t s, const FusedArgs& a, int items, int max_blocks) {
  if (team_width(a.w.nchunks) == 32) return fused_t<FMT, 32, R, 1, PRO, EPI, GRID>(s, a, items, max_blocks);
  switch (kc_for(a.w.nchunks)) {
    case 1: return fused_t<FMT, 64, R, 1, PRO, EPI, GRID>(s, a, items, max_blocks);
    case 2: return fused_t<FMT, 64, R, 2, PRO, EPI, GRID>(s, a, items, max_blocks);
    case 3: return fused_t<FMT, 64, R, 3, PRO, EPI, GRID>(s, a, items, max_blocks);
    case 5: return fused_t<FMT, 64, R, 5, PRO, EPI, GRID>(s, a, items, max_blocks);
    case 8: return fused_t<FMT, 64, R, 8, PRO, EPI, GRID>(s, a, items, max_blocks);
    case 16: return fused_t<FMT, 64, R, 16, PRO, EPI, GRID>(s, a, items, max_blocks);
    default: return hipErrorInvalidValue;  // rows longer than the model limits allow
  }
}

template <int R, int PRO, int EPI, int GRID>
static hipError_t fused(hipStream_t s, const FusedArgs& a, int items, int max_blocks) {
  switch (a.w.format) {
    case QH_FMT_F16: return fused_f<QH_FMT_F16, R, PRO, EPI, GRID>(s, a, items, max_blocks);
    case QH_FMT_INT8: return fused_f<QH_FMT_INT8, R, PRO, EPI, GRID>(s, a, items, max_blocks);
    default: return fused_f<QH_FMT_INT4, R, PRO, EPI, GRID>(s, a, items, max_blocks);
  }
}

int lm_head_blocks(const ModelDev& m) {
  const int teams = kBlock / team_width(m.lm_head.nchunks);
  return fused_blocks((m.vocab + kLmRows - 1) / kLmRows, teams, kLmMaxBlocks);
}

size_t lm_partials_bytes(const ModelDev& m) { return (size_t)lm_head_blocks(m) * sizeof(ArgPair); }

size_t attn_part_bytes(const ModelDev& m, int capacity) {
  return (size_t)m.heads * decode_attn_slots(capacity) * kPartStride * sizeof(float);
}

int launches_per_step(const ModelDev& m, StepInput in) {
  return (in == STEP_GATHER ? 1 : 0) + 5 * m.layers + 2;
}

// Records the event that opens a launch of `role` (see StepTimer).
static hipError_t mark(hipStream_t s, StepTimer* t, int role) {
  if (!t) return hipSuccess;
  if (t->n >= t->capacity) return hipErrorInvalidValue;
  t->roles[t->n] = role;
  return hipEventRecord(t->events[t->n++], s);
}

hipError_t enqueue_gather(hipStream_t s, const ModelDev& m, const CacheDev& c) {
  hipLaunchKernelGGL(k_embed, dim3(1), dim3(kBlock), 0, s, m.embed, c.tokens, c.state, c.capacity,
                     m.hidden, m.vocab, c.x);
  return hipGetLastError();
}

// Sets a launch up for a weight list (RoleList), else leaves it as the decode step's.
static void apply_list(FusedArgs& f, const RoleList* list) {
  if (!list) return;
  f.w = list->w;
  f.list_count = list->count;
  f.list_w = list->w_stride;
  f.list_s = list->s_stride;
  f.list_out = list->out_stride;
  f.list_part = list->part_stride;
  f.out = list->out;
  if (list->partials) f.partials = static_cast<ArgPair*>(list->partials);
  if (list->kc) {  // the q|k|v copies' own K/V append targets
    f.kc = list->kc;
    f.vt = list->vt;
    f.list_k = list->k_stride;
    f.list_v = list->v_stride;
  }
}

// The launch of `role` (QKV, ATTENTION, OPROJ, GATEUP or DOWN) for layer L; with `list`, the
// same launch over a list of copies of its weights (matrix roles only); `pick` (QKV): the
// previous step's pick made in this launch's prologue, its input row the picked token's.
static hipError_t layer_role(hipStream_t s, const ModelDev& m, const CacheDev& c, int L, int role,
                             const RoleList* list = nullptr, bool pick = false) {
  // A streaming grid (blocks per copy given) takes more rows per work item where that helps: each
  // team then walks many items, and the rows of one item share its loop overhead. A row is
  // summed in the same order either way (its chunks per lane and the butterfly depend on the
  // row length only).
  const bool stream = list && list->max_blocks > 0;
  const int mb = stream ? list->max_blocks : 1 << 30;  // blocks per copy
  const int kv_dim = m.kv_heads * m.head_dim;
  const LayerDev& l = m.layers_host[L];
  uint16_t* kc = c.kv + (size_t)L * c.layer_elems;
  uint16_t* vt = kc + c.key_elems;
  FusedArgs f{};
  f.f32 = m.numerics == QH_NUMERICS_FAST;
  if (list && role == QH_ROLE_ATTENTION) return hipErrorInvalidValue;
  switch (role) {
    case QH_ROLE_QKV:
      f.eps = m.eps;
      f.w = l.qkv;
      f.in = c.x;
      f.gain = l.in_norm;
      f.bias = l.qkv_bias;
      f.out = c.q;
      f.rope_cos = m.rope_cos;
      f.rope_sin = m.rope_sin;
      f.kc = kc;
      f.vt = vt;
      f.vstride = c.vstride;
      f.heads = m.heads;
      f.kv_heads = m.kv_heads;
      f.state = c.state;
      f.capacity = c.capacity;
      apply_list(f, list);
      if (stream)
        return fused<4, PRO_RMSNORM, EPI_QKV, GRID_GROUP>(s, f, ((m.heads + m.kv_heads) * 64 + kv_dim) / 4, mb);
      if (pick) {
        if (list) return hipErrorInvalidValue;
        f.pick_parts = static_cast<const ArgPair*>(c.lm_partials);
        f.pick_nparts = lm_head_blocks(m);
        f.pick_logits = c.logits;
        f.tokens = c.tokens;
        f.pred = c.pred;
        f.vocab = m.vocab;
        f.embed = m.embed;
        f.x = c.x;
        return fused<2, PRO_PICK, EPI_QKV, GRID_ONE>(s, f, (m.heads + m.kv_heads) * 32 + kv_dim / 2, mb);
      }
      return fused<2, PRO_RMSNORM, EPI_QKV, GRID_ONE>(s, f, (m.heads + m.kv_heads) * 32 + kv_dim / 2, mb);
    case QH_ROLE_ATTENTION:
      if (m.numerics == QH_NUMERICS_FAST) {
        SlotArgs a{};
        a.q = c.q;
        a.kc = kc;
        a.vt = vt;
        a.d_pos = c.state;
        a.part = c.part;
        a.capacity = c.capacity;
        a.vstride = c.vstride;
        a.heads = m.heads;
        a.kv_heads = m.kv_heads;
        return launch_attn_decode(s, a, 1, 1, c.attn);  // a long cache merges into c.attn
      } else {
        ExactArgs a{};
        a.q = c.q;
        a.kc = kc;
        a.vt = vt;
        a.d_pos = c.state;
        a.scores = c.scores;
        a.maxes = c.maxes;
        a.counters = c.attn_counters;
        a.out = c.attn;
        a.capacity = c.capacity;
        a.vstride = c.vstride;
        a.heads = m.heads;
        a.kv_heads = m.kv_heads;
        a.score_stride = c.score_stride;
        a.max_stride = attn_spans(c.capacity);
        if (c.capacity <= kPLds) {
          hipLaunchKernelGGL(k_attn_block, dim3(m.heads, 1), dim3(kAttnThreads), 0, s, a);
        } else {
          hipLaunchKernelGGL(k_attn_exact, dim3(attn_spans(c.capacity), m.heads, 1), dim3(kBlock), 0, s, a);
        }
      }
      return hipGetLastError();
    case QH_ROLE_OPROJ:
      f.w = l.o;
      f.out = c.x;
      if (m.numerics == QH_NUMERICS_FAST && !decode_attn_long(c.capacity)) {
        f.in = c.part;
        f.heads = m.heads;
        f.state = c.state;
        apply_list(f, list);
        if (stream) return fused<4, PRO_COMBINE, EPI_RESIDUAL, GRID_GROUP>(s, f, (l.o.rows + 3) / 4, mb);
        return fused<1, PRO_COMBINE, EPI_RESIDUAL, GRID_ONE>(s, f, l.o.rows, mb);
      }
      if (m.numerics == QH_NUMERICS_FAST) {  // a long cache: the attention output is merged already
        f.in = c.attn;
        apply_list(f, list);
        if (stream) return fused<1, PRO_COPY, EPI_RESIDUAL, GRID_RING>(s, f, l.o.rows, mb);
        return fused<1, PRO_COPY, EPI_RESIDUAL, GRID_ONE>(s, f, l.o.rows, mb);
      }
      f.in = c.attn;
      apply_list(f, list);
      if (stream) return fused<1, PRO_COPY, EPI_RESIDUAL, GRID_RING>(s, f, l.o.rows, mb);
      return fused<2, PRO_COPY, EPI_RESIDUAL, GRID_ONE>(s, f, (l.o.rows + 1) / 2, mb);
    case QH_ROLE_GATEUP:
      f.eps = m.eps;
      f.w = l.gu;
      f.in = c.x;
      f.gain = l.post_norm;
      f.out = c.h;
      apply_list(f, list);
      if (stream) return fused<4, PRO_RMSNORM, EPI_SWIGLU, GRID_GROUP>(s, f, l.gu.rows / 4, mb);
      return fused<2, PRO_RMSNORM, EPI_SWIGLU, GRID_ONE>(s, f, l.gu.rows / 2, mb);
    case QH_ROLE_DOWN:
      f.w = l.down;
      f.in = c.h;
      f.out = c.x;
      apply_list(f, list);
      if (stream) return fused<1, PRO_COPY, EPI_RESIDUAL, GRID_RING>(s, f, l.down.rows, mb);
      return fused<1, PRO_COPY, EPI_RESIDUAL, GRID_ONE>(s, f, l.down.rows, mb);
    default:
      return hipErrorInvalidValue;
  }
}

// The output head's matvec alone (final rmsnorm, lm_head, logits, block argmax partials);
// `advance`: the step's head, which moves the position on for the pick that follows.
static hipError_t head_matvec(hipStream_t s, const ModelDev& m, const CacheDev& c, const RoleList* list = nullptr,
                              bool advance = false) {
  FusedArgs f{};
  f.f32 = m.numerics == QH_NUMERICS_FAST;
  f.eps = m.eps;
  f.w = m.lm_head;
  f.in = c.x;
  f.gain = m.final_norm;
  f.out = c.logits;
  f.partials = static_cast<ArgPair*>(c.lm_partials);
  if (advance && !list) f.advance = c.state;
  apply_list(f, list);
  const int mb = list && list->max_blocks > 0 ? std::min(list->max_blocks, kLmMaxBlocks) : kLmMaxBlocks;
  return fused<kLmRows, PRO_RMSNORM, EPI_LOGITS, GRID_ANY>(s, f, (m.vocab + kLmRows - 1) / kLmRows, mb);
}

hipError_t enqueue_role_list(hipStream_t s, const ModelDev& m, const CacheDev& c, int role, const RoleList& list) {
  if (role == QH_ROLE_HEAD) return head_matvec(s, m, c, &list);
  return layer_role(s, m, c, 0, role, &list);
}

hipError_t enqueue_attention_list(hipStream_t s, const ModelDev& m, const CacheDev& c, const uint16_t* kv,
                                  int count, size_t copy_elems, float* part) {
  if (m.numerics != QH_NUMERICS_FAST) return hipErrorInvalidValue;
  SlotArgs a{};
  a.q = c.q;
  a.kc = kv;
  a.vt = kv + c.key_elems;
  a.d_pos = c.state;
  a.part = part;
  a.capacity = c.capacity;
  a.vstride = c.vstride;
  a.heads = m.heads;
  a.kv_heads = m.kv_heads;
  a.list_k = copy_elems;
  a.list_v = copy_elems;
  a.list_part = (size_t)m.heads * decode_attn_slots(c.capacity) * kPartStride;
  return launch_attn_decode(s, a, 1, count);  // the slots alone
}

hipError_t enqueue_role(hipStream_t s, const ModelDev& m, const CacheDev& c, int role, int layer) {
  if (role == QH_ROLE_HEAD) return head_matvec(s, m, c);
  if (layer < 0 || layer >= m.layers) return hipErrorInvalidValue;
  return layer_role(s, m, c, layer, role);
}

hipError_t enqueue_step(hipStream_t s, const ModelDev& m, const CacheDev& c, StepInput in,
                        bool logits, StepTimer* timer, bool defer_pick) {
  hipError_t e;
  if (in == STEP_GATHER) {
    if ((e = mark(s, timer, QH_ROLE_EMBED)) != hipSuccess) return e;
    if ((e = enqueue_gather(s, m, c)) != hipSuccess) return e;
  }
  for (int L = 0; L < m.layers; L++) {
    for (int role : {QH_ROLE_QKV, QH_ROLE_ATTENTION, QH_ROLE_OPROJ, QH_ROLE_GATEUP, QH_ROLE_DOWN}) {
      const bool pick = in == STEP_PICK && L == 0 && role == QH_ROLE_QKV;
      if ((e = mark(s, timer, role)) != hipSuccess) return e;
      if ((e = layer_role(s, m, c, L, role, nullptr, pick)) != hipSuccess) return e;
    }
  }
  if (!logits) {
    if ((e = mark(s, timer, QH_ROLE_HEAD)) != hipSuccess) return e;
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(64), 0, s, c.state);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  } else if (defer_pick) {
    if ((e = mark(s, timer, QH_ROLE_HEAD)) != hipSuccess) return e;
    if ((e = head_matvec(s, m, c, nullptr, true)) != hipSuccess) return e;
  } else if ((e = enqueue_head(s, m, c, timer)) != hipSuccess) {
    return e;
  }
  return mark(s, timer, QH_ROLE_COUNT);
}

hipError_t enqueue_head(hipStream_t s, const ModelDev& m, const CacheDev& c, StepTimer* timer) {
  hipError_t e;
  if ((e = mark(s, timer, QH_ROLE_HEAD)) != hipSuccess) return e;
  if ((e = head_matvec(s, m, c, nullptr, true)) != hipSuccess) return e;
  // The pick gathers the next input row, so it is timed with the gathers.
  if ((e = mark(s, timer, QH_ROLE_EMBED)) != hipSuccess) return e;
  return enqueue_pick(s, m, c);
}

hipError_t enqueue_pick(hipStream_t s, const ModelDev& m, const CacheDev& c) {
  hipLaunchKernelGGL(k_pick, dim3(1), dim3(kBlock), 0, s, static_cast<const ArgPair*>(c.lm_partials),
                     lm_head_blocks(m), c.logits, c.state, c.tokens, c.pred, c.capacity, m.embed, m.hidden,
                     m.vocab, c.x);
  return hipGetLastError();
}

}  // namespace qh
