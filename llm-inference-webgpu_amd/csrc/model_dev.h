// Device-side description of a finalized model and of one KV cache with its
// decode state: plain pointers and shapes, built once by model.cpp (the
// persistent equivalent of the reference's bind groups and uniform pool,
// src/gpu/device.js:187-206, src/gpu/model.js:100-124) and read by the
// launchers in decode.hip.
#pragma once

#include <algorithm>

#include "qh_internal.h"

namespace qh {

struct LayerDev {
  DMat qkv;          // [hidden + 2*kv_dim, hidden]: q rows, then k rows, then v rows
  DMat o;            // [hidden, hidden]
  DMat gu;           // [2*intermediate, hidden]: row 2i = gate row i, row 2i+1 = up row i
  DMat down;         // [hidden, intermediate]
  const float* qkv_bias;   // [hidden + 2*kv_dim]
  const float* in_norm;    // [hidden]
  const float* post_norm;  // [hidden]
};

struct ModelDev {
  int hidden, intermediate, layers, heads, kv_heads, head_dim, vocab, max_positions;
  int numerics;                 // QH_NUMERICS_*
  double eps;
  const LayerDev* layers_host;  // host array of per-layer descriptors
  DMat lm_head;                 // [vocab, hidden]
  const float* final_norm;
  const uint16_t* embed;        // [vocab, hidden] bf16
  const double* rope_cos;       // [max_positions, 32], f64 as the CPU path rotates
  const double* rope_sin;
};

struct CacheDev {
  int capacity;
  int vstride;         // value row length: capacity rounded up to 64
  // Per layer: keys [kv_heads][capacity][64], then values [kv_heads][64][vstride], f16.
  uint16_t* kv;
  size_t layer_elems;  // f16 elements per layer (keys + values)
  size_t key_elems;    // f16 elements of a layer's keys
  int* state;          // [0] position, [1] forced length (tokens below it are the caller's)
  int* tokens;         // [capacity + 1] token consumed at each position
  int* pred;           // [capacity] argmax after each position
  float* x;            // [hidden] residual stream
  float* q;            // [hidden] rotated queries
  float* attn;         // [hidden]
  float* h;            // [intermediate]
  float* logits;       // [vocab]
  float* scores;       // [heads][score_stride]: scores, then softmax weights
  float* maxes;        // [heads][spans(capacity)]: per-span score maxima
  int score_stride;    // capacity rounded up to 4
  int* attn_counters;  // [heads], zero between launches
  float* part;         // [heads][decode_attn_slots(capacity)][kPartStride]: split-K attention slot partials
  void* lm_partials;   // argmax block partials
  int lm_blocks;
};

// How a step obtains its input row: gathered from the embedding of tokens[pos],
// written into cache.x by the caller, carried over from the previous step (whose
// pick gathered the embedding of the token it chose), or picked in this step's first
// launch from the previous step's head (STEP_PICK: that step deferred its pick).
enum StepInput { STEP_GATHER = 0, STEP_HIDDEN = 1, STEP_CARRIED = 2, STEP_PICK = 3 };

// Optional per-launch timing: an event is recorded before every launch (tagged with
// its QH_ROLE_*) and one after the last, so launch i took events[i+1] - events[i].
struct StepTimer {
  hipEvent_t* events;
  int* roles;
  int capacity;  // events available
  int n;         // events recorded
};

// Workspace of the batched prefill for up to prefill_chunk() positions.
struct PrefillDev {
  int positions;       // rows every buffer holds
  float* X;            // [P][hidden] residual stream
  float* XN;           // [P][hidden] normalized
  float* QKV;          // [P][hidden + 2*kv_dim]
  float* Q;            // [P][hidden] rotated queries
  float* ATT;          // [P][hidden]
  float* Y;            // [P][hidden] o / down outputs
  float* GU;           // [P][2*intermediate] interleaved gate|up
  float* H;            // [P][intermediate]
  float* part;         // fast: [P][heads][kDecodeSlots][kPartStride] attention slot partials
  float* scores;       // exact past kPLds: [P][heads][score_stride] + [P][heads][spans]
  int* counters;       // exact: [P][heads], zero between launches
  void* scratch;       // matmul scratch (f64 activations, MFMA splits)
  size_t scratch_bytes;
};
struct PrefillBytes {
  size_t floats, counters, scratch;
};
constexpr int kPrefillChunk = 512;  // positions per batched prefill pass
// Positions per pass for this model and cache, and the workspace it needs.
int prefill_chunk(const ModelDev& m, const CacheDev& c);
PrefillBytes prefill_bytes(const ModelDev& m, const CacheDev& c, int matmul);
// Layers of positions past .. past+seq-1 over p.X (seq <= p.positions), writing the KV cache.
hipError_t enqueue_prefill_layers(hipStream_t s, const ModelDev& m, const CacheDev& c, const PrefillDev& p,
                                  int matmul, int past, int seq);
// p.X = embeddings of cache tokens[past .. past+seq-1].
hipError_t enqueue_embed_rows(hipStream_t s, const ModelDev& m, const CacheDev& c, const PrefillDev& p, int past,
                              int seq);

// Launches one decode position: [gather] -> layers -> (lm_head, which advances the position,
// then the argmax pick that records the token and gathers the next input row -- left to the
// next step's first launch with `defer_pick`, which that step then takes as STEP_PICK; or a
// position advance alone when `logits` is false).
hipError_t enqueue_step(hipStream_t s, const ModelDev& m, const CacheDev& c, StepInput in,
                        bool logits, StepTimer* timer = nullptr, bool defer_pick = false);
// The output head of the position state[0] over cache.x: final rmsnorm, lm_head, logits, the
// position advanced, and the pick (token recorded, next input row gathered).
hipError_t enqueue_head(hipStream_t s, const ModelDev& m, const CacheDev& c, StepTimer* timer = nullptr);
// The pick alone, after a head whose step deferred it (and that no STEP_PICK step follows).
hipError_t enqueue_pick(hipStream_t s, const ModelDev& m, const CacheDev& c);
// One launch of a decode role's kernel: QKV, ATTENTION, OPROJ, GATEUP or DOWN of `layer`, or
// HEAD (the output head's matvec, without the pick) -- the launches the step makes.
hipError_t enqueue_role(hipStream_t s, const ModelDev& m, const CacheDev& c, int role, int layer);
// cache.x = the embedding of tokens[position] (what STEP_GATHER starts with).
hipError_t enqueue_gather(hipStream_t s, const ModelDev& m, const CacheDev& c);
// Launches in one step with logits (the events a StepTimer needs, minus the final one).
int launches_per_step(const ModelDev& m, StepInput in);

// A decode matrix launch over `count` copies of its weights (for timing it over a working set
// larger than the last-level cache): copy z at w.data + z * w_stride bytes, its scales / zero
// points + z * s_stride floats, its output at out + z * out_stride floats, its argmax partials
// (the head) at partials + z * part_stride entries.
struct RoleList {
  DMat w;
  int count;
  size_t w_stride, s_stride, out_stride, part_stride;
  float* out;
  void* partials;
  int max_blocks;  // blocks per copy (0: the decode step's own grid)
  // QH_ROLE_QKV: where copy z appends its key and value rows: kc + z * k_stride and
  // vt + z * v_stride, laid out as the cache's (null: the cache itself).
  uint16_t* kc;
  uint16_t* vt;
  size_t k_stride, v_stride;
};
// The launch of QH_ROLE_QKV, OPROJ, GATEUP, DOWN (layer 0's operands otherwise) or HEAD over a list.
hipError_t enqueue_role_list(hipStream_t s, const ModelDev& m, const CacheDev& c, int role, const RoleList& list);
// The decode step's split-K attention launch (fast numerics) over `count` copies of one layer's
// cache (keys then values, copy_elems f16 apart from kv), partials per copy in `part`.
hipError_t enqueue_attention_list(hipStream_t s, const ModelDev& m, const CacheDev& c, const uint16_t* kv,
                                  int count, size_t copy_elems, float* part);
// Blocks the lm_head launch uses (sizes lm_partials).
int lm_head_blocks(const ModelDev& m);
size_t lm_partials_bytes(const ModelDev& m);
// Bytes of the split-K attention slot partials of one position (CacheDev::part).
size_t attn_part_bytes(const ModelDev& m, int capacity);

}  // namespace qh
