/*
 * libqwen_hip.so: the MI355X (gfx950) backend for the Qwen2.5 engine's GPU layer.
 *
 * This C ABI is the drop-in boundary. It replaces the operator surface the
 * reference's model loop calls into src/gpu (abho7/llm-inference-webgpu):
 * GpuContext (src/gpu/device.js:21-392), the eight WGSL kernels
 * (src/gpu/kernels.js:33-530) and GpuModel (src/gpu/model.js:69-403). A
 * Node-API addon (js/addon/qwen_napi.cpp) and a ctypes module (qwen_hip.py)
 * bind it; both only marshal arguments.
 *
 * Conventions
 *   - Plain C: opaque handles, plain pointers and sizes, int status (QH_OK = 0).
 *     On failure, qh_last_error() returns a message for the calling thread.
 *   - Pointers named d_* are device pointers (from qh_alloc or any HIP
 *     allocation on the context's device); h_* are host pointers, borrowed for
 *     the duration of the call.
 *   - Operators are asynchronous on the context's one stream, in call order,
 *     like WebGPU's queue (device.js:152-165). qh_download / qh_sync / calls
 *     returning host results wait.
 *   - A context is used by one thread at a time; forward/decode refuse
 *     reentrancy (src/gpu/model.js:228-232).
 *   - Every operator checks its arguments on the host before launching, so a
 *     shape the kernels do not support is an error, never a device fault.
 */
#ifndef QWEN_HIP_H
#define QWEN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QH_ABI_VERSION 1

/* Status codes. The reference throws Error / RangeError synchronously for misuse
 * (src/gpu/model.js:231,249-254; src/gpu/device.js:48-56,153,254). */
enum {
  QH_OK = 0,
  QH_ERR_INVALID = 1, /* bad argument or unsupported shape (Error) */
  QH_ERR_RANGE = 2,   /* cache capacity, rope table, vocabulary (RangeError) */
  QH_ERR_BUSY = 3,    /* forward() already running (model.js:231) */
  QH_ERR_DEVICE = 4,  /* HIP runtime failure, or no device */
  QH_ERR_NOMEM = 5,
  QH_ERR_STATE = 6    /* e.g. model not finalized, tensor missing */
};

/* Weight storage formats. QH_FMT_INT8 / QH_FMT_INT4 take the reference
 * quantizer's arrays verbatim (src/core/quantize.js:36-151): int8 codes
 * row-major + one f32 scale per row; int4 codes two per byte, low nibble =
 * even flat index, + one f32 scale and one f32 integer zero point per group. */
enum {
  QH_FMT_F32 = 0,  /* norms and biases */
  QH_FMT_F16 = 1,  /* the reference's shipping weight format (model.js:165-173) */
  QH_FMT_INT8 = 2,
  QH_FMT_INT4 = 3,
  QH_FMT_BF16 = 4  /* the checkpoint format; the embedding gather table */
};

const char* qh_last_error(void);
int qh_abi_version(void);

/* ------------------------------------------------------------------ context
 * GpuContext.create (device.js:47-77), describe (:382-391), done (:272). */
typedef struct qh_ctx qh_ctx;
int qh_device_count(int* count);
int qh_open(int device, qh_ctx** out);
int qh_close(qh_ctx* ctx);
/* JSON text: device name, arch, CU count, HBM bytes, LDS per workgroup. */
int qh_describe(qh_ctx* ctx, char* buf, size_t len);
int qh_sync(qh_ctx* ctx);
/* The context's hipStream_t, for callers that time or order their own work on it. */
void* qh_stream(qh_ctx* ctx);

/* ------------------------------------------------------------------- memory
 * GpuContext.upload / empty / readF32 (device.js:80-99, 229-251). */
int qh_alloc(qh_ctx* ctx, size_t bytes, void** d_out);
int qh_free(qh_ctx* ctx, void* d_ptr);
int qh_upload(qh_ctx* ctx, void* d_dst, const void* h_src, size_t bytes);
int qh_download(qh_ctx* ctx, void* h_dst, const void* d_src, size_t bytes);
int qh_memset(qh_ctx* ctx, void* d_dst, int value, size_t bytes);
/* GpuContext.copy (device.js:168-175): bytes from d_src to d_dst (non-overlapping), a
 * copy kernel on the context stream (so it can sit inside a captured graph). */
int qh_copy(qh_ctx* ctx, void* d_dst, const void* d_src, size_t bytes);

/* Device events on the context stream (GpuContext.timed, device.js:301-338). */
typedef struct qh_event qh_event;
int qh_event_create(qh_ctx* ctx, qh_event** out);
int qh_event_record(qh_ctx* ctx, qh_event* ev);
int qh_event_elapsed_ms(qh_event* start, qh_event* stop, float* ms); /* waits for stop */
int qh_event_destroy(qh_event* ev);

/* ---------------------------------------------------------------- operators
 * One descriptor for a weight matrix [rows, cols] in device memory. */
typedef struct {
  int32_t format;      /* QH_FMT_F16 | QH_FMT_INT8 | QH_FMT_INT4 */
  int32_t rows, cols;
  int32_t group;       /* int4 group size (a multiple of 32 dividing cols); else 0 */
  const void* d_data;  /* f16 [rows*cols] | int8 [rows*cols] | u8 [rows*cols/2] */
  const float* d_scales; /* int8 [rows] | int4 [rows*cols/group] */
  const float* d_zeros;  /* int4 [rows*cols/group] */
} qh_weight;

/* MATVEC / batchedMatvec (kernels.js:33-79, 232-290; dispatch model.js:284-317):
 * y[b, r] = sum_c W[r, c] * x[b, c] (+ bias[r]) for b < seq. Every position is summed in
 * the same order whatever `seq` is, so prefill agrees with decode bit for bit.
 * x f32 [seq, cols], bias f32 [rows] or NULL, y f32 [seq, rows]. */
int qh_matvec(qh_ctx* ctx, const qh_weight* w, const float* d_x, const float* d_bias,
              float* d_y, int32_t seq);
/* The batched-prefill contraction on the matrix cores (no counterpart kernel in the reference,
 * whose prefill is batchedMatvec, kernels.js:232-290, selected by model.js:297-306):
 * y [M, rows] = x [M, cols] . W^T (+ bias) for int8 / int4 weights, as int8 MFMA
 * (v_mfma_i32_16x16x64_i8) of the exact weight codes against each activation row written as a
 * 24-bit fixed-point integer in three int8 digit planes: every product and sum is exact in
 * int32, and the digits and scales are recombined in f64 once per output (int8) or per group
 * (int4), ~4e-7 relative to the f64 sum. cols must be a multiple of 32. x, y f32 [M, cols] /
 * [M, rows]. */
int qh_matmul_prefill(qh_ctx* ctx, const qh_weight* w, const float* d_x, const float* d_bias,
                      float* d_y, int32_t M);
/* qh_matmul_prefill without any allocation: no counterpart in the reference; for callers that
 * cannot allocate device memory (code under hipGraph capture, tight serving loops, harnesses
 * that forbid it). The same kernels and results, bit for bit, with the digit planes, row factors
 * and split partials in a 24 MiB array the library holds on each device from qh_open until the
 * process ends, instead of a temporary allocation per call. Shapes whose scratch exceeds it are
 * QH_ERR_RANGE (every M <= 512 with cols <= 8192 fits). Every call on one device shares that
 * array: calls that overlap on one GPU (another stream, another context) race; calls in order on
 * one stream do not. */
int qh_matmul_prefill_noalloc(qh_ctx* ctx, const qh_weight* w, const float* d_x, const float* d_bias,
                              float* d_y, int32_t M);
/* The isolated-matvec form: f16 activation x [cols], f32 y [rows]. */
int qh_matvec_xh(qh_ctx* ctx, const qh_weight* w, const uint16_t* d_x, float* d_y);
/* A list of `count` same-shape matrices in one launch: weight i starts at
 * d_data + i*data_stride bytes (scales / zeros at i*scale_stride floats), x_i at
 * d_x + i*x_stride halves (x_stride 0: one shared x), y_i at d_y + i*rows floats.
 * This is how a working set larger than the last-level cache is streamed in one launch. */
int qh_matvec_xh_list(qh_ctx* ctx, const qh_weight* w, int32_t count, size_t data_stride,
                      size_t scale_stride, const uint16_t* d_x, size_t x_stride, float* d_y);

/* RMSNORM (kernels.js:300-343): y = x / sqrt(mean(x^2) + eps) * gain, eps inside the root.
 * x, y f32 [rows, cols]; gain f32 [cols]. */
int qh_rmsnorm(qh_ctx* ctx, const float* d_x, const float* d_gain, float* d_y, int32_t rows,
               int32_t cols, double eps);

/* ROPE (kernels.js:360-389), in place over v [rows, heads*head_dim], half-split pairs
 * (j, j + head_dim/2), cos/sin tables [positions, head_dim/2] f32 indexed at base_pos + row.
 * `table_positions` bounds the index: base_pos + rows > table_positions is QH_ERR_RANGE. */
int qh_rope(qh_ctx* ctx, float* d_v, const float* d_cos, const float* d_sin,
            int32_t table_positions, int32_t rows, int32_t heads, int32_t head_dim,
            int32_t base_pos);
/* Host helper that builds the tables in f64 and stores f32 (src/core/ops.js:99-136). */
int qh_rope_tables(int32_t head_dim, double theta, int32_t positions, float* h_cos,
                   float* h_sin);

/* The KV append (model.js:336-338): k, v f32 [seq, kv_heads*head_dim] written as f16 at
 * positions past .. past+seq-1. The key cache is position-major per head
 * [kv_heads, capacity, head_dim]; the value cache is dimension-major per head
 * [kv_heads, head_dim, vstride] with vstride = capacity rounded up to a multiple of 64
 * (qh_value_cache_bytes gives its size), the layout the attention kernels stream. */
int qh_kv_append(qh_ctx* ctx, const float* d_k, const float* d_v, uint16_t* d_key_cache,
                 uint16_t* d_value_cache, int32_t capacity, int32_t kv_heads, int32_t head_dim,
                 int32_t past, int32_t seq);
/* Bytes of a value cache for `capacity` positions (no counterpart in the reference, whose
 * cache layout is internal to src/gpu/model.js). */
size_t qh_value_cache_bytes(int32_t capacity, int32_t kv_heads, int32_t head_dim);

/* ATTENTION (kernels.js:404-499): causal GQA over the f16 caches of qh_kv_append. Query t (absolute
 * position past+t) attends to positions 0..past+t. Query head h reads kv head
 * h / (heads/kv_heads). Scale 1/sqrt(head_dim). q (rotated), out f32 [seq, heads*head_dim].
 * Evaluated in the order of groupedAttention (src/core/attention.js:32-66): f64 dots stored
 * f32, softmax by the global max with an f64 sum, and a sequential f32 sum over positions, so
 * the result is the CPU's to the bit up to f64 ordering. head_dim must be 64. */
int qh_attention(qh_ctx* ctx, const float* d_q, const uint16_t* d_key_cache,
                 const uint16_t* d_value_cache, int32_t capacity, float* d_out, int32_t seq,
                 int32_t past, int32_t heads, int32_t kv_heads, int32_t head_dim);
/* As qh_attention with a split-K online softmax over 64-position chunks: the decode step's
 * attention, one block per (query, kv head, run of chunks) with the kv head's query heads as
 * the columns of f16 matrix-core products, so each K/V chunk is read once per kv head; 16 runs
 * per head up to 8192 positions of capacity, 128 past it; the runs are merged in order.
 * Exact only to f32 rounding (~1e-6 of the output); the fast form for long contexts. A
 * query's result does not depend on `seq`: prefill rows equal one-query calls bit for bit. */
int qh_attention_splitk(qh_ctx* ctx, const float* d_q, const uint16_t* d_key_cache,
                        const uint16_t* d_value_cache, int32_t capacity, float* d_out,
                        int32_t seq, int32_t past, int32_t heads, int32_t kv_heads,
                        int32_t head_dim);

/* As qh_attention on the matrix cores (the prefill's attention when the model's matmul mode is
 * QH_MATMUL_MFMA): a flash attention whose q.k and p.v products run on f16 MFMA with q and p
 * split into two f16 terms each, f32 accumulation, online softmax. Exact only to f32 rounding
 * (~1e-6 of the output). */
int qh_attention_mfma(qh_ctx* ctx, const float* d_q, const uint16_t* d_key_cache,
                      const uint16_t* d_value_cache, int32_t capacity, float* d_out, int32_t seq,
                      int32_t past, int32_t heads, int32_t kv_heads, int32_t head_dim);

/* qh_attention_splitk for one query (position `past`) against `count` caches of the same shape
 * in one launch: key cache i at d_key_cache + i*key_stride, value cache i at d_value_cache +
 * i*value_stride (f16 elements); out [count][heads*head_dim]. How a working set of caches larger
 * than the last-level cache is streamed (no counterpart in the reference). */
int qh_attention_splitk_list(qh_ctx* ctx, const float* d_q, const uint16_t* d_key_cache,
                             const uint16_t* d_value_cache, size_t key_stride, size_t value_stride,
                             int32_t count, int32_t capacity, float* d_out, int32_t past, int32_t heads,
                             int32_t kv_heads, int32_t head_dim);
/* The launch shape qh_attention_splitk_list takes for a query at position context-1 over
 * `count` caches with `kv_heads` kv heads: *h_slots runs of chunks per (cache, kv head) (1, 4,
 * 16 or 64; with one the block writes the output itself and no merge launch runs) and
 * *h_waves waves per run (1, 4 or 8). Host-only: it lets a test name the kernel a list call
 * runs (no counterpart in the reference). */
int qh_attention_list_plan(int32_t context, int32_t count, int32_t kv_heads, int32_t* h_slots,
                           int32_t* h_waves);

/* SWIGLU (kernels.js:502-515): gate = silu(gate) * up, in place. */
int qh_swiglu(qh_ctx* ctx, float* d_gate, const float* d_up, int32_t n);
/* ADD (kernels.js:518-530): x += delta. */
int qh_add(qh_ctx* ctx, float* d_x, const float* d_delta, int32_t n);
/* The caller's argmax (web/bench.html:129-131): strict '>' scan semantics -- the lowest index
 * of the maximum, NaN never wins unless at index 0. Waits; writes one int to *h_index. */
int qh_argmax(qh_ctx* ctx, const float* d_v, int32_t n, int32_t* h_index);

/* ------------------------------------------------------------ host helpers
 * The reference quantizer (src/core/quantize.js:36-132), restated for the load path. */
int qh_quantize_int8(const float* h_w, int32_t rows, int32_t cols, int8_t* h_q,
                     float* h_scales);
int qh_quantize_int4(const float* h_w, int32_t rows, int32_t cols, int32_t group,
                     uint8_t* h_q, float* h_scales, float* h_zeros);
/* The same conversion on the device, for the loader (GpuModel.load's per-tensor upload,
 * src/gpu/model.js:165-173: bf16ToF32Array, then quantizeInt8 / quantizeInt4 of
 * src/core/quantize.js:36-132 or f32ToF16Array of src/core/dtype.js:81-113). d_src holds
 * [rows, cols] values: src_format QH_FMT_BF16 (bits, widened exactly) or QH_FMT_F32. format
 * QH_FMT_F32 | F16 | INT8 (d_scales [rows]) | INT4 (d_scales, d_zeros [rows * cols/group]; group
 * even and dividing cols). Outputs as in qh_weight, bit-identical with qh_quantize_int8 /
 * qh_quantize_int4 and the reference's f16 narrowing (NaN payloads included). Asynchronous on
 * the context stream. */
int qh_quantize(qh_ctx* ctx, int32_t src_format, const void* d_src, int32_t rows, int32_t cols,
                int32_t format, int32_t group, void* d_data, float* d_scales, float* d_zeros);

/* Seeded synthetic inputs (the reference has no random-init facility). Counter-based, so any
 * element can be generated independently and every platform produces the same bits.
 * Values: std * (sum of 12 uniform u32 / 2^32 - 6), the Irwin-Hall approximation of N(0,1),
 * computed exactly in f64 and rounded once to f32. `name` selects the stream. */
int qh_synth_f32(uint64_t seed, const char* name, double std, size_t offset, size_t n,
                 float* h_out);
/* As qh_synth_f32, then rounded to bf16 (round to nearest even): a checkpoint tensor. */
int qh_synth_bf16(uint64_t seed, const char* name, double std, size_t offset, size_t n,
                  uint16_t* h_out);
/* Uniform token ids in [0, vocab). */
int qh_synth_tokens(uint64_t seed, const char* name, int32_t vocab, size_t n, int32_t* h_out);

/* -------------------------------------------------------------------- model
 * GpuModel (model.js:86-403) and GpuKVCache (model.js:69-84). */
typedef struct {
  int32_t hidden, intermediate, layers, heads, kv_heads, head_dim, vocab;
  double rope_theta, eps;
  int32_t max_positions; /* rope table rows (GpuModel.load maxPositions, model.js:148) */
} qh_config;

typedef struct qh_model qh_model;
typedef struct qh_cache qh_cache;

int qh_model_create(qh_ctx* ctx, const qh_config* cfg, qh_model** out);

/* Arithmetic of the model's forward/decode kernels.
 *   QH_NUMERICS_FAST (default): the arithmetic of the reference's WebGPU kernels -- matvecs
 *     summed in f32 (the quantization scale factored out of each 16-byte chunk), rmsnorm and
 *     swiglu in f32, split-K online-softmax attention (one pass over the f16 cache, each K/V
 *     chunk read once per kv head for the whole GQA group, q.k and p.v on f16 MFMA with q and p
 *     split into two f16 terms and f32 sums; slots merged in the o-projection's staging).
 *     Each launch agrees with the CPU path's
 *     arithmetic to ~1e-6 relative; logits of a whole forward within the reference's 1e-4
 *     (an f16 cache entry that rounds the other way moves later layers slightly).
 *   QH_NUMERICS_EXACT: every kernel evaluates the CPU path's arithmetic in its order (f64
 *     accumulation stored to f32, attention by the global max with a sequential f32 PV sum),
 *     so logits and the f16 cache are the oracle's bit for bit up to f64 ordering noise.
 * Set before the model's first cache is created. No counterpart in the reference, whose GPU
 * path has one f32 arithmetic (src/gpu/kernels.js). */
enum { QH_NUMERICS_FAST = 0, QH_NUMERICS_EXACT = 1 };
int qh_model_set_numerics(qh_model* m, int32_t numerics);

/* How forward() processes several positions (GpuModel.load's `matmul` option, model.js:87-98,
 * 133-138, 297-317):
 *   QH_MATMUL_BATCHED (default): all positions per layer, each weight read once per 8-position
 *     tile (batchedMatvec); every output is summed as the decode step sums it, so a prefill and
 *     the same positions decoded one by one give the same bits (README.md:256-272).
 *   QH_MATMUL_MATVEC: one decode step per position (the reference's 'matvec').
 *   QH_MATMUL_MFMA: all positions per layer, int8/int4 weights contracted on int8 MFMA
 *     (qh_matmul_prefill's digit planes; f16 weights use the batched tiles) and the prompt's
 *     attention on f16 MFMA (qh_attention_mfma); not bitwise equal to the others, within the
 *     reference's 1e-4 of them, as its 'tiled' path was (web/scaling.html:122-127). The
 *     reference's matmul option 'tiled' selects this mode in the bindings.
 * May be changed between forward() calls. */
enum { QH_MATMUL_BATCHED = 0, QH_MATMUL_MATVEC = 1, QH_MATMUL_MFMA = 2 };
int qh_model_set_matmul(qh_model* m, int32_t matmul);
/* Upload one tensor by its checkpoint name (src/core/config.js:88-119), copied from host.
 *   model.embed_tokens.weight  QH_FMT_BF16 [vocab, hidden]: the input gather table
 *   lm_head.weight             F16 | INT8 | INT4 [vocab, hidden]: the output projection (for a
 *                              tied model, the loader's copy of the embedding, model.js:184)
 *   model.norm.weight, model.layers.N.{input_layernorm,post_attention_layernorm}.weight  F32
 *   model.layers.N.self_attn.{q,k,v}_proj.bias  F32
 *   model.layers.N.self_attn.{q,k,v,o}_proj.weight, model.layers.N.mlp.{gate,up,down}_proj.weight
 *                              F16 | INT8 | INT4; all seven of a layer in one format.
 * rows/cols give the shape (cols = 1 for vectors); data/scales/zeros as in qh_weight. */
int qh_model_set_tensor(qh_model* m, const char* name, int32_t format, int32_t rows,
                        int32_t cols, int32_t group, const void* h_data, const float* h_scales,
                        const float* h_zeros);
/* As qh_model_set_tensor, from the checkpoint's own values: h_src holds [rows, cols] bf16 bits
 * (src_format QH_FMT_BF16) or f32 values (QH_FMT_F32), uploaded in that width and converted to
 * `format` on the device by qh_quantize's kernels -- GpuModel.load's per-tensor loop
 * (src/gpu/model.js:165-181) with the widening, quantizing and narrowing moved off the host.
 * The stored codes, scales and zero points equal those of qh_quantize_int8 / qh_quantize_int4
 * on the widened values. The gather table takes bf16 values as they are. */
int qh_model_load_tensor(qh_model* m, const char* name, int32_t src_format, int32_t rows,
                         int32_t cols, const void* h_src, int32_t format, int32_t group);
/* Checks that every tensor is present with its shape, builds the rope tables and the fused
 * device layouts. Afterwards the model is immutable. */
int qh_model_finalize(qh_model* m);
int qh_model_free(qh_model* m);
/* Device bytes held by the model's weights. */
int qh_model_bytes(qh_model* m, size_t* bytes);
/* The dimensions the model was created with (for bindings that size their outputs from the
 * model itself; the reference's GpuModel keeps its `config`, src/gpu/model.js:88). */
int qh_model_config(qh_model* m, qh_config* out);

int qh_cache_create(qh_model* m, int32_t capacity, qh_cache** out);  /* model.js:209 */
int qh_cache_free(qh_cache* c);
int qh_cache_length(qh_cache* c, int32_t* length);
/* Rewind to an earlier length (cache.reset() is length 0, model.js:83). */
int qh_cache_set_length(qh_cache* c, int32_t length);
/* [kv_heads, length, head_dim] f32 per layer (the ONNX 'present' layout, src/cpu/cache.js:97-115). */
int qh_cache_present(qh_cache* c, int32_t layer, float* h_key, float* h_value);

/* GpuModel.forward (model.js:227-402): `hidden` is the embedded input [seq, hidden] f32.
 * h_logits (may be NULL) receives the last position's [vocab] logits; h_argmax (may be NULL)
 * the device argmax of them. */
int qh_forward(qh_model* m, qh_cache* c, const float* h_hidden, int32_t seq, float* h_logits,
               int32_t* h_argmax);
/* As qh_forward, with the embedding gather done on the device from token ids. */
int qh_forward_tokens(qh_model* m, qh_cache* c, const int32_t* h_ids, int32_t seq,
                      float* h_logits, int32_t* h_argmax);
/* Greedy decode (the loop of web/bench.html:121-134) as `steps` replays of hipGraph-captured
 * decode steps: token -> gather -> 24 layers -> lm_head -> argmax -> next token, all on the
 * device (each step's argmax and the next token's gather made by the next step's first launch,
 * the last step's by a launch of its own). h_tokens [steps] receives the generated ids; the
 * first step consumes `first_token`. */
int qh_decode(qh_model* m, qh_cache* c, int32_t first_token, int32_t steps, int32_t* h_tokens);
/* Enqueue the graph replays without waiting (for timing); qh_decode_collect waits and copies. */
int qh_decode_launch(qh_model* m, qh_cache* c, int32_t first_token, int32_t steps);
int qh_decode_collect(qh_model* m, qh_cache* c, int32_t steps, int32_t* h_tokens);
/* Captures and uploads the cache's decode graphs (a first step, one later step, and a run of 8
 * later steps) now instead
 * of at the first decode that needs them, so a timed decode replays graphs that are already
 * resident. Optional: qh_decode_launch captures whatever is missing. No counterpart in the
 * reference, which records every step anew (src/gpu/model.js:261). */
int qh_decode_prepare(qh_model* m, qh_cache* c);
/* Scores a token sequence the way the reference's perplexity page does
 * (web/perplexity.html:146-170): ids[0..n-2] are fed one position at a time through the cache
 * (each step's input forced, as forward() of one token), and h_nll[t] (n - 1 doubles) receives
 * the negative log-likelihood of ids[t+1] under step t's logits, -(l[target] - max - log(sum
 * exp(l - max))) in f64 on the device. Perplexity is exp(mean(h_nll)). The cache advances by
 * n - 1 positions; QH_ERR_RANGE for ids outside the vocabulary or a cache without room. */
int qh_score(qh_model* m, qh_cache* c, const int32_t* h_ids, int32_t n, double* h_nll);

/* use_graph = 0: later decodes on this cache enqueue every kernel of a step directly instead
 * of replaying the captured graph (same kernels, same tokens), and batched forwards enqueue
 * every layer's kernels directly instead of replaying the graph of a prompt shape (first
 * position, length, matmul path, numerics) this cache has run before -- a shape is captured on
 * its second use, up to 8 shapes per cache. For tools that cannot follow graph launches. No
 * counterpart in the reference, which re-encodes every step (src/gpu/model.js:261). Default 1. */
int qh_decode_use_graph(qh_cache* c, int32_t use_graph);

/* Kernel roles of one decode step, the grouping of the reference's in-situ profile
 * ("GPU ms per token by role", web/decode-profile.html:88-192). */
enum {
  QH_ROLE_EMBED = 0,     /* embedding gather */
  QH_ROLE_QKV = 1,       /* rmsnorm + q|k|v matvec + bias */
  QH_ROLE_ATTENTION = 2, /* rope + f16 KV append + split-K GQA attention */
  QH_ROLE_OPROJ = 3,     /* o projection + residual */
  QH_ROLE_GATEUP = 4,    /* rmsnorm + gate|up matvec + swiglu */
  QH_ROLE_DOWN = 5,      /* down projection + residual */
  QH_ROLE_HEAD = 6,      /* final rmsnorm + lm_head + argmax */
  QH_ROLE_COUNT = 7
};
/* As qh_decode, but with direct launches, each timed from its dispatch's own start to its end
 * (the interval a kernel tracer reports, nothing enqueued between the launches), so each
 * kernel's in-situ time is measured (GpuContext.timed, src/gpu/device.js:301-338).
 * h_role_ms[QH_ROLE_COUNT] receives the summed milliseconds per role over all steps and
 * h_role_launches[QH_ROLE_COUNT] the launch counts. Tokens are identical to qh_decode's. */
int qh_decode_profile(qh_model* m, qh_cache* c, int32_t first_token, int32_t steps,
                      int32_t* h_tokens, float* h_role_ms, int32_t* h_role_launches);
/* The average duration of one decode launch of `role` (QH_ROLE_QKV .. QH_ROLE_DOWN, cycling
 * through the layers, or QH_ROLE_HEAD: the output head's matvec): `reps` of the step's own
 * launches at the cache's current position, back to back on the context stream between two
 * events, so no event sits between them (the hot-vs-cold isolation of
 * web/decode-profile.html:239-283). It overwrites the position's decode scratch (and, for the
 * residual roles, the hidden row): rewind or re-prefill before decoding on. */
int qh_decode_kernel_time(qh_model* m, qh_cache* c, int32_t role, int32_t reps, float* us_per_launch);
/* The same launch of `role` (QH_ROLE_QKV .. QH_ROLE_HEAD) timed cold: one launch reads
 * *copies copies of its operands (layer 0's matrix, the output head, or -- QH_ROLE_ATTENTION,
 * fast numerics -- layer 0's f16 cache) that together exceed min_bytes, so with min_bytes past
 * the 256 MB last-level cache every launch streams from HBM (the cold side of
 * web/decode-profile.html:239-283; BASELINE config 2 rotates >= 512 MiB the same way). The
 * copies are allocated, filled and freed by the call; *us_per_launch covers all copies. */
int qh_decode_kernel_time_cold(qh_model* m, qh_cache* c, int32_t role, size_t min_bytes, int32_t reps,
                               float* us_per_launch, int32_t* copies);
/* qh_decode_kernel_time_cold with the launch's grid sized for streaming instead of for one
 * step's latency (matrix roles; blocks_per_copy 0 = the step's own grid): each block stages its
 * activation vector once and then walks many rows with the next rows' loads in flight, in the
 * decode kernel's multi-item forms -- down and the head blocks_per_copy blocks per copy; q|k|v,
 * o-proj and gate|up as one flat list over the device's resident blocks (blocks_per_copy does
 * not change that grid), their epilogues batched per group of rows. q|k|v copies append their
 * key/value rows to scratch rows of their own, not to the cache. Every row is summed as the
 * step sums it: the call checks the first and the last copy's outputs against the step's own
 * launch shape bit for bit and fails with QH_ERR_STATE if they differ. Shows what the step's
 * kernels stream when latency does not size their grid. No counterpart in the reference. */
int qh_decode_kernel_time_stream(qh_model* m, qh_cache* c, int32_t role, size_t min_bytes, int32_t reps,
                                 int32_t blocks_per_copy, float* us_per_launch, int32_t* copies);
/* What bounds a batch-1 launch, measured on this device (no counterpart in the reference, which
 * measures the same bounds in web/decode-profile.html:288-327): `launches` launches of `blocks`
 * 256-thread blocks captured as one graph and replayed -- kind 0 does nothing; kind 1 reads the
 * 896-float vector the previous launch wrote (as every decode launch reads its predecessor's
 * output) and writes 4 floats per block; kind 2 is kind 1 reading nothing -- giving microseconds
 * per launch. */
int qh_probe_launch_floor(qh_ctx* ctx, int32_t kind, int32_t blocks, int32_t launches, float* us_per_launch);
/* The pure-read ceiling: a streaming read of `bytes` (allocated and freed here), GB/s. */
int qh_read_ceiling(qh_ctx* ctx, size_t bytes, int32_t reps, float* gbps);

/* Kernel-level parity access to one decode step (the reference's per-kernel harness,
 * web/kernels.html:56-134, checks each WGSL kernel against the CPU on the same inputs; these
 * entry points give the decode step's fused launches the same treatment). No counterpart in
 * the reference's GpuModel.
 *
 * The decode vectors of a cache: QH_VEC_X the residual row [hidden], QH_VEC_Q the rotated
 * queries [hidden], QH_VEC_H the swiglu output [intermediate], QH_VEC_LOGITS [vocab]; and,
 * read-only, QH_VEC_KEY / QH_VEC_VALUE: layer `layer`'s cache row at the current position
 * (cache length) as f32 [kv_heads * head_dim], kv head major. */
enum { QH_VEC_X = 0, QH_VEC_Q = 1, QH_VEC_H = 2, QH_VEC_LOGITS = 3, QH_VEC_KEY = 4, QH_VEC_VALUE = 5 };
/* Writes h_in (if not NULL) into the vector, then reads it into h_out (if not NULL). Waits. */
int qh_cache_vector(qh_cache* c, int32_t which, int32_t layer, const float* h_in, float* h_out);
/* Runs the one launch of `role` that a decode step makes for `layer`, at position = the cache
 * length (which does not advance), and waits:
 *   QH_ROLE_QKV        x -> rmsnorm -> q|k|v + bias -> rope -> q, and the f16 K/V row at the position
 *   QH_ROLE_ATTENTION  q and the cache rows 0..position -> attention (FAST: the slot partials)
 *   QH_ROLE_OPROJ      (FAST: merge of the slot partials) -> o-projection -> x += it
 *   QH_ROLE_GATEUP     x -> rmsnorm -> gate|up -> swiglu -> h
 *   QH_ROLE_DOWN       h -> down projection -> x += it
 *   QH_ROLE_HEAD       x -> final rmsnorm -> lm_head -> logits, and the argmax into *h_token
 *                      (the pick then overwrites x with that token's embedding; `layer` ignored)
 * h_token may be NULL (and is set to -1 for the other roles). */
int qh_decode_role(qh_model* m, qh_cache* c, int32_t role, int32_t layer, int32_t* h_token);

#ifdef __cplusplus
}
#endif
#endif
