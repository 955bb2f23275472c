// Host-side internals of libqwen_hip.so: the context, error reporting, and the
// launchers the C-ABI entry points call. Device code lives in *.hip files.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "qwen_hip.h"

namespace qh {

// Records a message for qh_last_error() on this thread and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define QH_HIP(expr)                                                               \
  do {                                                                             \
    hipError_t qh_e_ = (expr);                                                     \
    if (qh_e_ != hipSuccess)                                                       \
      return ::qh::fail(QH_ERR_DEVICE, "%s failed: %s", #expr, hipGetErrorString(qh_e_)); \
  } while (0)

#define QH_CHECK(cond, code, ...)                 \
  do {                                            \
    if (!(cond)) return ::qh::fail(code, __VA_ARGS__); \
  } while (0)

// Device view of one weight matrix, in the reference quantizer's layout.
// A "chunk" is 16 bytes of one row: 8 f16, 16 int8 or 32 int4 weights.
struct DMat {
  int32_t format;       // QH_FMT_F16 | QH_FMT_INT8 | QH_FMT_INT4
  const uint8_t* data;
  const float* scales;  // int8: [rows]; int4: [rows * gpr]
  const float* zeros;   // int4: [rows * gpr]
  int32_t rows, cols;
  int32_t row_bytes;    // bytes of one row
  int32_t nchunks;      // row_bytes / 16
  int32_t gpr;          // int4 groups per row
  int32_t cpg;          // int4 chunks per group (group / 32)
};

// Checks a qh_weight against what the kernels support and fills a DMat.
int make_dmat(const qh_weight* w, DMat* out);
int weights_per_chunk(int format);

// Row length of the dimension-major value cache [kv_heads][head_dim][vstride]: capacity
// rounded up to 64 positions (128 bytes), so every row, and every 64-position chunk of
// a row that split-K attention reads, starts on a cache line.
__host__ __device__ inline int value_stride(int capacity) { return (capacity + 63) & ~63; }
// Exact attention scores 256 positions per block ("span").
constexpr int kSpan = 256;
__host__ __device__ inline int attn_spans(int ctx) { return (ctx + kSpan - 1) / kSpan; }

}  // namespace qh

struct qh_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string name, arch;
  int cus = 0;
  size_t hbm_bytes = 0;
  size_t lds_per_block = 0;
  // Reusable scratch for operators that reduce across blocks (argmax, attention):
  // [0, kScratchCounterBytes) holds only counters, which every kernel leaves at
  // zero; block partials go after it; the argmax result sits in the last 64 bytes.
  void* d_scratch = nullptr;
  size_t scratch_bytes = 0;
  static constexpr size_t kScratchCounterBytes = 16384;
  int32_t* h_pinned = nullptr;  // 4-byte pinned readback slots
  // This device's copy of the no-allocation entry point's static scratch (or nullptr, and why).
  void* noalloc_scratch = nullptr;
  hipError_t noalloc_err = hipSuccess;
};

struct qh_event {
  hipEvent_t ev = nullptr;
};

// Kernel launchers (defined in the .hip files). They assume validated arguments.
namespace qh {
// x f32 [seq, cols]. When NB*cols doubles do not fit in LDS the kernel reads an f64 copy
// of x from `x64_scratch` (seq*cols doubles; NULL means the launcher allocates one).
hipError_t launch_matvec(hipStream_t s, const DMat& m, const float* x, const float* bias, float* y,
                         int seq, double* x64_scratch = nullptr);
size_t matvec_x64_bytes(const DMat& m, int seq);
// The same product summed in f32 (fast numerics), as the decode step's fused launches
// sum it in that mode. Needs cols % 4 == 0 and one staged position within 64 KiB of LDS
// (matvec_f32_supported).
hipError_t launch_matvec_f32(hipStream_t s, const DMat& m, const float* x, const float* bias, float* y,
                             int seq);
bool matvec_f32_supported(const DMat& m);
// The batched-prefill contraction on the int8 matrix cores over exact activation digits (int8 /
// int4 weights): y [M, rows] = x [M, cols] . W^T
// (+ bias). `scratch` holds `scratch_bytes` bytes; a launch that needs more returns
// hipErrorInvalidValue before any work. matmul_prefill_scratch_bytes(w, M) covers every
// launch of up to M rows.
hipError_t launch_matmul_prefill(hipStream_t s, const DMat& w, const float* x, const float* bias, float* y,
                                 int M, void* scratch, size_t scratch_bytes);
size_t matmul_prefill_scratch_bytes(const DMat& w, int M);
bool matmul_prefill_supported(const DMat& w);
// The pieces of that contraction, for callers that fuse its input and output rows.
// Row kernel: row m = sum of `splits` partial rows [splits][M][in_len] (+ bias); for
// ROW_SWIGLU silu(g)*u of interleaved gate|up pairs (in_len = 2n), else in_len = n; added
// into `resid` [M][n] when set; ROW_RMSNORM then normalizes it (f32, `gain`, `eps`); when
// `digits` is set it is written as the contraction's input: digit planes (step-major,
// M rounded up to 16-row tiles, Kp = digits_width(n) columns; digits_bytes) and row
// factors [M] (f64). n % 4 == 0, n <= 8192.
enum { ROW_PLAIN = 0, ROW_RMSNORM = 1, ROW_SWIGLU = 2 };
struct RowArgs {
  const float* in;
  int splits;
  const float* bias;
  float* resid;
  const float* gain;
  float eps;
  int M, n, Kp;
  int8_t* digits;
  double* row_factor;
};
hipError_t launch_rows(hipStream_t s, int op, const RowArgs& a);
size_t digits_bytes(int M, int K);
int digits_width(int K);
// y [M][N] = W x (+ bias) from digit planes; when the launch splits K, `part` receives the
// splits' partial rows [splits][M][N] without the bias and *splits_out says how many
// (gemm_partials_bytes(w, M) bytes cover every M up to the argument).
hipError_t launch_gemm_digits(hipStream_t s, const DMat& w, const int8_t* digits, const double* row_factor, int M,
                              const float* bias, float* y, float* part, size_t part_bytes, int* splits_out);
size_t gemm_partials_bytes(const DMat& w, int M);
hipError_t launch_matvec_xh_list(hipStream_t s, const DMat& m, int count, size_t data_stride,
                                 size_t scale_stride, const uint16_t* x, size_t x_stride, float* y);
// f32: the fast numerics' f32 rmsnorm (needs cols % 4 == 0, cols <= 8192 and 16-byte
// aligned rows); else the CPU path's f64 evaluation.
hipError_t launch_rmsnorm(hipStream_t s, const float* x, const float* gain, float* y, int rows,
                          int cols, double eps, bool f32 = false);
hipError_t launch_rope(hipStream_t s, float* v, const float* cos_t, const float* sin_t, int rows,
                       int heads, int head_dim, int base_pos);
// Keys [kv_heads][capacity][head_dim]; values dimension-major [kv_heads][head_dim][vstride],
// vstride = value_stride(capacity).
hipError_t launch_kv_append(hipStream_t s, const float* k, const float* v, uint16_t* kc,
                            uint16_t* vt, int capacity, int kv_heads, int head_dim, int past,
                            int seq);
// Exact-order attention. `scores` holds attention_exact_floats(seq, heads, past) floats
// (scores, then per-span maxima) and `counters` seq*heads ints, zero before the launch and
// left zero after it.
hipError_t launch_attention_exact(hipStream_t s, const float* q, const uint16_t* kc,
                                  const uint16_t* vt, int capacity, float* out, int seq, int past,
                                  int heads, int kv_heads, float* scores, int* counters);
size_t attention_exact_floats(int seq, int heads, int past);
// Split-K attention (the decode step's GQA-group slots, then their merge). `partials` holds
// attention_partials_floats(seq, heads, capacity) floats (no initial contents needed).
hipError_t launch_attention_splitk(hipStream_t s, const float* q, const uint16_t* kc,
                                   const uint16_t* vt, int capacity, float* out, int seq, int past,
                                   int heads, int kv_heads, float* partials);
size_t attention_partials_floats(int seq, int heads, int capacity);
// Flash attention on the matrix cores (f16 MFMA, q and p split in two f16 terms).
hipError_t launch_attention_mfma(hipStream_t s, const float* q, const uint16_t* kc, const uint16_t* vt,
                                 int capacity, float* out, int seq, int past, int heads, int kv_heads);
// One query (position past) against `count` same-shape caches: key cache i at kc + i*list_k,
// value cache i at vt + i*list_v (elements); out [count][heads*64]; `partials` holds
// attention_list_partials_floats(count, heads, kv_heads, past + 1) floats.
hipError_t launch_attention_splitk_list(hipStream_t s, const float* q, const uint16_t* kc, const uint16_t* vt,
                                        size_t list_k, size_t list_v, int count, int capacity, float* out,
                                        int past, int heads, int kv_heads, float* partials);
size_t attention_list_partials_floats(int count, int heads, int kv_heads, int ctx);
// The list operator's launch shape for a query at position ctx-1 over `count` caches: slots
// per (cache, kv head) and waves per slot.
void attention_list_plan(int ctx, int count, int kv_heads, int* slots, int* waves);
// f64 rope tables for `positions` rows of head_dim/2 angles (src/core/ops.js:99-136).
void rope_tables_f64(int head_dim, double theta, int positions, double* cos_t, double* sin_t);
hipError_t launch_swiglu(hipStream_t s, float* gate, const float* up, int n);
// Measurement: `launches` launches captured as one graph and replayed (kind 0: empty; 1: each
// reads the 896-float vector the previous one wrote, in buf [2][4096]; 2: the same launch reading
// nothing), and a streaming read of `bytes` (sink: 4096 words).
hipError_t probe_launch_floor(hipStream_t s, int kind, int blocks, int launches, float* buf, float* us_per_launch);
hipError_t read_ceiling(hipStream_t s, const void* p, size_t bytes, int reps, uint32_t* sink, float* ms_per_read);
hipError_t launch_add(hipStream_t s, float* x, const float* delta, int n);
// dst[0, bytes) = src[0, bytes): 16-byte vector copies when both are 16-byte aligned,
// bytes otherwise.
hipError_t launch_copy(hipStream_t s, void* dst, const void* src, size_t bytes);
// [rows, cols] checkpoint values (bf16 bits when `bf16`, else f32) converted to `format`:
// f32, f16, int8 (+ a scale per row) or int4 (+ a scale and zero per group; `group` even,
// dividing cols), as the host quantizer writes them.
hipError_t launch_convert(hipStream_t s, bool bf16, const void* src, int rows, int cols, int format,
                          int group, void* data, float* scales, float* zeros);
// Argmax into d_out[0]; `partials` holds argmax_partials_bytes(n) bytes; *counter is zero
// before the launch and left zero after it.
hipError_t launch_argmax(hipStream_t s, const float* v, int n, int* counter, void* partials,
                         int32_t* d_out);
size_t argmax_partials_bytes(int n);
// out[0] = -log softmax(logits[0..vocab))[*target] in f64 (the reference perplexity's expression).
hipError_t launch_nll(hipStream_t s, const float* logits, int vocab, const int32_t* target, double* out);
}  // namespace qh
