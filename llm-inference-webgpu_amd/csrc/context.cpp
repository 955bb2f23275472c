// Context, memory, events and the standalone operator entry points of the C ABI.
// Every entry point validates its arguments on the host before anything is
// launched, so an unsupported shape is an error code, never a device fault.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "qh_internal.h"

namespace {

// Scratch of qh_matmul_prefill_noalloc, the entry point that allocates nothing: one array on
// every device the library runs on, held until the process ends. The row kernel writes the
// activation digit planes and row factors into it and the contraction its split partials; each
// launch writes before it reads, so nothing in it has to start at zero. 24 MiB covers the digit
// planes of 512 rows of up to 8192 columns (12 MiB) plus the split partials, which stay within
// one 64 x 128 f32 tile per CU (256 x 32 KiB = 8 MiB) whatever the shape.
constexpr size_t kNoAllocScratchBytes = size_t(24) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// The array's device address per device. On the host, `scratch` only names the symbol; kernels
// and copies get the address hipGetSymbolAddress returns with that device current.
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kMaxDevices] = {};
hipError_t g_noalloc_err[kMaxDevices] = {};

// With `device` current: the address of its copy of `scratch` (resolved once per device), or
// nullptr and the lookup's error.
void* noalloc_scratch(int device, hipError_t* err) {
  if (device < 0 || device >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (!g_noalloc_ptr[device] && g_noalloc_err[device] == hipSuccess) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e == hipSuccess && ptr) g_noalloc_ptr[device] = ptr;
    else g_noalloc_err[device] = e != hipSuccess ? e : hipErrorInvalidSymbol;
  }
  *err = g_noalloc_err[device];
  return g_noalloc_ptr[device];
}

}  // namespace

namespace qh {

static thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

void clear_error() { g_error.clear(); }

int weights_per_chunk(int format) {
  switch (format) {
    case QH_FMT_F16: return 8;
    case QH_FMT_INT8: return 16;
    case QH_FMT_INT4: return 32;
    default: return 0;
  }
}

int make_dmat(const qh_weight* w, DMat* out) {
  QH_CHECK(w, QH_ERR_INVALID, "weight descriptor is NULL");
  const int per = weights_per_chunk(w->format);
  QH_CHECK(per > 0, QH_ERR_INVALID, "weight format %d is not a matrix format", w->format);
  QH_CHECK(w->rows > 0 && w->cols > 0, QH_ERR_INVALID, "weight shape [%d, %d] is empty", w->rows,
           w->cols);
  QH_CHECK(w->cols % per == 0, QH_ERR_INVALID,
           "cols %d must be a multiple of %d for this format (16-byte row chunks)", w->cols, per);
  QH_CHECK(w->d_data, QH_ERR_INVALID, "weight data is NULL");
  QH_CHECK(((uintptr_t)w->d_data & 15) == 0, QH_ERR_INVALID, "weight data must be 16-byte aligned");
  DMat m{};
  m.format = w->format;
  m.data = static_cast<const uint8_t*>(w->d_data);
  m.rows = w->rows;
  m.cols = w->cols;
  m.row_bytes = w->format == QH_FMT_F16 ? w->cols * 2 : w->format == QH_FMT_INT8 ? w->cols : w->cols / 2;
  m.nchunks = m.row_bytes / 16;
  if (w->format == QH_FMT_INT8) {
    QH_CHECK(w->d_scales, QH_ERR_INVALID, "int8 weight needs per-row scales");
    m.scales = w->d_scales;
  }
  if (w->format == QH_FMT_INT4) {
    QH_CHECK(w->group >= 32 && w->group % 32 == 0 && w->cols % w->group == 0, QH_ERR_INVALID,
             "int4 group %d must be a multiple of 32 dividing cols %d", w->group, w->cols);
    QH_CHECK(w->d_scales && w->d_zeros, QH_ERR_INVALID, "int4 weight needs scales and zeros");
    m.scales = w->d_scales;
    m.zeros = w->d_zeros;
    m.gpr = w->cols / w->group;
    m.cpg = w->group / 32;
  }
  *out = m;
  return QH_OK;
}

}  // namespace qh

using qh::fail;

extern "C" {

const char* qh_last_error(void) { return qh::g_error.c_str(); }
int qh_abi_version(void) { return QH_ABI_VERSION; }

int qh_device_count(int* count) {
  QH_CHECK(count, QH_ERR_INVALID, "count is NULL");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) n = 0;
  *count = n;
  return QH_OK;
}

int qh_open(int device, qh_ctx** out) {
  QH_CHECK(out, QH_ERR_INVALID, "out is NULL");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    return fail(QH_ERR_DEVICE, "no HIP device is available (this library has no CPU fallback)");
  }
  QH_CHECK(device >= 0 && device < n, QH_ERR_INVALID, "device %d out of range (have %d)", device, n);
  QH_HIP(hipSetDevice(device));
  hipDeviceProp_t p;
  QH_HIP(hipGetDeviceProperties(&p, device));
  qh_ctx* c = new qh_ctx();
  c->device = device;
  c->name = p.name;
  c->arch = p.gcnArchName;
  c->cus = p.multiProcessorCount;
  c->hbm_bytes = p.totalGlobalMem;
  c->lds_per_block = p.sharedMemPerBlock;
  if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
    delete c;
    return fail(QH_ERR_DEVICE, "hipStreamCreate failed");
  }
  c->scratch_bytes = 1 << 20;
  if (hipMalloc(&c->d_scratch, c->scratch_bytes) != hipSuccess ||
      hipMemsetAsync(c->d_scratch, 0, c->scratch_bytes, c->stream) != hipSuccess ||
      hipStreamSynchronize(c->stream) != hipSuccess ||
      hipHostMalloc((void**)&c->h_pinned, 64, hipHostMallocDefault) != hipSuccess) {
    hipFree(c->d_scratch);
    hipStreamDestroy(c->stream);
    delete c;
    return fail(QH_ERR_NOMEM, "context scratch allocation failed");
  }
  // The no-allocation entry point's scratch, resolved once per device at set-up; a failed
  // lookup is reported by that entry point, not here.
  c->noalloc_scratch = noalloc_scratch(device, &c->noalloc_err);
  *out = c;
  return QH_OK;
}

int qh_close(qh_ctx* ctx) {
  if (!ctx) return QH_OK;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->stream);
  hipFree(ctx->d_scratch);
  hipHostFree(ctx->h_pinned);
  hipStreamDestroy(ctx->stream);
  delete ctx;
  return QH_OK;
}

int qh_describe(qh_ctx* ctx, char* buf, size_t len) {
  QH_CHECK(ctx && buf && len > 0, QH_ERR_INVALID, "describe needs a context and a buffer");
  snprintf(buf, len,
           "{\"name\": \"%s\", \"arch\": \"%s\", \"compute_units\": %d, \"hbm_bytes\": %zu, "
           "\"lds_per_block\": %zu, \"abi\": %d}",
           ctx->name.c_str(), ctx->arch.c_str(), ctx->cus, ctx->hbm_bytes, ctx->lds_per_block,
           QH_ABI_VERSION);
  return QH_OK;
}

int qh_sync(qh_ctx* ctx) {
  QH_CHECK(ctx, QH_ERR_INVALID, "context is NULL");
  QH_HIP(hipStreamSynchronize(ctx->stream));
  return QH_OK;
}

void* qh_stream(qh_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int qh_alloc(qh_ctx* ctx, size_t bytes, void** d_out) {
  QH_CHECK(ctx && d_out, QH_ERR_INVALID, "alloc needs a context and an output pointer");
  *d_out = nullptr;
  QH_HIP(hipSetDevice(ctx->device));
  if (hipMalloc(d_out, bytes ? bytes : 4) != hipSuccess) {
    return fail(QH_ERR_NOMEM, "hipMalloc of %zu bytes failed", bytes);
  }
  return QH_OK;
}

int qh_free(qh_ctx* ctx, void* d_ptr) {
  QH_CHECK(ctx, QH_ERR_INVALID, "context is NULL");
  if (!d_ptr) return QH_OK;
  QH_HIP(hipStreamSynchronize(ctx->stream));
  QH_HIP(hipFree(d_ptr));
  return QH_OK;
}

int qh_upload(qh_ctx* ctx, void* d_dst, const void* h_src, size_t bytes) {
  QH_CHECK(ctx && d_dst && (h_src || !bytes), QH_ERR_INVALID, "upload needs buffers");
  QH_HIP(hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice, ctx->stream));
  QH_HIP(hipStreamSynchronize(ctx->stream));
  return QH_OK;
}

int qh_download(qh_ctx* ctx, void* h_dst, const void* d_src, size_t bytes) {
  QH_CHECK(ctx && d_src && (h_dst || !bytes), QH_ERR_INVALID, "download needs buffers");
  QH_HIP(hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  QH_HIP(hipStreamSynchronize(ctx->stream));
  return QH_OK;
}

int qh_memset(qh_ctx* ctx, void* d_dst, int value, size_t bytes) {
  QH_CHECK(ctx && d_dst, QH_ERR_INVALID, "memset needs a buffer");
  QH_HIP(hipMemsetAsync(d_dst, value, bytes, ctx->stream));
  return QH_OK;
}

int qh_copy(qh_ctx* ctx, void* d_dst, const void* d_src, size_t bytes) {
  QH_CHECK(ctx && ((d_dst && d_src) || !bytes), QH_ERR_INVALID, "copy needs buffers");
  const uintptr_t lo = (uintptr_t)d_dst, hi = (uintptr_t)d_src;
  QH_CHECK(lo + bytes <= hi || hi + bytes <= lo, QH_ERR_INVALID, "copy ranges overlap");
  if (!bytes) return QH_OK;
  QH_HIP(qh::launch_copy(ctx->stream, d_dst, d_src, bytes));
  return QH_OK;
}

int qh_quantize(qh_ctx* ctx, int32_t src_format, const void* d_src, int32_t rows, int32_t cols,
                int32_t format, int32_t group, void* d_data, float* d_scales, float* d_zeros) {
  QH_CHECK(ctx && d_src && d_data && rows >= 1 && cols >= 1, QH_ERR_INVALID,
           "quantize needs a context, a non-empty source and an output");
  QH_CHECK(src_format == QH_FMT_BF16 || src_format == QH_FMT_F32, QH_ERR_INVALID,
           "quantize reads bf16 or f32 values (src_format %d)", src_format);
  QH_CHECK(format == QH_FMT_F32 || format == QH_FMT_F16 || format == QH_FMT_INT8 || format == QH_FMT_INT4,
           QH_ERR_INVALID, "quantize writes f32, f16, int8 or int4 (format %d)", format);
  QH_CHECK(format != QH_FMT_INT8 || d_scales, QH_ERR_INVALID, "int8 needs a scale per row");
  if (format == QH_FMT_INT4) {
    QH_CHECK(d_scales && d_zeros, QH_ERR_INVALID, "int4 needs a scale and a zero point per group");
    QH_CHECK(group >= 2, QH_ERR_RANGE, "groupSize must be an integer of at least 2, got %d", group);
    QH_CHECK(cols % group == 0, QH_ERR_RANGE, "groupSize %d does not divide %d columns", group, cols);
    QH_CHECK(group % 2 == 0, QH_ERR_INVALID, "groupSize %d must be even to pack a byte within a group", group);
  }
  QH_HIP(qh::launch_convert(ctx->stream, src_format == QH_FMT_BF16, d_src, rows, cols, format, group, d_data,
                            d_scales, d_zeros));
  return QH_OK;
}

int qh_event_create(qh_ctx* ctx, qh_event** out) {
  QH_CHECK(ctx && out, QH_ERR_INVALID, "event_create needs a context");
  qh_event* e = new qh_event();
  if (hipEventCreate(&e->ev) != hipSuccess) {
    delete e;
    return fail(QH_ERR_DEVICE, "hipEventCreate failed");
  }
  *out = e;
  return QH_OK;
}

int qh_event_record(qh_ctx* ctx, qh_event* ev) {
  QH_CHECK(ctx && ev, QH_ERR_INVALID, "event_record needs a context and an event");
  QH_HIP(hipEventRecord(ev->ev, ctx->stream));
  return QH_OK;
}

int qh_event_elapsed_ms(qh_event* start, qh_event* stop, float* ms) {
  QH_CHECK(start && stop && ms, QH_ERR_INVALID, "elapsed needs two events");
  QH_HIP(hipEventSynchronize(stop->ev));
  QH_HIP(hipEventElapsedTime(ms, start->ev, stop->ev));
  return QH_OK;
}

int qh_event_destroy(qh_event* ev) {
  if (!ev) return QH_OK;
  hipEventDestroy(ev->ev);
  delete ev;
  return QH_OK;
}

// --------------------------------------------------------------- operators --

int qh_matvec(qh_ctx* ctx, const qh_weight* w, const float* d_x, const float* d_bias, float* d_y,
              int32_t seq) {
  QH_CHECK(ctx, QH_ERR_INVALID, "context is NULL");
  qh::DMat m;
  int rc = qh::make_dmat(w, &m);
  if (rc) return rc;
  QH_CHECK(d_x && d_y, QH_ERR_INVALID, "matvec needs x and y");
  QH_CHECK(seq >= 1, QH_ERR_INVALID, "seq %d must be at least 1", seq);
  QH_HIP(qh::launch_matvec(ctx->stream, m, d_x, d_bias, d_y, seq));
  return QH_OK;
}

}  // extern "C"

// The argument checks both forms of the MFMA prefill share.
static int check_matmul_prefill(qh_ctx* ctx, const qh_weight* w, const float* d_x, const float* d_y, int32_t M,
                                qh::DMat* m) {
  QH_CHECK(ctx, QH_ERR_INVALID, "context is NULL");
  int rc = qh::make_dmat(w, m);
  if (rc) return rc;
  QH_CHECK(m->format == QH_FMT_INT8 || m->format == QH_FMT_INT4, QH_ERR_INVALID,
           "the MFMA prefill takes int8 or int4 weights (format %d given)", m->format);
  QH_CHECK(m->cols % 32 == 0, QH_ERR_INVALID, "cols %d must be a multiple of 32", m->cols);
  QH_CHECK(qh::matmul_prefill_supported(*m), QH_ERR_INVALID,
           "the MFMA prefill takes int8, or int4 in groups of a multiple of 64 columns (group %d, cols %d)",
           w->group, m->cols);
  QH_CHECK(m->cols <= 8192, QH_ERR_INVALID, "the MFMA prefill stages rows of at most 8192 columns (cols %d)",
           m->cols);
  QH_CHECK(d_x && d_y, QH_ERR_INVALID, "matmul needs x and y");
  QH_CHECK(((uintptr_t)d_x & 15) == 0, QH_ERR_INVALID, "x must be 16-byte aligned");
  QH_CHECK(M >= 1, QH_ERR_INVALID, "M %d must be at least 1", M);
  return QH_OK;
}

extern "C" {

int qh_matmul_prefill(qh_ctx* ctx, const qh_weight* w, const float* d_x, const float* d_bias,
                      float* d_y, int32_t M) {
  qh::DMat m;
  int rc = check_matmul_prefill(ctx, w, d_x, d_y, M, &m);
  if (rc) return rc;
  void* tmp = nullptr;
  const size_t scratch = qh::matmul_prefill_scratch_bytes(m, M);
  QH_HIP(hipMallocAsync(&tmp, scratch, ctx->stream));
  hipError_t e = qh::launch_matmul_prefill(ctx->stream, m, d_x, d_bias, d_y, M, tmp, scratch);
  QH_HIP(hipFreeAsync(tmp, ctx->stream));
  QH_HIP(e);
  return QH_OK;
}

int qh_matmul_prefill_noalloc(qh_ctx* ctx, const qh_weight* w, const float* d_x, const float* d_bias,
                              float* d_y, int32_t M) {
  qh::DMat m;
  int rc = check_matmul_prefill(ctx, w, d_x, d_y, M, &m);
  if (rc) return rc;
  // The digit planes alone grow with M: past the scratch they reject a large M before the
  // partials' per-M scan below runs.
  QH_CHECK(qh::digits_bytes(M, m.cols) <= kNoAllocScratchBytes &&
               qh::matmul_prefill_scratch_bytes(m, M) <= kNoAllocScratchBytes,
           QH_ERR_RANGE,
           "the no-allocation MFMA prefill has %zu bytes of scratch; M %d x cols %d needs more "
           "(every M <= 512 with cols <= 8192 fits)",
           kNoAllocScratchBytes, M, m.cols);
  QH_CHECK(ctx->noalloc_scratch, QH_ERR_DEVICE, "the no-allocation scratch of device %d is unavailable: %s",
           ctx->device, hipGetErrorString(ctx->noalloc_err));
  QH_HIP(qh::launch_matmul_prefill(ctx->stream, m, d_x, d_bias, d_y, M, ctx->noalloc_scratch, kNoAllocScratchBytes));
  return QH_OK;
}

int qh_matvec_xh(qh_ctx* ctx, const qh_weight* w, const uint16_t* d_x, float* d_y) {
  return qh_matvec_xh_list(ctx, w, 1, 0, 0, d_x, 0, d_y);
}

int qh_matvec_xh_list(qh_ctx* ctx, const qh_weight* w, int32_t count, size_t data_stride,
                      size_t scale_stride, const uint16_t* d_x, size_t x_stride, float* d_y) {
  QH_CHECK(ctx, QH_ERR_INVALID, "context is NULL");
  qh::DMat m;
  int rc = qh::make_dmat(w, &m);
  if (rc) return rc;
  QH_CHECK(m.format == QH_FMT_INT8, QH_ERR_INVALID,
           "the f16-activation matvec takes int8 weights (format %d given)", m.format);
  QH_CHECK(count >= 1, QH_ERR_INVALID, "count %d must be at least 1", count);
  QH_CHECK(d_x && d_y, QH_ERR_INVALID, "matvec needs x and y");
  QH_CHECK(((uintptr_t)d_x & 15) == 0 && x_stride % 8 == 0, QH_ERR_INVALID,
           "x must be 16-byte aligned with a stride that is a multiple of 8 halves");
  QH_CHECK(count == 1 || (data_stride >= (size_t)m.rows * m.row_bytes && data_stride % 16 == 0 &&
                          scale_stride >= (size_t)m.rows),
           QH_ERR_INVALID, "list strides overlap the matrices or break 16-byte alignment");
  QH_HIP(qh::launch_matvec_xh_list(ctx->stream, m, count, data_stride, scale_stride, d_x, x_stride,
                                   d_y));
  return QH_OK;
}

int qh_rmsnorm(qh_ctx* ctx, const float* d_x, const float* d_gain, float* d_y, int32_t rows,
               int32_t cols, double eps) {
  QH_CHECK(ctx && d_x && d_gain && d_y, QH_ERR_INVALID, "rmsnorm needs x, gain and y");
  QH_CHECK(rows >= 1 && cols >= 1 && cols <= 8192, QH_ERR_INVALID,
           "rmsnorm shape [%d, %d] unsupported (cols up to 8192)", rows, cols);
  QH_HIP(qh::launch_rmsnorm(ctx->stream, d_x, d_gain, d_y, rows, cols, eps));
  return QH_OK;
}

int qh_rope(qh_ctx* ctx, float* d_v, const float* d_cos, const float* d_sin,
            int32_t table_positions, int32_t rows, int32_t heads, int32_t head_dim,
            int32_t base_pos) {
  QH_CHECK(ctx && d_v && d_cos && d_sin, QH_ERR_INVALID, "rope needs v and the tables");
  QH_CHECK(rows >= 1 && heads >= 1 && head_dim >= 2 && head_dim % 2 == 0 && base_pos >= 0,
           QH_ERR_INVALID, "rope shape rows=%d heads=%d head_dim=%d base=%d unsupported", rows,
           heads, head_dim, base_pos);
  QH_CHECK(base_pos + rows <= table_positions, QH_ERR_RANGE,
           "position %d exceeds the %d-entry rope table", base_pos + rows, table_positions);
  QH_HIP(qh::launch_rope(ctx->stream, d_v, d_cos, d_sin, rows, heads, head_dim, base_pos));
  return QH_OK;
}

size_t qh_value_cache_bytes(int32_t capacity, int32_t kv_heads, int32_t head_dim) {
  if (capacity < 1 || kv_heads < 1 || head_dim < 1) return 0;
  return (size_t)kv_heads * head_dim * qh::value_stride(capacity) * sizeof(uint16_t);
}

int qh_kv_append(qh_ctx* ctx, const float* d_k, const float* d_v, uint16_t* d_key_cache,
                 uint16_t* d_value_cache, int32_t capacity, int32_t kv_heads, int32_t head_dim,
                 int32_t past, int32_t seq) {
  QH_CHECK(ctx && d_k && d_v && d_key_cache && d_value_cache, QH_ERR_INVALID,
           "kv_append needs k, v and both caches");
  QH_CHECK(kv_heads >= 1 && head_dim >= 1 && seq >= 1 && past >= 0, QH_ERR_INVALID,
           "kv_append shape unsupported");
  QH_CHECK(past + seq <= capacity, QH_ERR_RANGE, "cache holds %d of %d; cannot add %d", past,
           capacity, seq);
  QH_HIP(qh::launch_kv_append(ctx->stream, d_k, d_v, d_key_cache, d_value_cache, capacity, kv_heads,
                              head_dim, past, seq));
  return QH_OK;
}

static int check_attention(qh_ctx* ctx, const float* d_q, const uint16_t* d_key_cache,
                           const uint16_t* d_value_cache, int32_t capacity, float* d_out,
                           int32_t seq, int32_t past, int32_t heads, int32_t kv_heads,
                           int32_t head_dim) {
  QH_CHECK(ctx && d_q && d_key_cache && d_value_cache && d_out, QH_ERR_INVALID,
           "attention needs q, both caches and out");
  QH_CHECK(head_dim == 64, QH_ERR_INVALID, "attention supports head_dim 64 (got %d)", head_dim);
  QH_CHECK(kv_heads >= 1 && heads >= kv_heads && heads % kv_heads == 0 && heads / kv_heads <= 8,
           QH_ERR_INVALID, "heads %d / kv_heads %d must group evenly, at most 8 per kv head", heads,
           kv_heads);
  QH_CHECK(seq >= 1 && past >= 0, QH_ERR_INVALID, "attention needs seq >= 1 and past >= 0");
  QH_CHECK(past + seq <= capacity, QH_ERR_RANGE, "attention over %d positions exceeds capacity %d",
           past + seq, capacity);
  return QH_OK;
}

int qh_attention(qh_ctx* ctx, const float* d_q, const uint16_t* d_key_cache,
                 const uint16_t* d_value_cache, int32_t capacity, float* d_out, int32_t seq,
                 int32_t past, int32_t heads, int32_t kv_heads, int32_t head_dim) {
  int rc = check_attention(ctx, d_q, d_key_cache, d_value_cache, capacity, d_out, seq, past, heads,
                           kv_heads, head_dim);
  if (rc) return rc;
  // Scores and span maxima in the context scratch's partial region, counters in its counter
  // region (after the argmax counter), when they fit; else a temporary buffer.
  const size_t floats = qh::attention_exact_floats(seq, heads, past);
  const size_t room = ctx->scratch_bytes - qh_ctx::kScratchCounterBytes - 64;
  const size_t n_counters = (size_t)seq * heads;
  if ((n_counters + 16) * sizeof(int) <= qh_ctx::kScratchCounterBytes && floats * sizeof(float) <= room) {
    float* buf = reinterpret_cast<float*>(static_cast<char*>(ctx->d_scratch) + qh_ctx::kScratchCounterBytes);
    int* counters = static_cast<int*>(ctx->d_scratch) + 16;
    QH_HIP(qh::launch_attention_exact(ctx->stream, d_q, d_key_cache, d_value_cache, capacity, d_out,
                                      seq, past, heads, kv_heads, buf, counters));
    return QH_OK;
  }
  const size_t counter_bytes = (n_counters * sizeof(int) + 255) & ~(size_t)255;
  void* tmp = nullptr;
  QH_HIP(hipMallocAsync(&tmp, counter_bytes + floats * sizeof(float), ctx->stream));
  QH_HIP(hipMemsetAsync(tmp, 0, counter_bytes, ctx->stream));
  hipError_t e = qh::launch_attention_exact(
      ctx->stream, d_q, d_key_cache, d_value_cache, capacity, d_out, seq, past, heads, kv_heads,
      reinterpret_cast<float*>(static_cast<char*>(tmp) + counter_bytes), static_cast<int*>(tmp));
  QH_HIP(hipFreeAsync(tmp, ctx->stream));
  QH_HIP(e);
  return QH_OK;
}

int qh_attention_mfma(qh_ctx* ctx, const float* d_q, const uint16_t* d_key_cache,
                      const uint16_t* d_value_cache, int32_t capacity, float* d_out, int32_t seq,
                      int32_t past, int32_t heads, int32_t kv_heads, int32_t head_dim) {
  int rc = check_attention(ctx, d_q, d_key_cache, d_value_cache, capacity, d_out, seq, past, heads,
                           kv_heads, head_dim);
  if (rc) return rc;
  QH_HIP(qh::launch_attention_mfma(ctx->stream, d_q, d_key_cache, d_value_cache, capacity, d_out, seq, past,
                                   heads, kv_heads));
  return QH_OK;
}

int qh_attention_splitk(qh_ctx* ctx, const float* d_q, const uint16_t* d_key_cache,
                        const uint16_t* d_value_cache, int32_t capacity, float* d_out, int32_t seq,
                        int32_t past, int32_t heads, int32_t kv_heads, int32_t head_dim) {
  int rc = check_attention(ctx, d_q, d_key_cache, d_value_cache, capacity, d_out, seq, past, heads,
                           kv_heads, head_dim);
  if (rc) return rc;
  const size_t bytes = qh::attention_partials_floats(seq, heads, capacity) * sizeof(float);
  // Partials in the context scratch after its counter region; larger prefill shapes get a
  // temporary buffer.
  if (bytes <= ctx->scratch_bytes - qh_ctx::kScratchCounterBytes - 64) {
    float* parts = reinterpret_cast<float*>(static_cast<char*>(ctx->d_scratch) + qh_ctx::kScratchCounterBytes);
    QH_HIP(qh::launch_attention_splitk(ctx->stream, d_q, d_key_cache, d_value_cache, capacity, d_out,
                                       seq, past, heads, kv_heads, parts));
    return QH_OK;
  }
  void* tmp = nullptr;
  QH_HIP(hipMallocAsync(&tmp, bytes, ctx->stream));
  hipError_t e = qh::launch_attention_splitk(ctx->stream, d_q, d_key_cache, d_value_cache, capacity,
                                             d_out, seq, past, heads, kv_heads, static_cast<float*>(tmp));
  QH_HIP(hipFreeAsync(tmp, ctx->stream));
  QH_HIP(e);
  return QH_OK;
}

int qh_attention_splitk_list(qh_ctx* ctx, const float* d_q, const uint16_t* d_key_cache,
                             const uint16_t* d_value_cache, size_t key_stride, size_t value_stride,
                             int32_t count, int32_t capacity, float* d_out, int32_t past, int32_t heads,
                             int32_t kv_heads, int32_t head_dim) {
  int rc = check_attention(ctx, d_q, d_key_cache, d_value_cache, capacity, d_out, 1, past, heads, kv_heads,
                           head_dim);
  if (rc) return rc;
  QH_CHECK(count >= 1 && count <= 65535, QH_ERR_INVALID, "count %d must be in 1..65535", count);
  const size_t kel = (size_t)kv_heads * capacity * 64;
  const size_t vel = qh_value_cache_bytes(capacity, kv_heads, 64) / 2;
  QH_CHECK(count == 1 || (key_stride >= kel && value_stride >= vel && key_stride % 8 == 0 && value_stride % 8 == 0),
           QH_ERR_INVALID, "cache strides overlap the caches or break 16-byte alignment");
  void* tmp = nullptr;
  QH_HIP(hipMallocAsync(&tmp, qh::attention_list_partials_floats(count, heads, kv_heads, past + 1) * sizeof(float), ctx->stream));
  hipError_t e = qh::launch_attention_splitk_list(ctx->stream, d_q, d_key_cache, d_value_cache, key_stride,
                                                  value_stride, count, capacity, d_out, past, heads, kv_heads,
                                                  static_cast<float*>(tmp));
  QH_HIP(hipFreeAsync(tmp, ctx->stream));
  QH_HIP(e);
  return QH_OK;
}

int qh_attention_list_plan(int32_t context, int32_t count, int32_t kv_heads, int32_t* h_slots,
                           int32_t* h_waves) {
  QH_CHECK(context >= 1 && count >= 1 && kv_heads >= 1 && h_slots && h_waves, QH_ERR_INVALID,
           "list plan needs context, count and kv_heads >= 1 and two outputs");
  int slots = 0, waves = 0;
  qh::attention_list_plan(context, count, kv_heads, &slots, &waves);
  *h_slots = slots;
  *h_waves = waves;
  return QH_OK;
}

int qh_swiglu(qh_ctx* ctx, float* d_gate, const float* d_up, int32_t n) {
  QH_CHECK(ctx && d_gate && d_up && n >= 1, QH_ERR_INVALID, "swiglu needs gate, up and n >= 1");
  QH_HIP(qh::launch_swiglu(ctx->stream, d_gate, d_up, n));
  return QH_OK;
}

int qh_add(qh_ctx* ctx, float* d_x, const float* d_delta, int32_t n) {
  QH_CHECK(ctx && d_x && d_delta && n >= 1, QH_ERR_INVALID, "add needs x, delta and n >= 1");
  QH_HIP(qh::launch_add(ctx->stream, d_x, d_delta, n));
  return QH_OK;
}

int qh_argmax(qh_ctx* ctx, const float* d_v, int32_t n, int32_t* h_index) {
  QH_CHECK(ctx && d_v && h_index && n >= 1, QH_ERR_INVALID, "argmax needs v, n >= 1 and an output");
  QH_CHECK(qh::argmax_partials_bytes(n) + qh_ctx::kScratchCounterBytes + 64 <= ctx->scratch_bytes,
           QH_ERR_INVALID, "argmax over %d values exceeds the context scratch", n);
  char* base = static_cast<char*>(ctx->d_scratch);
  int32_t* d_out = reinterpret_cast<int32_t*>(base + ctx->scratch_bytes - 64);
  QH_HIP(qh::launch_argmax(ctx->stream, d_v, n, reinterpret_cast<int*>(base),
                           base + qh_ctx::kScratchCounterBytes, d_out));
  QH_HIP(hipMemcpyAsync(ctx->h_pinned, d_out, 4, hipMemcpyDeviceToHost, ctx->stream));
  QH_HIP(hipStreamSynchronize(ctx->stream));
  *h_index = ctx->h_pinned[0];
  return QH_OK;
}

}  // extern "C"

extern "C" {

int qh_probe_launch_floor(qh_ctx* ctx, int32_t kind, int32_t blocks, int32_t launches, float* us_per_launch) {
  QH_CHECK(ctx && us_per_launch, QH_ERR_INVALID, "probe_launch_floor needs a context and an output");
  QH_CHECK(kind >= 0 && kind <= 2 && blocks >= 1 && blocks <= 65536 && launches >= 1 && launches <= 4096,
           QH_ERR_INVALID, "probe kind 0..2, blocks 1..65536 and launches 1..4096");
  QH_HIP(hipSetDevice(ctx->device));
  float* buf = nullptr;
  QH_HIP(hipMalloc((void**)&buf, 2 * 4096 * sizeof(float)));
  hipError_t e = hipMemsetAsync(buf, 0, 2 * 4096 * sizeof(float), ctx->stream);
  if (e == hipSuccess) e = qh::probe_launch_floor(ctx->stream, kind, blocks, launches, buf, us_per_launch);
  hipStreamSynchronize(ctx->stream);
  hipFree(buf);
  QH_HIP(e);
  return QH_OK;
}

int qh_read_ceiling(qh_ctx* ctx, size_t bytes, int32_t reps, float* gbps) {
  QH_CHECK(ctx && gbps, QH_ERR_INVALID, "read_ceiling needs a context and an output");
  QH_CHECK(bytes >= ((size_t)1 << 20) && bytes <= ((size_t)64 << 30) && bytes % 64 == 0 && reps >= 1,
           QH_ERR_INVALID, "read_ceiling reads 1 MiB .. 64 GiB (a multiple of 64 bytes), reps >= 1");
  QH_HIP(hipSetDevice(ctx->device));
  void* p = nullptr;
  uint32_t* sink = nullptr;
  QH_HIP(hipMalloc(&p, bytes));
  hipError_t e = hipMalloc((void**)&sink, 4096 * sizeof(uint32_t));
  if (e == hipSuccess) e = hipMemsetAsync(p, 0x5a, bytes, ctx->stream);
  float ms = 0.f;
  if (e == hipSuccess) e = qh::read_ceiling(ctx->stream, p, bytes, reps, sink, &ms);
  hipStreamSynchronize(ctx->stream);
  hipFree(p);
  if (sink) hipFree(sink);
  QH_HIP(e);
  *gbps = (float)(bytes / (ms * 1e-3) / 1e9);
  return QH_OK;
}

}  // extern "C"
