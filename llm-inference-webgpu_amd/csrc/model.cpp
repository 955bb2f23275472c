// GpuModel / GpuKVCache (src/gpu/model.js:69-403) as C-ABI objects.
//
// Loading: tensors arrive by checkpoint name (src/core/config.js:88-119) in the
// formats the reference quantizer produces, are uploaded as-is, and finalize()
// rearranges them into the fused device layouts the decode kernels read: q|k|v
// stacked into one matrix, gate and up rows interleaved. Rows are only moved,
// never requantized, so every code and scale is the quantizer's own.
//
// Stepping: forward() runs one decode position at a time through the same
// launches as decode() (so a prefill and a decode of the same tokens produce
// the same bits, the reference's prefill == decode property, README.md:256-272);
// decode() replays a hipGraph of one step whose kernels read the position and
// the token from device memory, so nothing is re-encoded per token.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <functional>
#include <vector>

#include "model_dev.h"
#include "qh_internal.h"

using qh::fail;

namespace {

struct Staged {
  int format = -1;
  int rows = 0, cols = 0, group = 0;
  void* data = nullptr;
  float* scales = nullptr;
  float* zeros = nullptr;
};

const char* const kLayerNames[] = {
    "input_layernorm.weight", "self_attn.q_proj.weight", "self_attn.q_proj.bias",
    "self_attn.k_proj.weight", "self_attn.k_proj.bias",  "self_attn.v_proj.weight",
    "self_attn.v_proj.bias",   "self_attn.o_proj.weight", "post_attention_layernorm.weight",
    "mlp.gate_proj.weight",    "mlp.up_proj.weight",      "mlp.down_proj.weight"};

bool is_matrix_format(int f) { return f == QH_FMT_F16 || f == QH_FMT_INT8 || f == QH_FMT_INT4; }

size_t data_bytes(int format, size_t rows, size_t cols) {
  switch (format) {
    case QH_FMT_F32: return rows * cols * 4;
    case QH_FMT_F16:
    case QH_FMT_BF16: return rows * cols * 2;
    case QH_FMT_INT8: return rows * cols;
    case QH_FMT_INT4: return rows * cols / 2;
    default: return 0;
  }
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu, mant = h & 0x3ffu, out;
  if (exp == 0x1f) {
    out = sign | 0x7f800000u | (mant << 13);
  } else if (exp == 0) {
    if (mant == 0) {
      out = sign;
    } else {
      int e = -1;
      do { mant <<= 1; e++; } while ((mant & 0x400u) == 0);
      out = sign | ((uint32_t)(127 - 15 - e) << 23) | ((mant & 0x3ffu) << 13);
    }
  } else {
    out = sign | ((exp - 15 + 127) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &out, 4);
  return f;
}

}  // namespace

struct qh_model {
  qh_ctx* ctx = nullptr;
  qh_config cfg{};
  std::map<std::string, Staged> staged;
  bool finalized = false;
  std::vector<void*> allocs;
  std::vector<qh::LayerDev> layers;
  qh::ModelDev dev{};
  size_t bytes = 0;
  int live_caches = 0;
  int caches_made = 0;
  int numerics = QH_NUMERICS_FAST;
  int matmul = QH_MATMUL_BATCHED;

  int alloc(size_t n, void** p) {
    if (hipMalloc(p, n ? n : 4) != hipSuccess) return fail(QH_ERR_NOMEM, "hipMalloc of %zu bytes failed", n);
    allocs.push_back(*p);
    bytes += n;
    return QH_OK;
  }
  // Moves a staged buffer into the model's permanent set.
  void keep(void* p) {
    if (p) allocs.push_back(p);
  }
};

// One batched-prefill chunk's launches (embedding gather, every layer) captured as a graph,
// keyed by what the launches bake in: the first position, the chunk length, the matmul path
// and numerics, and whether the rows are gathered from token ids.
struct PrefillGraph {
  int past, n, matmul, numerics, tokens;
  int uses;            // times the shape was run; it is captured on its second use
  uint64_t last;       // least-recently-used stamp
  hipGraph_t graph;
  hipGraphExec_t exec;
};
constexpr int kPrefillGraphs = 8;  // shapes kept per cache

struct qh_cache {
  qh_model* m = nullptr;
  qh::CacheDev dev{};
  int length = 0;
  std::vector<void*> allocs;
  hipGraph_t graph_first = nullptr;    // a decode call's first step: carried input, pick deferred
  hipGraphExec_t exec_first = nullptr;
  hipGraph_t graph = nullptr;          // one later step: the previous pick in its first launch
  hipGraphExec_t exec = nullptr;
  hipGraph_t graph_run = nullptr;      // kGraphRun such steps back to back
  hipGraphExec_t exec_run = nullptr;
  bool use_graph = true;  // false: decode enqueues every kernel directly
  bool busy = false;
  int pending_start = 0, pending_steps = 0;
  float* d_hidden = nullptr;
  size_t hidden_cap = 0;
  int32_t* h_pinned = nullptr;  // [0..1] state staging, [2] argmax readback
  // Prefill chunks seen, and graphs of those run twice (all valid while pw_mem is).
  std::vector<PrefillGraph> pgraphs;
  uint64_t pclock = 0;
  // Batched-prefill workspace (allocated at the first batched forward).
  qh::PrefillDev pw{};
  qh::PrefillBytes pw_bytes{};
  void* pw_mem = nullptr;
  int pw_matmul = -1;  // the matmul mode the workspace was last checked for

  int alloc(size_t n, void** p) {
    if (hipMalloc(p, n ? n : 4) != hipSuccess) return fail(QH_ERR_NOMEM, "hipMalloc of %zu bytes failed", n);
    allocs.push_back(*p);
    return QH_OK;
  }
};

// Destroys the cache's prefill graphs (the caller has synchronized the stream).
static void drop_prefill_graphs(qh_cache* c) {
  for (PrefillGraph& g : c->pgraphs) {
    if (g.exec) hipGraphExecDestroy(g.exec);
    if (g.graph) hipGraphDestroy(g.graph);
  }
  c->pgraphs.clear();
}

static void free_staged(Staged& s) {
  hipFree(s.data);
  hipFree(s.scales);
  hipFree(s.zeros);
  s = Staged{};
}

extern "C" {

int qh_model_create(qh_ctx* ctx, const qh_config* cfg, qh_model** out) {
  QH_CHECK(ctx && cfg && out, QH_ERR_INVALID, "model_create needs a context, a config and an output");
  *out = nullptr;
  const qh_config& c = *cfg;
  QH_CHECK(c.hidden > 0 && c.intermediate > 0 && c.layers > 0 && c.heads > 0 && c.kv_heads > 0 &&
               c.vocab > 0 && c.max_positions > 0,
           QH_ERR_INVALID, "config dimensions must be positive");
  QH_CHECK(c.head_dim == 64 && c.hidden == c.heads * c.head_dim, QH_ERR_INVALID,
           "the kernels implement head_dim 64 with hidden = heads * head_dim (got %d, %d x %d)",
           c.hidden, c.heads, c.head_dim);
  QH_CHECK(c.heads % c.kv_heads == 0 && c.heads / c.kv_heads <= 8, QH_ERR_INVALID,
           "num_attention_heads %d is not divisible by num_key_value_heads %d (or groups > 8)",
           c.heads, c.kv_heads);
  // The decode kernels stage a whole activation vector in LDS as f64 (8192 values) and keep a
  // lane's share of a row in registers (at most 16 chunks of a 64-lane team).
  QH_CHECK(c.hidden % 32 == 0 && c.intermediate % 32 == 0 && c.hidden <= 8192 &&
               c.intermediate <= 8192,
           QH_ERR_INVALID, "hidden and intermediate must be multiples of 32 up to 8192");
  qh_model* m = new qh_model();
  m->ctx = ctx;
  m->cfg = c;
  *out = m;
  return QH_OK;
}

// The shape and formats a checkpoint name allows (src/core/config.js:88-119); a vector comes
// back as [n, 1]. A matrix must also fit the kernels' layout rules (make_dmat).
static int check_tensor(qh_model* m, const char* name, int32_t format, int32_t* rows_io, int32_t* cols_io,
                        int32_t group) {
  QH_CHECK(!m->finalized, QH_ERR_STATE, "model is finalized; tensors are immutable");
  int32_t& rows = *rows_io;
  int32_t& cols = *cols_io;
  const qh_config& c = m->cfg;
  const int kv_dim = c.kv_heads * c.head_dim;
  const std::string n = name;
  // Expected shape and whether a matrix format is allowed.
  int er = 0, ec = 0;
  bool matrix = false, bf16 = false;
  if (n == "model.embed_tokens.weight") {
    er = c.vocab, ec = c.hidden, bf16 = true;
  } else if (n == "lm_head.weight") {
    er = c.vocab, ec = c.hidden, matrix = true;
  } else if (n == "model.norm.weight") {
    er = c.hidden, ec = 1;
  } else if (n.rfind("model.layers.", 0) == 0) {
    const char* p = name + 13;
    char* end = nullptr;
    const long L = strtol(p, &end, 10);
    QH_CHECK(end != p && *end == '.' && L >= 0 && L < c.layers, QH_ERR_INVALID,
             "unexpected tensor %s", name);
    const std::string suffix = end + 1;
    if (suffix == "input_layernorm.weight" || suffix == "post_attention_layernorm.weight") {
      er = c.hidden, ec = 1;
    } else if (suffix == "self_attn.q_proj.bias") {
      er = c.hidden, ec = 1;
    } else if (suffix == "self_attn.k_proj.bias" || suffix == "self_attn.v_proj.bias") {
      er = kv_dim, ec = 1;
    } else if (suffix == "self_attn.q_proj.weight" || suffix == "self_attn.o_proj.weight") {
      er = c.hidden, ec = c.hidden, matrix = true;
    } else if (suffix == "self_attn.k_proj.weight" || suffix == "self_attn.v_proj.weight") {
      er = kv_dim, ec = c.hidden, matrix = true;
    } else if (suffix == "mlp.gate_proj.weight" || suffix == "mlp.up_proj.weight") {
      er = c.intermediate, ec = c.hidden, matrix = true;
    } else if (suffix == "mlp.down_proj.weight") {
      er = c.hidden, ec = c.intermediate, matrix = true;
    } else {
      return fail(QH_ERR_INVALID, "unexpected tensor %s", name);
    }
  } else {
    return fail(QH_ERR_INVALID, "unexpected tensor %s", name);
  }
  const bool vector = ec == 1;
  if (vector) {
    QH_CHECK(format == QH_FMT_F32 && (size_t)rows * cols == (size_t)er, QH_ERR_INVALID,
             "%s: expected f32 [%d], got format %d [%d, %d]", name, er, format, rows, cols);
    rows = er, cols = 1;
  } else {
    QH_CHECK(rows == er && cols == ec, QH_ERR_INVALID, "%s: expected shape [%d,%d], got [%d,%d]",
             name, er, ec, rows, cols);
    if (bf16) {
      QH_CHECK(format == QH_FMT_BF16, QH_ERR_INVALID, "%s is the bf16 gather table", name);
    } else {
      QH_CHECK(matrix && is_matrix_format(format), QH_ERR_INVALID,
               "%s must be f16, int8 or int4 (format %d)", name, format);
      qh_weight w{format, rows, cols, format == QH_FMT_INT4 ? group : 0, (const void*)16, nullptr, nullptr};
      w.d_scales = (const float*)16;
      w.d_zeros = (const float*)16;
      qh::DMat probe;
      int rc = qh::make_dmat(&w, &probe);
      if (rc) return fail(rc, "%s: %s", name, qh_last_error());
    }
  }
  return QH_OK;
}

// Keeps `s` as the tensor `name`, releasing an earlier upload of it.
static void keep_staged(qh_model* m, const char* name, const Staged& s) {
  auto it = m->staged.find(name);
  if (it != m->staged.end()) free_staged(it->second);
  m->staged[name] = s;
}

int qh_model_set_tensor(qh_model* m, const char* name, int32_t format, int32_t rows, int32_t cols,
                        int32_t group, const void* h_data, const float* h_scales,
                        const float* h_zeros) {
  QH_CHECK(m && name && h_data, QH_ERR_INVALID, "set_tensor needs a model, a name and data");
  int rc = check_tensor(m, name, format, &rows, &cols, group);
  if (rc) return rc;
  QH_CHECK(!is_matrix_format(format) || format == QH_FMT_F16 || h_scales, QH_ERR_INVALID, "%s needs scales",
           name);
  QH_CHECK(format != QH_FMT_INT4 || h_zeros, QH_ERR_INVALID, "%s needs zero points", name);
  QH_HIP(hipSetDevice(m->ctx->device));
  Staged s;
  s.format = format;
  s.rows = rows;
  s.cols = cols;
  s.group = format == QH_FMT_INT4 ? group : 0;
  const size_t nb = data_bytes(format, rows, cols);
  const size_t ns = format == QH_FMT_INT8 ? (size_t)rows : format == QH_FMT_INT4 ? (size_t)rows * (cols / group) : 0;
  // Every copy and fill of the library goes on the context's stream, which does not
  // synchronize with the null stream; the host arrays are borrowed, so wait before returning.
  hipStream_t st = m->ctx->stream;
  bool ok = hipMalloc(&s.data, nb) == hipSuccess &&
            hipMemcpyAsync(s.data, h_data, nb, hipMemcpyHostToDevice, st) == hipSuccess;
  if (ok && ns) {
    ok = hipMalloc((void**)&s.scales, ns * 4) == hipSuccess &&
         hipMemcpyAsync(s.scales, h_scales, ns * 4, hipMemcpyHostToDevice, st) == hipSuccess;
  }
  if (ok && format == QH_FMT_INT4) {
    ok = hipMalloc((void**)&s.zeros, ns * 4) == hipSuccess &&
         hipMemcpyAsync(s.zeros, h_zeros, ns * 4, hipMemcpyHostToDevice, st) == hipSuccess;
  }
  ok = hipStreamSynchronize(st) == hipSuccess && ok;
  if (!ok) {
    free_staged(s);
    return fail(QH_ERR_NOMEM, "uploading %s failed", name);
  }
  keep_staged(m, name, s);
  return QH_OK;
}

int qh_model_load_tensor(qh_model* m, const char* name, int32_t src_format, int32_t rows, int32_t cols,
                         const void* h_src, int32_t format, int32_t group) {
  QH_CHECK(m && name && h_src, QH_ERR_INVALID, "load_tensor needs a model, a name and data");
  QH_CHECK(src_format == QH_FMT_BF16 || src_format == QH_FMT_F32, QH_ERR_INVALID,
           "%s: checkpoint values are bf16 or f32 (src_format %d)", name, src_format);
  int rc = check_tensor(m, name, format, &rows, &cols, group);
  if (rc) return rc;
  // The gather table, or an f32 vector of an f32 checkpoint: nothing to convert.
  if (format == src_format) return qh_model_set_tensor(m, name, format, rows, cols, group, h_src, nullptr, nullptr);
  QH_CHECK(format != QH_FMT_BF16, QH_ERR_INVALID, "%s: the bf16 gather table takes bf16 values", name);
  QH_HIP(hipSetDevice(m->ctx->device));
  Staged s;
  s.format = format;
  s.rows = rows;
  s.cols = cols;
  s.group = format == QH_FMT_INT4 ? group : 0;
  const size_t nb = data_bytes(format, rows, cols);
  const size_t ns = format == QH_FMT_INT8 ? (size_t)rows : format == QH_FMT_INT4 ? (size_t)rows * (cols / group) : 0;
  const size_t src_bytes = data_bytes(src_format, rows, cols);
  hipStream_t st = m->ctx->stream;
  void* d_src = nullptr;
  bool ok = hipMalloc(&d_src, src_bytes) == hipSuccess && hipMalloc(&s.data, nb) == hipSuccess;
  if (ok && ns) ok = hipMalloc((void**)&s.scales, ns * 4) == hipSuccess;
  if (ok && format == QH_FMT_INT4) ok = hipMalloc((void**)&s.zeros, ns * 4) == hipSuccess;
  if (!ok) {
    hipFree(d_src);
    free_staged(s);
    return fail(QH_ERR_NOMEM, "allocating %s failed", name);
  }
  // The borrowed host array is read before the synchronize below returns.
  ok = hipMemcpyAsync(d_src, h_src, src_bytes, hipMemcpyHostToDevice, st) == hipSuccess &&
       qh::launch_convert(st, src_format == QH_FMT_BF16, d_src, rows, cols, format, s.group, s.data, s.scales,
                          s.zeros) == hipSuccess;
  ok = hipStreamSynchronize(st) == hipSuccess && ok;
  hipFree(d_src);
  if (!ok) {
    free_staged(s);
    return fail(QH_ERR_DEVICE, "converting %s on the device failed", name);
  }
  keep_staged(m, name, s);
  return QH_OK;
}

}  // extern "C"

namespace {

int dmat_of(const Staged& s, void* data, float* scales, float* zeros, int rows, qh::DMat* out) {
  qh_weight w{s.format, rows, s.cols, s.group, data, scales, zeros};
  return qh::make_dmat(&w, out);
}

// Stacks matrices of one format and width row-wise into a new buffer.
int stack_rows(qh_model* m, const std::vector<const Staged*>& parts, qh::DMat* out) {
  const Staged& a = *parts[0];
  int rows = 0;
  for (const Staged* p : parts) {
    QH_CHECK(p->format == a.format && p->cols == a.cols && p->group == a.group, QH_ERR_INVALID,
             "fused projections must share format, width and group");
    rows += p->rows;
  }
  const size_t rb = data_bytes(a.format, 1, a.cols);
  const size_t gpr = a.format == QH_FMT_INT4 ? (size_t)(a.cols / a.group) : 1;
  void* data = nullptr;
  float *scales = nullptr, *zeros = nullptr;
  int rc = m->alloc(rb * rows, &data);
  if (!rc && a.format != QH_FMT_F16) rc = m->alloc(gpr * rows * 4, (void**)&scales);
  if (!rc && a.format == QH_FMT_INT4) rc = m->alloc(gpr * rows * 4, (void**)&zeros);
  if (rc) return rc;
  hipStream_t st = m->ctx->stream;
  size_t r0 = 0;
  for (const Staged* p : parts) {
    QH_HIP(hipMemcpyAsync((char*)data + r0 * rb, p->data, rb * p->rows, hipMemcpyDeviceToDevice, st));
    if (scales)
      QH_HIP(hipMemcpyAsync(scales + r0 * gpr, p->scales, gpr * p->rows * 4, hipMemcpyDeviceToDevice, st));
    if (zeros)
      QH_HIP(hipMemcpyAsync(zeros + r0 * gpr, p->zeros, gpr * p->rows * 4, hipMemcpyDeviceToDevice, st));
    r0 += p->rows;
  }
  return dmat_of(a, data, scales, zeros, rows, out);
}

// Interleaves the rows of two same-shape matrices: row 2i = a[i], row 2i+1 = b[i].
int interleave_rows(qh_model* m, const Staged& a, const Staged& b, qh::DMat* out) {
  QH_CHECK(a.format == b.format && a.cols == b.cols && a.group == b.group && a.rows == b.rows,
           QH_ERR_INVALID, "gate and up projections must share format and shape");
  const size_t rb = data_bytes(a.format, 1, a.cols);
  const size_t gpr = a.format == QH_FMT_INT4 ? (size_t)(a.cols / a.group) : 1;
  const int rows = 2 * a.rows;
  void* data = nullptr;
  float *scales = nullptr, *zeros = nullptr;
  int rc = m->alloc(rb * rows, &data);
  if (!rc && a.format != QH_FMT_F16) rc = m->alloc(gpr * rows * 4, (void**)&scales);
  if (!rc && a.format == QH_FMT_INT4) rc = m->alloc(gpr * rows * 4, (void**)&zeros);
  if (rc) return rc;
  hipStream_t st = m->ctx->stream;
  for (int k = 0; k < 2; k++) {
    const Staged& s = k == 0 ? a : b;
    QH_HIP(hipMemcpy2DAsync((char*)data + k * rb, 2 * rb, s.data, rb, rb, s.rows, hipMemcpyDeviceToDevice, st));
    if (scales)
      QH_HIP(hipMemcpy2DAsync((char*)scales + k * gpr * 4, 2 * gpr * 4, s.scales, gpr * 4, gpr * 4, s.rows,
                              hipMemcpyDeviceToDevice, st));
    if (zeros)
      QH_HIP(hipMemcpy2DAsync((char*)zeros + k * gpr * 4, 2 * gpr * 4, s.zeros, gpr * 4, gpr * 4, s.rows,
                              hipMemcpyDeviceToDevice, st));
  }
  return dmat_of(a, data, scales, zeros, rows, out);
}

}  // namespace

extern "C" {

int qh_model_finalize(qh_model* m) {
  QH_CHECK(m, QH_ERR_INVALID, "model is NULL");
  QH_CHECK(!m->finalized, QH_ERR_STATE, "model is already finalized");
  const qh_config& c = m->cfg;
  // Every tensor the architecture implies must be present (config.js:126-152).
  std::vector<std::string> missing;
  auto need = [&](const std::string& n) {
    if (!m->staged.count(n)) missing.push_back(n);
  };
  need("model.embed_tokens.weight");
  need("lm_head.weight");
  need("model.norm.weight");
  for (int L = 0; L < c.layers; L++)
    for (const char* s : kLayerNames) need("model.layers." + std::to_string(L) + "." + s);
  if (!missing.empty()) {
    std::string list;
    for (size_t i = 0; i < missing.size() && i < 5; i++) list += (i ? ", " : "") + missing[i];
    return fail(QH_ERR_STATE, "missing %zu tensors: %s%s", missing.size(), list.c_str(),
                missing.size() > 5 ? ", ..." : "");
  }
  QH_HIP(hipSetDevice(m->ctx->device));
  const int kv_dim = c.kv_heads * c.head_dim;
  m->layers.resize(c.layers);
  std::vector<std::string> consumed;
  for (int L = 0; L < c.layers; L++) {
    const std::string p = "model.layers." + std::to_string(L) + ".";
    auto& S = m->staged;
    qh::LayerDev& d = m->layers[L];
    int rc = stack_rows(m, {&S[p + "self_attn.q_proj.weight"], &S[p + "self_attn.k_proj.weight"],
                            &S[p + "self_attn.v_proj.weight"]},
                        &d.qkv);
    if (!rc) rc = interleave_rows(m, S[p + "mlp.gate_proj.weight"], S[p + "mlp.up_proj.weight"], &d.gu);
    if (rc) return rc;
    const Staged& o = S[p + "self_attn.o_proj.weight"];
    const Staged& dn = S[p + "mlp.down_proj.weight"];
    if ((rc = dmat_of(o, o.data, o.scales, o.zeros, o.rows, &d.o))) return rc;
    if ((rc = dmat_of(dn, dn.data, dn.scales, dn.zeros, dn.rows, &d.down))) return rc;
    float* bias = nullptr;
    if ((rc = m->alloc((size_t)(c.hidden + 2 * kv_dim) * 4, (void**)&bias))) return rc;
    hipStream_t st = m->ctx->stream;
    QH_HIP(hipMemcpyAsync(bias, S[p + "self_attn.q_proj.bias"].data, (size_t)c.hidden * 4, hipMemcpyDeviceToDevice, st));
    QH_HIP(hipMemcpyAsync(bias + c.hidden, S[p + "self_attn.k_proj.bias"].data, (size_t)kv_dim * 4,
                          hipMemcpyDeviceToDevice, st));
    QH_HIP(hipMemcpyAsync(bias + c.hidden + kv_dim, S[p + "self_attn.v_proj.bias"].data, (size_t)kv_dim * 4,
                          hipMemcpyDeviceToDevice, st));
    d.qkv_bias = bias;
    d.in_norm = static_cast<const float*>(S[p + "input_layernorm.weight"].data);
    d.post_norm = static_cast<const float*>(S[p + "post_attention_layernorm.weight"].data);
    for (const char* keep : {"self_attn.o_proj.weight", "mlp.down_proj.weight", "input_layernorm.weight",
                             "post_attention_layernorm.weight"}) {
      Staged& s = S[p + keep];
      m->keep(s.data);
      m->keep(s.scales);
      m->keep(s.zeros);
      m->bytes += data_bytes(s.format, s.rows, s.cols);
      s = Staged{};
    }
    for (const char* used : {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                             "mlp.gate_proj.weight", "mlp.up_proj.weight", "self_attn.q_proj.bias",
                             "self_attn.k_proj.bias", "self_attn.v_proj.bias"}) {
      consumed.push_back(p + used);
    }
  }
  Staged& lm = m->staged["lm_head.weight"];
  int rc = dmat_of(lm, lm.data, lm.scales, lm.zeros, lm.rows, &m->dev.lm_head);
  if (rc) return rc;
  m->keep(lm.data), m->keep(lm.scales), m->keep(lm.zeros);
  m->bytes += data_bytes(lm.format, lm.rows, lm.cols);
  lm = Staged{};
  Staged& fn = m->staged["model.norm.weight"];
  m->dev.final_norm = static_cast<const float*>(fn.data);
  m->keep(fn.data);
  fn = Staged{};
  Staged& em = m->staged["model.embed_tokens.weight"];
  m->dev.embed = static_cast<const uint16_t*>(em.data);
  m->keep(em.data);
  m->bytes += data_bytes(QH_FMT_BF16, em.rows, em.cols);
  em = Staged{};
  // The stacking copies read the staged buffers: let them finish before freeing those.
  QH_HIP(hipStreamSynchronize(m->ctx->stream));
  for (auto& n : consumed) free_staged(m->staged[n]);
  m->staged.clear();

  // Rope cos/sin in f64 from the host's libm: the values src/core/ops.js:147-159 rotates
  // by (ropeInPlace evaluates them per call; here they are tabulated once).
  std::vector<double> cs((size_t)c.max_positions * 32), sn((size_t)c.max_positions * 32);
  qh::rope_tables_f64(c.head_dim, c.rope_theta, c.max_positions, cs.data(), sn.data());
  double *dcos = nullptr, *dsin = nullptr;
  if ((rc = m->alloc(cs.size() * 8, (void**)&dcos)) || (rc = m->alloc(sn.size() * 8, (void**)&dsin))) return rc;
  QH_HIP(hipMemcpyAsync(dcos, cs.data(), cs.size() * 8, hipMemcpyHostToDevice, m->ctx->stream));
  QH_HIP(hipMemcpyAsync(dsin, sn.data(), sn.size() * 8, hipMemcpyHostToDevice, m->ctx->stream));
  QH_HIP(hipStreamSynchronize(m->ctx->stream));

  qh::ModelDev& d = m->dev;
  d.hidden = c.hidden;
  d.intermediate = c.intermediate;
  d.layers = c.layers;
  d.heads = c.heads;
  d.kv_heads = c.kv_heads;
  d.head_dim = c.head_dim;
  d.vocab = c.vocab;
  d.max_positions = c.max_positions;
  d.eps = c.eps;
  d.layers_host = m->layers.data();
  d.rope_cos = dcos;
  d.rope_sin = dsin;
  if (m->numerics == QH_NUMERICS_FAST && c.heads > 16) m->numerics = QH_NUMERICS_EXACT;
  d.numerics = m->numerics;
  m->finalized = true;
  return QH_OK;
}

int qh_model_set_numerics(qh_model* m, int32_t numerics) {
  QH_CHECK(m, QH_ERR_INVALID, "model is NULL");
  QH_CHECK(numerics == QH_NUMERICS_FAST || numerics == QH_NUMERICS_EXACT, QH_ERR_INVALID,
           "unknown numerics mode %d", numerics);
  QH_CHECK(m->caches_made == 0, QH_ERR_STATE, "set the numerics before the model's first cache");
  QH_CHECK(numerics != QH_NUMERICS_FAST || m->cfg.heads <= 16, QH_ERR_INVALID,
           "fast numerics supports at most 16 query heads (got %d)", m->cfg.heads);
  m->numerics = numerics;
  m->dev.numerics = numerics;
  return QH_OK;
}

int qh_model_set_matmul(qh_model* m, int32_t matmul) {
  QH_CHECK(m, QH_ERR_INVALID, "model is NULL");
  QH_CHECK(matmul == QH_MATMUL_BATCHED || matmul == QH_MATMUL_MATVEC || matmul == QH_MATMUL_MFMA,
           QH_ERR_INVALID, "unknown matmul mode %d", matmul);
  m->matmul = matmul;
  return QH_OK;
}

int qh_model_free(qh_model* m) {
  if (!m) return QH_OK;
  QH_CHECK(m->live_caches == 0, QH_ERR_STATE, "free the model's %d caches first", m->live_caches);
  hipSetDevice(m->ctx->device);
  hipStreamSynchronize(m->ctx->stream);
  for (auto& kv : m->staged) free_staged(kv.second);
  for (void* p : m->allocs) hipFree(p);
  delete m;
  return QH_OK;
}

int qh_model_bytes(qh_model* m, size_t* bytes) {
  QH_CHECK(m && bytes, QH_ERR_INVALID, "model_bytes needs a model and an output");
  *bytes = m->bytes;
  return QH_OK;
}

int qh_model_config(qh_model* m, qh_config* out) {
  QH_CHECK(m && out, QH_ERR_INVALID, "model_config needs a model and an output");
  *out = m->cfg;
  return QH_OK;
}

int qh_cache_create(qh_model* m, int32_t capacity, qh_cache** out) {
  QH_CHECK(m && out, QH_ERR_INVALID, "cache_create needs a model and an output");
  *out = nullptr;
  QH_CHECK(m->finalized, QH_ERR_STATE, "finalize the model before creating a cache");
  QH_CHECK(capacity >= 1, QH_ERR_RANGE, "cache capacity must be a positive integer, got %d", capacity);
  QH_HIP(hipSetDevice(m->ctx->device));
  const qh::ModelDev& md = m->dev;
  qh_cache* c = new qh_cache();
  c->m = m;
  qh::CacheDev& d = c->dev;
  d.capacity = capacity;
  d.vstride = qh::value_stride(capacity);
  d.key_elems = (size_t)md.kv_heads * capacity * md.head_dim;
  d.layer_elems = d.key_elems + (size_t)md.kv_heads * md.head_dim * d.vstride;
  d.score_stride = (capacity + 3) & ~3;
  const int spans = qh::attn_spans(capacity);
  const size_t kv_bytes = (size_t)md.layers * d.layer_elems * 2;
  int rc = QH_OK;
  auto A = [&](size_t n, void** p) {
    if (!rc) rc = c->alloc(n, p);
  };
  A(kv_bytes, (void**)&d.kv);
  A(256, (void**)&d.state);
  A((size_t)(capacity + 1) * 4, (void**)&d.tokens);
  A((size_t)capacity * 4, (void**)&d.pred);
  A((size_t)md.hidden * 4, (void**)&d.x);
  A((size_t)md.hidden * 4, (void**)&d.q);
  A((size_t)md.hidden * 4, (void**)&d.attn);
  A((size_t)md.intermediate * 4, (void**)&d.h);
  A((size_t)md.vocab * 4, (void**)&d.logits);
  A((size_t)md.heads * d.score_stride * 4, (void**)&d.scores);
  A((size_t)md.heads * spans * 4, (void**)&d.maxes);
  A(256, (void**)&d.attn_counters);
  A(qh::attn_part_bytes(md, capacity), (void**)&d.part);
  A(qh::lm_partials_bytes(md), &d.lm_partials);
  if (!rc && hipHostMalloc((void**)&c->h_pinned, 64, hipHostMallocDefault) != hipSuccess) {
    rc = fail(QH_ERR_NOMEM, "pinned allocation failed");
  }
  hipStream_t st = m->ctx->stream;  // ordered before every later use of the cache
  if (!rc && (hipMemsetAsync(d.kv, 0, kv_bytes, st) != hipSuccess || hipMemsetAsync(d.state, 0, 256, st) != hipSuccess ||
              hipMemsetAsync(d.tokens, 0, (size_t)(capacity + 1) * 4, st) != hipSuccess ||
              hipMemsetAsync(d.pred, 0, (size_t)capacity * 4, st) != hipSuccess ||
              hipMemsetAsync(d.attn_counters, 0, 256, st) != hipSuccess || hipStreamSynchronize(st) != hipSuccess)) {
    rc = fail(QH_ERR_DEVICE, "clearing the cache failed");
  }
  d.lm_blocks = qh::lm_head_blocks(md);
  if (rc) {
    for (void* p : c->allocs) hipFree(p);
    if (c->h_pinned) hipHostFree(c->h_pinned);
    delete c;
    return rc;
  }
  m->live_caches++;
  m->caches_made++;
  *out = c;
  return QH_OK;
}

int qh_cache_free(qh_cache* c) {
  if (!c) return QH_OK;
  QH_CHECK(!c->busy, QH_ERR_BUSY, "cache has a decode in flight; collect it first");
  hipSetDevice(c->m->ctx->device);
  hipStreamSynchronize(c->m->ctx->stream);
  if (c->exec_first) hipGraphExecDestroy(c->exec_first);
  if (c->graph_first) hipGraphDestroy(c->graph_first);
  if (c->exec) hipGraphExecDestroy(c->exec);
  if (c->graph) hipGraphDestroy(c->graph);
  if (c->exec_run) hipGraphExecDestroy(c->exec_run);
  if (c->graph_run) hipGraphDestroy(c->graph_run);
  drop_prefill_graphs(c);
  for (void* p : c->allocs) hipFree(p);
  hipFree(c->d_hidden);
  if (c->pw_mem) hipFree(c->pw_mem);
  hipHostFree(c->h_pinned);
  c->m->live_caches--;
  delete c;
  return QH_OK;
}

int qh_cache_length(qh_cache* c, int32_t* length) {
  QH_CHECK(c && length, QH_ERR_INVALID, "cache_length needs a cache and an output");
  *length = c->length;
  return QH_OK;
}

int qh_cache_set_length(qh_cache* c, int32_t length) {
  QH_CHECK(c, QH_ERR_INVALID, "cache is NULL");
  QH_CHECK(!c->busy, QH_ERR_BUSY, "cache has a decode in flight");
  QH_CHECK(length >= 0 && length <= c->length, QH_ERR_RANGE,
           "can rewind to 0..%d positions, not %d", c->length, length);
  c->length = length;
  return QH_OK;
}

int qh_cache_present(qh_cache* c, int32_t layer, float* h_key, float* h_value) {
  QH_CHECK(c && h_key && h_value, QH_ERR_INVALID, "cache_present needs a cache and outputs");
  const qh::ModelDev& md = c->m->dev;
  QH_CHECK(layer >= 0 && layer < md.layers, QH_ERR_RANGE, "layer %d out of range", layer);
  QH_CHECK(!c->busy, QH_ERR_BUSY, "cache has a decode in flight");
  const qh::CacheDev& d = c->dev;
  std::vector<uint16_t> buf(d.layer_elems);
  QH_HIP(hipMemcpyAsync(buf.data(), d.kv + (size_t)layer * d.layer_elems, buf.size() * 2, hipMemcpyDeviceToHost,
                        c->m->ctx->stream));
  QH_HIP(hipStreamSynchronize(c->m->ctx->stream));
  const int n = c->length, hd = md.head_dim;
  const uint16_t* vt = buf.data() + d.key_elems;
  for (int h = 0; h < md.kv_heads; h++) {
    for (int t = 0; t < n; t++) {
      for (int i = 0; i < hd; i++) {
        const size_t to = ((size_t)h * n + t) * hd + i;
        h_key[to] = f16_to_f32(buf[((size_t)h * d.capacity + t) * hd + i]);
        h_value[to] = f16_to_f32(vt[((size_t)h * hd + i) * d.vstride + t]);
      }
    }
  }
  return QH_OK;
}

}  // extern "C"

namespace {

// Guards of GpuModel.#forward (src/gpu/model.js:247-254).
int check_room(qh_cache* c, int add) {
  const int total = c->length + add;
  QH_CHECK(total <= c->dev.capacity, QH_ERR_RANGE, "cache holds %d of %d; cannot add %d", c->length,
           c->dev.capacity, add);
  QH_CHECK(total <= c->m->dev.max_positions, QH_ERR_RANGE,
           "position %d exceeds the %d-entry rope table", total, c->m->dev.max_positions);
  return QH_OK;
}

int set_state(qh_cache* c, int pos, int forced) {
  c->h_pinned[0] = pos;
  c->h_pinned[1] = forced;
  QH_HIP(hipMemcpyAsync(c->dev.state, c->h_pinned, 8, hipMemcpyHostToDevice, c->m->ctx->stream));
  return QH_OK;
}

int finish_forward(qh_cache* c, int seq, float* h_logits, int32_t* h_argmax) {
  hipStream_t s = c->m->ctx->stream;
  const int last = c->length + seq - 1;
  if (h_logits) {
    QH_HIP(hipMemcpyAsync(h_logits, c->dev.logits, (size_t)c->m->dev.vocab * 4, hipMemcpyDeviceToHost, s));
  }
  if (h_argmax) QH_HIP(hipMemcpyAsync(c->h_pinned + 2, c->dev.pred + last, 4, hipMemcpyDeviceToHost, s));
  QH_HIP(hipStreamSynchronize(s));
  if (h_argmax) *h_argmax = c->h_pinned[2];
  c->length += seq;
  return QH_OK;
}

// The batched-prefill workspace for the model's current matmul mode: one allocation,
// carved in the order prefill_bytes() counts it.
int ensure_prefill(qh_cache* c) {
  qh_model* m = c->m;
  // The sizes depend on the model, the cache and the matmul mode only: checked once per mode
  // (they walk every layer matrix on the host, in front of the forward's first launch).
  if (c->pw_mem && c->pw_matmul == m->matmul) return QH_OK;
  const qh::PrefillBytes b = qh::prefill_bytes(m->dev, c->dev, m->matmul);
  if (c->pw_mem && b.floats <= c->pw_bytes.floats && b.counters <= c->pw_bytes.counters &&
      b.scratch <= c->pw_bytes.scratch) {
    c->pw_matmul = m->matmul;
    return QH_OK;
  }
  hipStream_t s = m->ctx->stream;
  QH_HIP(hipStreamSynchronize(s));
  drop_prefill_graphs(c);  // they address the workspace being replaced
  if (c->pw_mem) hipFree(c->pw_mem);
  c->pw_mem = nullptr;
  const size_t fbytes = (b.floats * 4 + 255) & ~(size_t)255, cbytes = (b.counters * 4 + 255) & ~(size_t)255;
  if (hipMalloc(&c->pw_mem, fbytes + cbytes + b.scratch + 256) != hipSuccess) {
    c->pw_mem = nullptr;
    return fail(QH_ERR_NOMEM, "prefill workspace of %zu bytes", fbytes + cbytes + b.scratch);
  }
  QH_HIP(hipMemsetAsync(static_cast<char*>(c->pw_mem) + fbytes, 0, cbytes, s));
  c->pw_bytes = b;
  c->pw_matmul = m->matmul;
  const qh::ModelDev& d = m->dev;
  const size_t P = qh::prefill_chunk(d, c->dev);
  const size_t hd = d.hidden, kv = (size_t)d.kv_heads * d.head_dim, f = d.intermediate;
  float* p = static_cast<float*>(c->pw_mem);
  qh::PrefillDev& w = c->pw;
  w.positions = (int)P;
  w.X = p, p += P * hd;
  w.XN = p, p += P * hd;
  w.Q = p, p += P * hd;
  w.ATT = p, p += P * hd;
  w.Y = p, p += P * hd;
  w.QKV = p, p += P * (hd + 2 * kv);
  w.GU = p, p += P * 2 * f;
  w.H = p, p += P * f;
  w.part = w.scores = p;
  w.counters = reinterpret_cast<int*>(static_cast<char*>(c->pw_mem) + fbytes);
  w.scratch = static_cast<char*>(c->pw_mem) + fbytes + cbytes;
  w.scratch_bytes = b.scratch;
  return QH_OK;
}

// One chunk's launches (the gather from token ids, unless the rows came from the host, and
// every layer). A shape run before is replayed from its graph (captured on its second use,
// so a one-off length pays no capture), which removes the host's per-launch cost and the
// device's gaps between the ~250 launches; the least recently used of kPrefillGraphs shapes
// makes room for a new one. use_graph = 0 (qh_decode_use_graph) enqueues directly.
static int prefill_chunk(qh_cache* c, bool tokens, int past, int n) {
  qh_model* m = c->m;
  hipStream_t s = m->ctx->stream;
  const qh::ModelDev& d = m->dev;
  auto enqueue = [&]() -> hipError_t {
    if (tokens) {
      const hipError_t e = qh::enqueue_embed_rows(s, d, c->dev, c->pw, past, n);
      if (e != hipSuccess) return e;
    }
    return qh::enqueue_prefill_layers(s, d, c->dev, c->pw, m->matmul, past, n);
  };
  if (!c->use_graph) {
    QH_HIP(enqueue());
    return QH_OK;
  }
  PrefillGraph* g = nullptr;
  for (PrefillGraph& e : c->pgraphs)
    if (e.past == past && e.n == n && e.matmul == m->matmul && e.numerics == d.numerics && e.tokens == tokens) g = &e;
  if (!g) {
    if ((int)c->pgraphs.size() >= kPrefillGraphs) {
      auto lru = std::min_element(c->pgraphs.begin(), c->pgraphs.end(),
                                  [](const PrefillGraph& a, const PrefillGraph& b) { return a.last < b.last; });
      QH_HIP(hipStreamSynchronize(s));
      if (lru->exec) hipGraphExecDestroy(lru->exec);
      if (lru->graph) hipGraphDestroy(lru->graph);
      c->pgraphs.erase(lru);
    }
    c->pgraphs.push_back(PrefillGraph{past, n, m->matmul, d.numerics, tokens, 0, 0, nullptr, nullptr});
    g = &c->pgraphs.back();
  }
  g->last = ++c->pclock;
  if (!g->exec && ++g->uses >= 2) {
    QH_HIP(hipStreamSynchronize(s));
    QH_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed));
    const hipError_t e = enqueue();
    hipGraph_t graph = nullptr;
    const hipError_t e2 = hipStreamEndCapture(s, &graph);
    if (e != hipSuccess || e2 != hipSuccess) {
      if (graph) hipGraphDestroy(graph);
      QH_HIP(e != hipSuccess ? e : e2);
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t e3 = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e3 != hipSuccess) {
      hipGraphDestroy(graph);
      QH_HIP(e3);
    }
    g->graph = graph;
    g->exec = exec;
  }
  if (g->exec) QH_HIP(hipGraphLaunch(g->exec, s));
  else QH_HIP(enqueue());
  return QH_OK;
}

// forward() over seq > 1 positions, batched: the input rows (host `h_hidden`, else the
// cache's tokens) pass through the layers in chunks, then the last row through the head.
int batched_forward(qh_cache* c, const float* h_hidden, int seq, bool want, int forced) {
  qh_model* m = c->m;
  int rc = ensure_prefill(c);
  if (rc) return rc;
  hipStream_t s = m->ctx->stream;
  const qh::ModelDev& d = m->dev;
  const int P = c->pw.positions;
  int n = 0;
  for (int done = 0; done < seq; done += n) {
    n = std::min(P, seq - done);
    const int past = c->length + done;
    if (h_hidden) {
      QH_HIP(hipMemcpyAsync(c->pw.X, h_hidden + (size_t)done * d.hidden, (size_t)n * d.hidden * 4,
                            hipMemcpyHostToDevice, s));
    }
    if ((rc = prefill_chunk(c, h_hidden == nullptr, past, n))) return rc;
  }
  QH_HIP(hipMemcpyAsync(c->dev.x, c->pw.X + (size_t)(n - 1) * d.hidden, (size_t)d.hidden * 4,
                        hipMemcpyDeviceToDevice, s));
  if (want) {
    if ((rc = set_state(c, c->length + seq - 1, forced))) return rc;
    QH_HIP(qh::enqueue_head(s, d, c->dev));
  } else if ((rc = set_state(c, c->length + seq, forced))) {
    return rc;
  }
  return QH_OK;
}

struct BusyGuard {
  qh_cache* c;
  explicit BusyGuard(qh_cache* c_) : c(c_) { c->busy = true; }
  ~BusyGuard() { c->busy = false; }
};

}  // namespace

extern "C" {

int qh_forward(qh_model* m, qh_cache* c, const float* h_hidden, int32_t seq, float* h_logits,
               int32_t* h_argmax) {
  QH_CHECK(m && c && h_hidden && c->m == m, QH_ERR_INVALID, "forward needs a model, its cache and input");
  QH_CHECK(!c->busy, QH_ERR_BUSY, "forward() is already running; await it first");
  QH_CHECK(seq >= 1, QH_ERR_INVALID, "forward: need at least one position");
  int rc = check_room(c, seq);
  if (rc) return rc;
  BusyGuard guard(c);
  QH_HIP(hipSetDevice(m->ctx->device));
  hipStream_t s = m->ctx->stream;
  const bool want = h_logits || h_argmax;
  if (seq > 1 && m->matmul != QH_MATMUL_MATVEC) {
    if ((rc = batched_forward(c, h_hidden, seq, want, INT_MAX))) return rc;
    return finish_forward(c, seq, h_logits, h_argmax);
  }
  const size_t need = (size_t)seq * m->dev.hidden * 4;
  if (need > c->hidden_cap) {
    QH_HIP(hipStreamSynchronize(s));
    hipFree(c->d_hidden);
    c->d_hidden = nullptr;
    c->hidden_cap = 0;
    QH_HIP(hipMalloc((void**)&c->d_hidden, need));
    c->hidden_cap = need;
  }
  QH_HIP(hipMemcpyAsync(c->d_hidden, h_hidden, need, hipMemcpyHostToDevice, s));
  if ((rc = set_state(c, c->length, INT_MAX))) return rc;
  for (int t = 0; t < seq; t++) {
    QH_HIP(hipMemcpyAsync(c->dev.x, c->d_hidden + (size_t)t * m->dev.hidden, (size_t)m->dev.hidden * 4,
                          hipMemcpyDeviceToDevice, s));
    QH_HIP(qh::enqueue_step(s, m->dev, c->dev, qh::STEP_HIDDEN, want && t == seq - 1));
  }
  return finish_forward(c, seq, h_logits, h_argmax);
}

int qh_forward_tokens(qh_model* m, qh_cache* c, const int32_t* h_ids, int32_t seq, float* h_logits,
                      int32_t* h_argmax) {
  QH_CHECK(m && c && h_ids && c->m == m, QH_ERR_INVALID, "forward needs a model, its cache and ids");
  QH_CHECK(!c->busy, QH_ERR_BUSY, "forward() is already running; await it first");
  QH_CHECK(seq >= 1, QH_ERR_INVALID, "forward: need at least one token");
  for (int t = 0; t < seq; t++) {
    QH_CHECK(h_ids[t] >= 0 && h_ids[t] < m->dev.vocab, QH_ERR_RANGE,
             "token %d at position %d is outside the vocabulary", h_ids[t], t);
  }
  int rc = check_room(c, seq);
  if (rc) return rc;
  BusyGuard guard(c);
  QH_HIP(hipSetDevice(m->ctx->device));
  hipStream_t s = m->ctx->stream;
  QH_HIP(hipMemcpyAsync(c->dev.tokens + c->length, h_ids, (size_t)seq * 4, hipMemcpyHostToDevice, s));
  const bool want = h_logits || h_argmax;
  if (seq > 1 && m->matmul != QH_MATMUL_MATVEC) {
    if ((rc = batched_forward(c, nullptr, seq, want, c->length + seq))) return rc;
    return finish_forward(c, seq, h_logits, h_argmax);
  }
  if ((rc = set_state(c, c->length, c->length + seq))) return rc;
  for (int t = 0; t < seq; t++) {
    QH_HIP(qh::enqueue_step(s, m->dev, c->dev, qh::STEP_GATHER, want && t == seq - 1));
  }
  return finish_forward(c, seq, h_logits, h_argmax);
}

int qh_score(qh_model* m, qh_cache* c, const int32_t* h_ids, int32_t n, double* h_nll) {
  QH_CHECK(m && c && h_ids && h_nll && c->m == m, QH_ERR_INVALID, "score needs a model, its cache, ids and an output");
  QH_CHECK(!c->busy, QH_ERR_BUSY, "forward() is already running; await it first");
  QH_CHECK(n >= 2, QH_ERR_INVALID, "score needs at least two tokens (the first is context only)");
  for (int t = 0; t < n; t++) {
    QH_CHECK(h_ids[t] >= 0 && h_ids[t] < m->dev.vocab, QH_ERR_RANGE,
             "token %d at position %d is outside the vocabulary", h_ids[t], t);
  }
  int rc = check_room(c, n - 1);
  if (rc) return rc;
  BusyGuard guard(c);
  QH_HIP(hipSetDevice(m->ctx->device));
  hipStream_t s = m->ctx->stream;
  struct Scratch {
    int32_t* ids = nullptr;
    double* nll = nullptr;
    ~Scratch() {
      hipFree(ids);
      hipFree(nll);
    }
  } d;
  QH_HIP(hipMalloc((void**)&d.ids, (size_t)n * 4));
  QH_HIP(hipMalloc((void**)&d.nll, (size_t)(n - 1) * 8));
  QH_HIP(hipMemcpyAsync(d.ids, h_ids, (size_t)n * 4, hipMemcpyHostToDevice, s));
  // ids[0..n-2] are fed (teacher-forced); ids[t+1] is scored under step t's logits.
  QH_HIP(hipMemcpyAsync(c->dev.tokens + c->length, d.ids, (size_t)(n - 1) * 4, hipMemcpyDeviceToDevice, s));
  if ((rc = set_state(c, c->length, c->length + n - 1))) return rc;
  for (int t = 0; t < n - 1; t++) {
    QH_HIP(qh::enqueue_step(s, m->dev, c->dev, qh::STEP_GATHER, true));
    QH_HIP(qh::launch_nll(s, c->dev.logits, m->dev.vocab, d.ids + t + 1, d.nll + t));
  }
  QH_HIP(hipMemcpyAsync(h_nll, d.nll, (size_t)(n - 1) * 8, hipMemcpyDeviceToHost, s));
  QH_HIP(hipStreamSynchronize(s));
  c->length += n - 1;
  return QH_OK;
}

constexpr int kGraphRun = 8;  // decode steps per replayed run graph

// A decode call of n steps: a gather of the first input row, a first step that takes it and
// leaves its pick to the next step's first launch, n - 1 steps that make their predecessor's
// pick in that launch and leave theirs to the next, and the last step's pick on its own.
//
// Captures the cache's decode graphs that are not captured yet: the first step, one later
// step, and (`run`) kGraphRun later steps back to back. Each is uploaded to the device once,
// so its first replay costs what every later one does.
static int capture_graphs(qh_model* m, qh_cache* c, bool run) {
  hipStream_t s = m->ctx->stream;
  auto capture = [&](int n, qh::StepInput in, hipGraph_t* graph, hipGraphExec_t* exec) -> int {
    QH_HIP(hipStreamSynchronize(s));
    QH_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed));
    hipError_t e = hipSuccess;
    for (int i = 0; i < n && e == hipSuccess; i++) e = qh::enqueue_step(s, m->dev, c->dev, in, true, nullptr, true);
    hipGraph_t g = nullptr;
    hipError_t e2 = hipStreamEndCapture(s, &g);
    QH_HIP(e);
    QH_HIP(e2);
    *graph = g;
    QH_HIP(hipGraphInstantiate(exec, g, nullptr, nullptr, 0));
    QH_HIP(hipGraphUpload(*exec, s));
    QH_HIP(hipStreamSynchronize(s));
    return QH_OK;
  };
  int rc = QH_OK;
  if (!c->exec_first && (rc = capture(1, qh::STEP_CARRIED, &c->graph_first, &c->exec_first))) return rc;
  if (!c->exec && (rc = capture(1, qh::STEP_PICK, &c->graph, &c->exec))) return rc;
  if (run && !c->exec_run && (rc = capture(kGraphRun, qh::STEP_PICK, &c->graph_run, &c->exec_run))) return rc;
  return QH_OK;
}

int qh_decode_prepare(qh_model* m, qh_cache* c) {
  QH_CHECK(m && c && c->m == m, QH_ERR_INVALID, "decode_prepare needs a model and its cache");
  QH_CHECK(!c->busy, QH_ERR_BUSY, "forward() is already running; await it first");
  QH_HIP(hipSetDevice(m->ctx->device));
  if (!c->use_graph) return QH_OK;
  return capture_graphs(m, c, true);
}

int qh_decode_launch(qh_model* m, qh_cache* c, int32_t first_token, int32_t steps) {
  QH_CHECK(m && c && c->m == m, QH_ERR_INVALID, "decode needs a model and its cache");
  QH_CHECK(!c->busy, QH_ERR_BUSY, "forward() is already running; await it first");
  QH_CHECK(steps >= 1, QH_ERR_INVALID, "decode needs steps >= 1");
  QH_CHECK(first_token >= 0 && first_token < m->dev.vocab, QH_ERR_RANGE,
           "token %d is outside the vocabulary", first_token);
  int rc = check_room(c, steps);
  if (rc) return rc;
  QH_HIP(hipSetDevice(m->ctx->device));
  hipStream_t s = m->ctx->stream;
  // The steps after the first are identical launches (position and tokens live on the
  // device), so a graph of kGraphRun of them replays runs of steps with one launch each.
  if (c->use_graph && (rc = capture_graphs(m, c, steps - 1 >= kGraphRun))) return rc;
  c->h_pinned[3] = first_token;
  QH_HIP(hipMemcpyAsync(c->dev.tokens + c->length, c->h_pinned + 3, 4, hipMemcpyHostToDevice, s));
  if ((rc = set_state(c, c->length, c->length + 1))) return rc;
  // The launches of capture_graphs' decode call.
  QH_HIP(qh::enqueue_gather(s, m->dev, c->dev));
  if (c->use_graph) QH_HIP(hipGraphLaunch(c->exec_first, s));
  else QH_HIP(qh::enqueue_step(s, m->dev, c->dev, qh::STEP_CARRIED, true, nullptr, true));
  for (int i = 1; i < steps;) {
    if (c->use_graph && steps - i >= kGraphRun) {
      QH_HIP(hipGraphLaunch(c->exec_run, s));
      i += kGraphRun;
      continue;
    }
    if (c->use_graph) QH_HIP(hipGraphLaunch(c->exec, s));
    else QH_HIP(qh::enqueue_step(s, m->dev, c->dev, qh::STEP_PICK, true, nullptr, true));
    i++;
  }
  QH_HIP(qh::enqueue_pick(s, m->dev, c->dev));
  c->busy = true;
  c->pending_start = c->length;
  c->pending_steps = steps;
  c->length += steps;
  return QH_OK;
}

int qh_decode_use_graph(qh_cache* c, int32_t use_graph) {
  QH_CHECK(c, QH_ERR_INVALID, "decode_use_graph needs a cache");
  QH_CHECK(!c->busy, QH_ERR_BUSY, "forward() is already running; await it first");
  c->use_graph = use_graph != 0;
  return QH_OK;
}

int qh_decode_collect(qh_model* m, qh_cache* c, int32_t steps, int32_t* h_tokens) {
  QH_CHECK(m && c && c->m == m, QH_ERR_INVALID, "decode needs a model and its cache");
  QH_CHECK(c->busy && c->pending_steps > 0, QH_ERR_STATE, "no decode in flight");
  QH_CHECK(steps == c->pending_steps, QH_ERR_INVALID, "collect %d steps, %d were launched", steps,
           c->pending_steps);
  hipStream_t s = m->ctx->stream;
  hipError_t e = hipSuccess;
  if (h_tokens) e = hipMemcpyAsync(h_tokens, c->dev.pred + c->pending_start, (size_t)steps * 4, hipMemcpyDeviceToHost, s);
  hipError_t e2 = hipStreamSynchronize(s);
  c->busy = false;
  c->pending_steps = 0;
  QH_HIP(e);
  QH_HIP(e2);
  return QH_OK;
}

int qh_decode(qh_model* m, qh_cache* c, int32_t first_token, int32_t steps, int32_t* h_tokens) {
  int rc = qh_decode_launch(m, c, first_token, steps);
  if (rc) return rc;
  return qh_decode_collect(m, c, steps, h_tokens);
}

int qh_decode_kernel_time(qh_model* m, qh_cache* c, int32_t role, int32_t reps, float* us_per_launch) {
  QH_CHECK(m && c && c->m == m && us_per_launch, QH_ERR_INVALID, "kernel_time needs a model, its cache and an output");
  QH_CHECK(!c->busy, QH_ERR_BUSY, "forward() is already running; await it first");
  QH_CHECK(role >= QH_ROLE_QKV && role <= QH_ROLE_HEAD, QH_ERR_INVALID, "role %d has no single decode kernel", role);
  QH_CHECK(reps >= 1, QH_ERR_INVALID, "reps must be >= 1");
  QH_CHECK(c->length < c->dev.capacity, QH_ERR_RANGE, "the cache is full");
  QH_HIP(hipSetDevice(m->ctx->device));
  hipStream_t s = m->ctx->stream;
  int rc = set_state(c, c->length, c->length + 1);
  if (rc) return rc;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  QH_HIP(hipEventCreate(&e0));
  hipError_t err = hipEventCreate(&e1);
  if (err == hipSuccess) err = qh::enqueue_role(s, m->dev, c->dev, role, 0);  // warm
  if (err == hipSuccess) err = hipEventRecord(e0, s);
  for (int r = 0; r < reps && err == hipSuccess; r++) err = qh::enqueue_role(s, m->dev, c->dev, role, r % m->dev.layers);
  if (err == hipSuccess) err = hipEventRecord(e1, s);
  if (err == hipSuccess) err = hipEventSynchronize(e1);
  float ms = 0.f;
  if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
  hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  QH_HIP(err);
  *us_per_launch = ms * 1e3f / reps;
  return QH_OK;
}

// One decode launch of `role` over copies of its operands that together exceed `min_bytes`
// (larger than the last-level cache, so every launch streams from HBM): copies of layer 0's
// matrix for the layer roles, of the output head for QH_ROLE_HEAD, of layer 0's cache for
// QH_ROLE_ATTENTION. The copies and their outputs are allocated here and freed before return.
int qh_decode_kernel_time_cold(qh_model* m, qh_cache* c, int32_t role, size_t min_bytes, int32_t reps,
                               float* us_per_launch, int32_t* copies) {
  return qh_decode_kernel_time_stream(m, c, role, min_bytes, reps, 0, us_per_launch, copies);
}

int qh_decode_kernel_time_stream(qh_model* m, qh_cache* c, int32_t role, size_t min_bytes, int32_t reps,
                                 int32_t blocks_per_copy, float* us_per_launch, int32_t* copies) {
  QH_CHECK(m && c && c->m == m && us_per_launch && copies, QH_ERR_INVALID,
           "kernel_time_cold needs a model, its cache and outputs");
  QH_CHECK(blocks_per_copy >= 0 && (blocks_per_copy == 0 || role != QH_ROLE_ATTENTION), QH_ERR_INVALID,
           "blocks_per_copy must be >= 0, and 0 for the attention (its grid is one block per slot)");
  QH_CHECK(!c->busy, QH_ERR_BUSY, "forward() is already running; await it first");
  QH_CHECK(role >= QH_ROLE_QKV && role <= QH_ROLE_HEAD, QH_ERR_INVALID, "role %d has no single decode kernel", role);
  QH_CHECK(role != QH_ROLE_ATTENTION || m->dev.numerics == QH_NUMERICS_FAST, QH_ERR_INVALID,
           "the attention list form is the fast-numerics split-K launch");
  QH_CHECK(reps >= 1 && min_bytes >= 1 && min_bytes <= ((size_t)64 << 30), QH_ERR_INVALID,
           "reps must be >= 1 and min_bytes in [1, 64 GiB]");
  QH_CHECK(c->length < c->dev.capacity, QH_ERR_RANGE, "the cache is full");
  QH_HIP(hipSetDevice(m->ctx->device));
  hipStream_t s = m->ctx->stream;
  int rc = set_state(c, c->length, c->length + 1);
  if (rc) return rc;
  const qh::ModelDev& md = m->dev;
  const qh::CacheDev& cd = c->dev;
  std::vector<void*> held;
  auto grab = [&](size_t bytes, void** p) -> hipError_t {
    hipError_t e = hipMalloc(p, bytes);
    if (e == hipSuccess) held.push_back(*p);
    return e;
  };
  auto round256 = [](size_t b) { return (b + 255) & ~(size_t)255; };
  hipError_t err = hipSuccess;
  int count = 1;
  std::function<hipError_t()> launch;
  qh::RoleList list{};
  size_t out_len = 0, ostride = 0;  // matrix roles: floats of one copy's output, and between copies
  if (role == QH_ROLE_ATTENTION) {
    const size_t elems = cd.layer_elems, stride = round256(elems * 2) / 2;
    count = (int)std::max<size_t>(1, (min_bytes + elems * 2 - 1) / (elems * 2));
    uint16_t* kv = nullptr;
    float* part = nullptr;
    err = grab((size_t)count * stride * 2, (void**)&kv);
    if (err == hipSuccess) err = grab((size_t)count * qh::attn_part_bytes(md, cd.capacity), (void**)&part);
    for (int z = 0; z < count && err == hipSuccess; z++)
      err = hipMemcpyAsync(kv + (size_t)z * stride, cd.kv, elems * 2, hipMemcpyDeviceToDevice, s);
    launch = [&, kv, part, stride]() { return qh::enqueue_attention_list(s, md, cd, kv, count, stride, part); };
  } else {
    const qh::LayerDev& l = md.layers_host[0];
    const qh::DMat& w = role == QH_ROLE_HEAD ? md.lm_head
                        : role == QH_ROLE_QKV ? l.qkv
                        : role == QH_ROLE_OPROJ ? l.o
                        : role == QH_ROLE_GATEUP ? l.gu : l.down;
    const size_t data = (size_t)w.rows * w.row_bytes;
    const size_t nscale = w.format == QH_FMT_INT4 ? (size_t)w.rows * w.gpr : w.format == QH_FMT_INT8 ? w.rows : 0;
    const size_t per = data + nscale * 4 * (w.format == QH_FMT_INT4 ? 2 : 1);
    count = (int)std::max<size_t>(1, (min_bytes + per - 1) / per);
    const size_t dstride = round256(data), sstride = round256(nscale * 4) / 4;
    out_len = role == QH_ROLE_HEAD ? md.vocab : role == QH_ROLE_GATEUP ? md.intermediate : md.hidden;
    ostride = round256(out_len * 4) / 4;
    uint8_t* d = nullptr;
    float *sc = nullptr, *zr = nullptr, *out = nullptr;
    void* partials = nullptr;
    err = grab((size_t)count * dstride, (void**)&d);
    if (err == hipSuccess && nscale) err = grab((size_t)count * sstride * 4, (void**)&sc);
    if (err == hipSuccess && w.format == QH_FMT_INT4) err = grab((size_t)count * sstride * 4, (void**)&zr);
    if (err == hipSuccess) err = grab((size_t)count * ostride * 4, (void**)&out);
    if (err == hipSuccess) err = hipMemsetAsync(out, 0, (size_t)count * ostride * 4, s);
    if (err == hipSuccess && role == QH_ROLE_HEAD) err = grab((size_t)count * qh::lm_partials_bytes(md), &partials);
    for (int z = 0; z < count && err == hipSuccess; z++) {
      err = hipMemcpyAsync(d + (size_t)z * dstride, w.data, data, hipMemcpyDeviceToDevice, s);
      if (err == hipSuccess && sc)
        err = hipMemcpyAsync(sc + (size_t)z * sstride, w.scales, nscale * 4, hipMemcpyDeviceToDevice, s);
      if (err == hipSuccess && zr)
        err = hipMemcpyAsync(zr + (size_t)z * sstride, w.zeros, nscale * 4, hipMemcpyDeviceToDevice, s);
    }
    list.w = w;
    list.w.data = d;
    list.w.scales = sc;
    list.w.zeros = zr;
    list.count = count;
    list.w_stride = dstride;
    list.s_stride = sstride;
    list.out_stride = ostride;
    list.part_stride = (size_t)qh::lm_head_blocks(md);  // argmax partial entries per copy
    list.out = out;
    list.partials = partials;
    list.max_blocks = blocks_per_copy;
    if (role == QH_ROLE_QKV && err == hipSuccess) {
      // Each copy appends its key and value rows where no other copy does, as each layer
      // appends to its own cache in the step (all copies appending to one cache would put
      // every copy's stores on the same few cache lines): copy z's key rows and value
      // entries land 64 elements (one 128-byte line) after copy z-1's, in an area shaped
      // like one layer's cache and longer by that shift. The cache itself is untouched.
      const size_t shift = 64, ke = cd.key_elems + (size_t)count * shift,
                   ve = cd.layer_elems - cd.key_elems + (size_t)count * shift;
      uint16_t* kv = nullptr;
      err = grab((ke + ve) * sizeof(uint16_t), (void**)&kv);
      if (err == hipSuccess) {
        list.kc = kv;
        list.vt = kv + ke;
        list.k_stride = shift;
        list.v_stride = shift;
      }
    }
    launch = [&]() { return qh::enqueue_role_list(s, md, cd, role, list); };
  }
  hipEvent_t e0 = nullptr, e1 = nullptr;
  if (err == hipSuccess) err = hipEventCreate(&e0);
  if (err == hipSuccess) err = hipEventCreate(&e1);
  if (err == hipSuccess) err = launch();  // warm
  if (err == hipSuccess) err = hipEventRecord(e0, s);
  for (int r = 0; r < reps && err == hipSuccess; r++) err = launch();
  if (err == hipSuccess) err = hipEventRecord(e1, s);
  if (err == hipSuccess) err = hipEventSynchronize(e1);
  float ms = 0.f;
  if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  // A streaming grid runs the loop form of the kernel, with more rows per work item for some
  // roles; each row is summed in the same order, so its outputs must equal those of the decode
  // step's own launch shape (blocks_per_copy 0) bit for bit. Checked on the first and the last
  // copy, each form launched once from zeroed outputs (the residual roles add into them).
  bool differs = false;
  if (err == hipSuccess && role != QH_ROLE_ATTENTION && blocks_per_copy > 0) {
    std::vector<float> got(2 * out_len), want(2 * out_len);
    auto run_once = [&](int max_blocks, float* host) -> hipError_t {
      list.max_blocks = max_blocks;
      hipError_t e = hipMemsetAsync(list.out, 0, (size_t)count * ostride * 4, s);
      if (e == hipSuccess) e = qh::enqueue_role_list(s, md, cd, role, list);
      if (e == hipSuccess) e = hipMemcpyAsync(host, list.out, out_len * 4, hipMemcpyDeviceToHost, s);
      if (e == hipSuccess)
        e = hipMemcpyAsync(host + out_len, list.out + (size_t)(count - 1) * ostride, out_len * 4,
                           hipMemcpyDeviceToHost, s);
      if (e == hipSuccess) e = hipStreamSynchronize(s);
      return e;
    };
    err = run_once(blocks_per_copy, got.data());
    if (err == hipSuccess) err = run_once(0, want.data());
    differs = err == hipSuccess && std::memcmp(got.data(), want.data(), got.size() * sizeof(float)) != 0;
  }
  hipStreamSynchronize(s);
  for (void* p : held) hipFree(p);
  QH_HIP(err);
  QH_CHECK(!differs, QH_ERR_STATE, "role %d: the streaming grid's outputs differ from the decode step's launch",
           role);
  *us_per_launch = ms * 1e3f / reps;
  *copies = count;
  return QH_OK;
}

int qh_decode_role(qh_model* m, qh_cache* c, int32_t role, int32_t layer, int32_t* h_token) {
  QH_CHECK(m && c && c->m == m, QH_ERR_INVALID, "decode_role needs a model and its cache");
  QH_CHECK(!c->busy, QH_ERR_BUSY, "forward() is already running; await it first");
  QH_CHECK(role >= QH_ROLE_QKV && role <= QH_ROLE_HEAD, QH_ERR_INVALID, "role %d has no single decode launch", role);
  QH_CHECK(role == QH_ROLE_HEAD || (layer >= 0 && layer < m->dev.layers), QH_ERR_RANGE, "layer %d out of range",
           layer);
  QH_CHECK(c->length < c->dev.capacity, QH_ERR_RANGE, "the cache is full");
  QH_HIP(hipSetDevice(m->ctx->device));
  hipStream_t s = m->ctx->stream;
  const int pos = c->length;
  int rc = set_state(c, pos, pos + 1);
  if (rc) return rc;
  if (role == QH_ROLE_HEAD) {
    // The head and the pick, as a step ends; the pick's gather of the next row is undone by
    // the caller rewriting x before the next role.
    QH_HIP(qh::enqueue_head(s, m->dev, c->dev));
    QH_HIP(hipMemcpyAsync(c->h_pinned + 2, c->dev.pred + pos, 4, hipMemcpyDeviceToHost, s));
  } else {
    QH_HIP(qh::enqueue_role(s, m->dev, c->dev, role, layer));
  }
  QH_HIP(hipStreamSynchronize(s));
  if (h_token) *h_token = role == QH_ROLE_HEAD ? c->h_pinned[2] : -1;
  return QH_OK;
}

int qh_cache_vector(qh_cache* c, int32_t which, int32_t layer, const float* h_in, float* h_out) {
  QH_CHECK(c, QH_ERR_INVALID, "cache_vector needs a cache");
  QH_CHECK(!c->busy, QH_ERR_BUSY, "cache has a decode in flight");
  const qh::ModelDev& md = c->m->dev;
  const qh::CacheDev& d = c->dev;
  hipStream_t s = c->m->ctx->stream;
  QH_HIP(hipSetDevice(c->m->ctx->device));
  if (which == QH_VEC_KEY || which == QH_VEC_VALUE) {
    QH_CHECK(!h_in, QH_ERR_INVALID, "the cache rows are read-only here");
    QH_CHECK(layer >= 0 && layer < md.layers, QH_ERR_RANGE, "layer %d out of range", layer);
    QH_CHECK(c->length < d.capacity, QH_ERR_RANGE, "the cache is full");
    if (!h_out) return QH_OK;
    const int pos = c->length, hd = md.head_dim;
    const uint16_t* base = d.kv + (size_t)layer * d.layer_elems;
    std::vector<uint16_t> row((size_t)md.kv_heads * hd);
    for (int h = 0; h < md.kv_heads; h++) {
      if (which == QH_VEC_KEY) {
        QH_HIP(hipMemcpyAsync(row.data() + (size_t)h * hd, base + ((size_t)h * d.capacity + pos) * hd, hd * 2,
                              hipMemcpyDeviceToHost, s));
      } else {
        // One value per dimension row of the dimension-major cache.
        QH_HIP(hipMemcpy2DAsync(row.data() + (size_t)h * hd, 2, base + d.key_elems + (size_t)h * hd * d.vstride + pos,
                                (size_t)d.vstride * 2, 2, hd, hipMemcpyDeviceToHost, s));
      }
    }
    QH_HIP(hipStreamSynchronize(s));
    for (size_t i = 0; i < row.size(); i++) h_out[i] = f16_to_f32(row[i]);
    return QH_OK;
  }
  float* dev = nullptr;
  size_t n = 0;
  switch (which) {
    case QH_VEC_X: dev = d.x, n = md.hidden; break;
    case QH_VEC_Q: dev = d.q, n = md.hidden; break;
    case QH_VEC_H: dev = d.h, n = md.intermediate; break;
    case QH_VEC_LOGITS: dev = d.logits, n = md.vocab; break;
    default: return fail(QH_ERR_INVALID, "unknown decode vector %d", which);
  }
  if (h_in) QH_HIP(hipMemcpyAsync(dev, h_in, n * 4, hipMemcpyHostToDevice, s));
  if (h_out) QH_HIP(hipMemcpyAsync(h_out, dev, n * 4, hipMemcpyDeviceToHost, s));
  QH_HIP(hipStreamSynchronize(s));
  return QH_OK;
}

int qh_decode_profile(qh_model* m, qh_cache* c, int32_t first_token, int32_t steps,
                      int32_t* h_tokens, float* h_role_ms, int32_t* h_role_launches) {
  QH_CHECK(m && c && c->m == m && h_role_ms && h_role_launches, QH_ERR_INVALID,
           "decode_profile needs a model, its cache and role outputs");
  QH_CHECK(!c->busy, QH_ERR_BUSY, "forward() is already running; await it first");
  QH_CHECK(steps >= 1, QH_ERR_INVALID, "decode needs steps >= 1");
  QH_CHECK(first_token >= 0 && first_token < m->dev.vocab, QH_ERR_RANGE,
           "token %d is outside the vocabulary", first_token);
  int rc = check_room(c, steps);
  if (rc) return rc;
  BusyGuard guard(c);
  QH_HIP(hipSetDevice(m->ctx->device));
  hipStream_t s = m->ctx->stream;
  const int n_ev = qh::launches_per_step(m->dev, qh::STEP_CARRIED) + 1;
  std::vector<hipEvent_t> ev(n_ev, nullptr);
  std::vector<int> roles(n_ev, 0);
  for (auto& e : ev) QH_HIP(hipEventCreate(&e));
  for (int r = 0; r < QH_ROLE_COUNT; r++) h_role_ms[r] = 0.f, h_role_launches[r] = 0;
  const int start = c->length;
  c->h_pinned[3] = first_token;
  hipError_t err = hipMemcpyAsync(c->dev.tokens + start, c->h_pinned + 3, 4, hipMemcpyHostToDevice, s);
  if (err == hipSuccess && (rc = set_state(c, start, start + 1))) err = hipErrorUnknown;
  // The same launches as a decode call (capture_graphs), the last step ending with its pick.
  if (err == hipSuccess) err = qh::enqueue_gather(s, m->dev, c->dev);
  for (int i = 0; i < steps && err == hipSuccess; i++) {
    qh::StepTimer t{ev.data(), roles.data(), n_ev, 0};
    err = qh::enqueue_step(s, m->dev, c->dev, i == 0 ? qh::STEP_CARRIED : qh::STEP_PICK, true, &t, i + 1 < steps);
    if (err == hipSuccess) err = hipStreamSynchronize(s);
    for (int k = 0; err == hipSuccess && k + 1 < t.n; k++) {
      float ms = 0.f;
      err = hipEventElapsedTime(&ms, ev[k], ev[k + 1]);
      h_role_ms[roles[k]] += ms;
      h_role_launches[roles[k]] += 1;
    }
  }
  if (err == hipSuccess && h_tokens) {
    err = hipMemcpyAsync(h_tokens, c->dev.pred + start, (size_t)steps * 4, hipMemcpyDeviceToHost, s);
    if (err == hipSuccess) err = hipStreamSynchronize(s);
  }
  for (auto& e : ev) hipEventDestroy(e);
  if (rc) return rc;
  QH_HIP(err);
  c->length += steps;
  return QH_OK;
}

}  // extern "C"
