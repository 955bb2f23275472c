// Node-API binding of libqwen_hip.so: argument marshalling only. Every function
// takes and returns plain JS values and typed arrays, calls one C-ABI entry
// point, and turns a non-zero status into a thrown Error (RangeError for
// QH_ERR_RANGE, as the reference throws for capacity and rope bounds,
// src/gpu/model.js:249-254) carrying qh_last_error()'s message. Handles are
// napi externals; the JS driver (../gpu_model.js) owns their lifetime.
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "qwen_hip.h"

namespace {

#define NAPI_OK(call)                                         \
  do {                                                        \
    if ((call) != napi_ok) {                                  \
      napi_throw_error(env, nullptr, "node-api call failed"); \
      return nullptr;                                         \
    }                                                         \
  } while (0)

napi_value fail(napi_env env, int rc) {
  const char* msg = qh_last_error();
  std::string code = "QH_ERR_" + std::to_string(rc);
  if (rc == QH_ERR_RANGE) napi_throw_range_error(env, code.c_str(), msg);
  else napi_throw_error(env, code.c_str(), msg);
  return nullptr;
}

#define QH_CALL(expr)              \
  do {                             \
    int rc_ = (expr);              \
    if (rc_ != QH_OK) return fail(env, rc_); \
  } while (0)

struct Args {
  napi_value v[12];
  size_t n = 12;
};

bool get_args(napi_env env, napi_callback_info info, Args& a, size_t need) {
  if (napi_get_cb_info(env, info, &a.n, a.v, nullptr, nullptr) != napi_ok || a.n < need) {
    napi_throw_type_error(env, nullptr, "missing arguments");
    return false;
  }
  return true;
}

bool to_i32(napi_env env, napi_value v, int32_t* out) {
  if (napi_get_value_int32(env, v, out) != napi_ok) {
    napi_throw_type_error(env, nullptr, "expected a number");
    return false;
  }
  return true;
}

bool to_f64(napi_env env, napi_value v, double* out) {
  if (napi_get_value_double(env, v, out) != napi_ok) {
    napi_throw_type_error(env, nullptr, "expected a number");
    return false;
  }
  return true;
}

bool to_str(napi_env env, napi_value v, std::string* out) {
  size_t len = 0;
  if (napi_get_value_string_utf8(env, v, nullptr, 0, &len) != napi_ok) {
    napi_throw_type_error(env, nullptr, "expected a string");
    return false;
  }
  out->resize(len + 1);
  napi_get_value_string_utf8(env, v, &(*out)[0], len + 1, &len);
  out->resize(len);
  return true;
}

const char* type_name(napi_typedarray_type t) {
  switch (t) {
    case napi_int8_array: return "Int8Array";
    case napi_uint8_array: return "Uint8Array";
    case napi_uint16_array: return "Uint16Array";
    case napi_int32_array: return "Int32Array";
    case napi_float32_array: return "Float32Array";
    default: return "a typed array";
  }
}

// A typed array of exactly the element type `want` holding at least `need` elements; with
// `optional`, null / undefined give nullptr. Anything else throws (TypeError for the wrong
// kind of value, RangeError for too few elements), so no C entry point reads past a caller's
// array.
bool to_array(napi_env env, napi_value v, napi_typedarray_type want, const char* what, size_t need, bool optional,
              void** data) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (optional && (t == napi_null || t == napi_undefined)) {
    *data = nullptr;
    return true;
  }
  bool is_ta = false;
  napi_is_typedarray(env, v, &is_ta);
  napi_typedarray_type type = napi_int8_array;
  size_t length = 0, offset = 0;
  napi_value ab;
  if (is_ta) napi_get_typedarray_info(env, v, &type, &length, data, &ab, &offset);
  if (!is_ta || type != want) {
    const std::string msg = std::string(what) + " must be a " + type_name(want);
    napi_throw_type_error(env, nullptr, msg.c_str());
    return false;
  }
  if (length < need) {
    const std::string msg = std::string(what) + " holds " + std::to_string(length) + " values where " +
                            std::to_string(need) + " are needed";
    napi_throw_range_error(env, nullptr, msg.c_str());
    return false;
  }
  return true;
}

bool positive(napi_env env, int32_t rows, int32_t cols) {
  if (rows >= 1 && cols >= 1) return true;
  napi_throw_range_error(env, nullptr, "rows and cols must be positive");
  return false;
}

template <typename T>
bool to_handle(napi_env env, napi_value v, T** out) {
  void* p = nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "expected a live handle");
    return false;
  }
  *out = static_cast<T*>(p);
  return true;
}

napi_value external(napi_env env, void* p) {
  napi_value v;
  napi_create_external(env, p, nullptr, nullptr, &v);
  return v;
}

napi_value typed(napi_env env, napi_typedarray_type type, size_t count, size_t el, void** data) {
  napi_value ab, ta;
  if (napi_create_arraybuffer(env, count * el, data, &ab) != napi_ok) return nullptr;
  napi_create_typedarray(env, type, count, ab, 0, &ta);
  return ta;
}

napi_value num(napi_env env, double d) {
  napi_value v;
  napi_create_double(env, d, &v);
  return v;
}

// ------------------------------------------------------------------ context
napi_value Open(napi_env env, napi_callback_info info) {
  Args a;
  int32_t dev = 0;
  if (!get_args(env, info, a, 1) || !to_i32(env, a.v[0], &dev)) return nullptr;
  qh_ctx* c = nullptr;
  QH_CALL(qh_open(dev, &c));
  return external(env, c);
}

napi_value Close(napi_env env, napi_callback_info info) {
  Args a;
  qh_ctx* c;
  if (!get_args(env, info, a, 1) || !to_handle(env, a.v[0], &c)) return nullptr;
  QH_CALL(qh_close(c));
  return nullptr;
}

napi_value Describe(napi_env env, napi_callback_info info) {
  Args a;
  qh_ctx* c;
  if (!get_args(env, info, a, 1) || !to_handle(env, a.v[0], &c)) return nullptr;
  char buf[1024];
  QH_CALL(qh_describe(c, buf, sizeof buf));
  napi_value s;
  napi_create_string_utf8(env, buf, NAPI_AUTO_LENGTH, &s);
  return s;
}

// ------------------------------------------------------------- host helpers
napi_value SynthBf16(napi_env env, napi_callback_info info) {  // (seed, name, std, n)
  Args a;
  double seed, std_, n;
  std::string name;
  if (!get_args(env, info, a, 4) || !to_f64(env, a.v[0], &seed) || !to_str(env, a.v[1], &name) ||
      !to_f64(env, a.v[2], &std_) || !to_f64(env, a.v[3], &n))
    return nullptr;
  void* d;
  napi_value out = typed(env, napi_uint16_array, (size_t)n, 2, &d);
  QH_CALL(qh_synth_bf16((uint64_t)seed, name.c_str(), std_, 0, (size_t)n, static_cast<uint16_t*>(d)));
  return out;
}

napi_value SynthTokens(napi_env env, napi_callback_info info) {  // (seed, name, vocab, n)
  Args a;
  double seed;
  int32_t vocab, n;
  std::string name;
  if (!get_args(env, info, a, 4) || !to_f64(env, a.v[0], &seed) || !to_str(env, a.v[1], &name) ||
      !to_i32(env, a.v[2], &vocab) || !to_i32(env, a.v[3], &n))
    return nullptr;
  void* d;
  napi_value out = typed(env, napi_int32_array, (size_t)n, 4, &d);
  QH_CALL(qh_synth_tokens((uint64_t)seed, name.c_str(), vocab, (size_t)n, static_cast<int32_t*>(d)));
  return out;
}

napi_value QuantizeInt8(napi_env env, napi_callback_info info) {  // (Float32Array, rows, cols)
  Args a;
  void* w;
  int32_t rows, cols;
  if (!get_args(env, info, a, 3) || !to_i32(env, a.v[1], &rows) || !to_i32(env, a.v[2], &cols) ||
      !positive(env, rows, cols) ||
      !to_array(env, a.v[0], napi_float32_array, "weights", (size_t)rows * cols, false, &w))
    return nullptr;
  void *q, *s;
  napi_value tq = typed(env, napi_int8_array, (size_t)rows * cols, 1, &q);
  napi_value ts = typed(env, napi_float32_array, (size_t)rows, 4, &s);
  QH_CALL(qh_quantize_int8(static_cast<const float*>(w), rows, cols, static_cast<int8_t*>(q),
                           static_cast<float*>(s)));
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "q", tq);
  napi_set_named_property(env, o, "scales", ts);
  return o;
}

napi_value QuantizeInt4(napi_env env, napi_callback_info info) {  // (Float32Array, rows, cols, group)
  Args a;
  void* w;
  int32_t rows, cols, group;
  if (!get_args(env, info, a, 4) || !to_i32(env, a.v[1], &rows) || !to_i32(env, a.v[2], &cols) ||
      !to_i32(env, a.v[3], &group) || !positive(env, rows, cols) ||
      !to_array(env, a.v[0], napi_float32_array, "weights", (size_t)rows * cols, false, &w))
    return nullptr;
  if (group < 2 || cols % group) return fail(env, qh_quantize_int4(nullptr, rows, cols, group, nullptr, nullptr, nullptr));
  const size_t ng = (size_t)rows * (cols / group);
  void *q, *s, *z;
  napi_value tq = typed(env, napi_uint8_array, (size_t)rows * cols / 2, 1, &q);
  napi_value ts = typed(env, napi_float32_array, ng, 4, &s);
  napi_value tz = typed(env, napi_float32_array, ng, 4, &z);
  QH_CALL(qh_quantize_int4(static_cast<const float*>(w), rows, cols, group, static_cast<uint8_t*>(q),
                           static_cast<float*>(s), static_cast<float*>(z)));
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "q", tq);
  napi_set_named_property(env, o, "scales", ts);
  napi_set_named_property(env, o, "zeros", tz);
  return o;
}

// -------------------------------------------------------------------- model
bool prop_i32(napi_env env, napi_value o, const char* k, int32_t* out) {
  napi_value v;
  return napi_get_named_property(env, o, k, &v) == napi_ok && to_i32(env, v, out);
}
bool prop_f64(napi_env env, napi_value o, const char* k, double* out) {
  napi_value v;
  return napi_get_named_property(env, o, k, &v) == napi_ok && to_f64(env, v, out);
}

napi_value ModelCreate(napi_env env, napi_callback_info info) {  // (ctx, config)
  Args a;
  qh_ctx* c;
  if (!get_args(env, info, a, 2) || !to_handle(env, a.v[0], &c)) return nullptr;
  qh_config cfg{};
  napi_value o = a.v[1];
  if (!prop_i32(env, o, "hidden", &cfg.hidden) || !prop_i32(env, o, "intermediate", &cfg.intermediate) ||
      !prop_i32(env, o, "layers", &cfg.layers) || !prop_i32(env, o, "heads", &cfg.heads) ||
      !prop_i32(env, o, "kvHeads", &cfg.kv_heads) || !prop_i32(env, o, "headDim", &cfg.head_dim) ||
      !prop_i32(env, o, "vocab", &cfg.vocab) || !prop_f64(env, o, "ropeTheta", &cfg.rope_theta) ||
      !prop_f64(env, o, "eps", &cfg.eps) || !prop_i32(env, o, "maxPositions", &cfg.max_positions))
    return nullptr;
  qh_model* m = nullptr;
  QH_CALL(qh_model_create(c, &cfg, &m));
  return external(env, m);
}

napi_value ModelSetMode(napi_env env, napi_callback_info info) {  // (model, 'numerics'|'matmul', value)
  Args a;
  qh_model* m;
  std::string which;
  int32_t v;
  if (!get_args(env, info, a, 3) || !to_handle(env, a.v[0], &m) || !to_str(env, a.v[1], &which) ||
      !to_i32(env, a.v[2], &v))
    return nullptr;
  QH_CALL(which == "numerics" ? qh_model_set_numerics(m, v) : qh_model_set_matmul(m, v));
  return nullptr;
}

// (model, name, format, rows, cols, group, data, scales|null, zeros|null)
napi_value ModelSetTensor(napi_env env, napi_callback_info info) {
  Args a;
  qh_model* m;
  std::string name;
  int32_t fmt, rows, cols, group;
  void *data, *scales, *zeros;
  if (!get_args(env, info, a, 9) || !to_handle(env, a.v[0], &m) || !to_str(env, a.v[1], &name) ||
      !to_i32(env, a.v[2], &fmt) || !to_i32(env, a.v[3], &rows) || !to_i32(env, a.v[4], &cols) ||
      !to_i32(env, a.v[5], &group) || !positive(env, rows, cols))
    return nullptr;
  // The arrays each format stores (qh_model_set_tensor): codes or values, then scales and
  // zero points. An int4 group that does not divide the row is the C call's error to report.
  const size_t n = (size_t)rows * cols;
  const bool grouped = fmt == QH_FMT_INT4 && group > 0 && cols % group == 0;
  const size_t groups = grouped ? (size_t)rows * (cols / group) : 0;
  bool ok = true;
  switch (fmt) {
    case QH_FMT_F32:
      ok = to_array(env, a.v[6], napi_float32_array, "data", n, false, &data);
      scales = zeros = nullptr;
      break;
    case QH_FMT_F16:
    case QH_FMT_BF16:
      ok = to_array(env, a.v[6], napi_uint16_array, "data", n, false, &data);
      scales = zeros = nullptr;
      break;
    case QH_FMT_INT8:
      ok = to_array(env, a.v[6], napi_int8_array, "codes", n, false, &data) &&
           to_array(env, a.v[7], napi_float32_array, "scales", (size_t)rows, false, &scales);
      zeros = nullptr;
      break;
    case QH_FMT_INT4:
      ok = to_array(env, a.v[6], napi_uint8_array, "codes", (n + 1) / 2, false, &data) &&
           to_array(env, a.v[7], napi_float32_array, "scales", groups, false, &scales) &&
           to_array(env, a.v[8], napi_float32_array, "zeros", groups, false, &zeros);
      break;
    default:
      data = scales = zeros = nullptr;  // an unknown format: the C call reports it
  }
  if (!ok) return nullptr;
  QH_CALL(qh_model_set_tensor(m, name.c_str(), fmt, rows, cols, group, data, static_cast<const float*>(scales),
                              static_cast<const float*>(zeros)));
  return nullptr;
}

// (model, name, srcFormat, rows, cols, data, format, group): the checkpoint's values converted
// on the device.
napi_value ModelLoadTensor(napi_env env, napi_callback_info info) {
  Args a;
  qh_model* m;
  std::string name;
  int32_t src_fmt, rows, cols, fmt, group;
  void* data;
  if (!get_args(env, info, a, 8) || !to_handle(env, a.v[0], &m) || !to_str(env, a.v[1], &name) ||
      !to_i32(env, a.v[2], &src_fmt) || !to_i32(env, a.v[3], &rows) || !to_i32(env, a.v[4], &cols) ||
      !to_i32(env, a.v[6], &fmt) || !to_i32(env, a.v[7], &group) || !positive(env, rows, cols))
    return nullptr;
  // bf16 checkpoints arrive as their bits, f32 ones as values
  const napi_typedarray_type want = src_fmt == QH_FMT_BF16 || src_fmt == QH_FMT_F16 ? napi_uint16_array
                                                                                   : napi_float32_array;
  if (!to_array(env, a.v[5], want, "data", (size_t)rows * cols, false, &data)) return nullptr;
  QH_CALL(qh_model_load_tensor(m, name.c_str(), src_fmt, rows, cols, data, fmt, group));
  return nullptr;
}

napi_value ModelFinalize(napi_env env, napi_callback_info info) {
  Args a;
  qh_model* m;
  if (!get_args(env, info, a, 1) || !to_handle(env, a.v[0], &m)) return nullptr;
  QH_CALL(qh_model_finalize(m));
  size_t bytes = 0;
  QH_CALL(qh_model_bytes(m, &bytes));
  return num(env, (double)bytes);
}

napi_value ModelFree(napi_env env, napi_callback_info info) {
  Args a;
  qh_model* m;
  if (!get_args(env, info, a, 1) || !to_handle(env, a.v[0], &m)) return nullptr;
  QH_CALL(qh_model_free(m));
  return nullptr;
}

napi_value CacheCreate(napi_env env, napi_callback_info info) {  // (model, capacity)
  Args a;
  qh_model* m;
  int32_t cap;
  if (!get_args(env, info, a, 2) || !to_handle(env, a.v[0], &m) || !to_i32(env, a.v[1], &cap)) return nullptr;
  qh_cache* c = nullptr;
  QH_CALL(qh_cache_create(m, cap, &c));
  return external(env, c);
}

napi_value CacheFree(napi_env env, napi_callback_info info) {
  Args a;
  qh_cache* c;
  if (!get_args(env, info, a, 1) || !to_handle(env, a.v[0], &c)) return nullptr;
  QH_CALL(qh_cache_free(c));
  return nullptr;
}

napi_value CacheLength(napi_env env, napi_callback_info info) {  // (cache[, newLength])
  Args a;
  qh_cache* c;
  if (!get_args(env, info, a, 1) || !to_handle(env, a.v[0], &c)) return nullptr;
  if (a.n >= 2) {
    int32_t len;
    if (!to_i32(env, a.v[1], &len)) return nullptr;
    QH_CALL(qh_cache_set_length(c, len));
  }
  int32_t len = 0;
  QH_CALL(qh_cache_length(c, &len));
  return num(env, len);
}

// (model, cache, Int32Array ids | Float32Array hidden [seq * hidden], seq, wantLogits) ->
// {logits, argmax}; the logits array has the model's vocabulary size.
napi_value Forward(napi_env env, napi_callback_info info) {
  Args a;
  qh_model* m;
  qh_cache* c;
  void* in;
  int32_t seq;
  bool want = true;
  if (!get_args(env, info, a, 5) || !to_handle(env, a.v[0], &m) || !to_handle(env, a.v[1], &c) ||
      !to_i32(env, a.v[3], &seq))
    return nullptr;
  napi_get_value_bool(env, a.v[4], &want);
  qh_config cfg{};
  QH_CALL(qh_model_config(m, &cfg));
  bool is_ta = false;
  napi_typedarray_type type = napi_float32_array;
  napi_is_typedarray(env, a.v[2], &is_ta);
  if (is_ta) {
    size_t len, off;
    napi_value ab;
    napi_get_typedarray_info(env, a.v[2], &type, &len, &in, &ab, &off);
  }
  const size_t rows = seq > 0 ? (size_t)seq : 0;
  if (type == napi_int32_array) {
    if (!to_array(env, a.v[2], napi_int32_array, "token ids", rows, false, &in)) return nullptr;
  } else if (!to_array(env, a.v[2], napi_float32_array, "hidden", rows * cfg.hidden, false, &in)) {
    return nullptr;
  }
  void* lp = nullptr;
  napi_value logits = nullptr;
  if (want) logits = typed(env, napi_float32_array, (size_t)cfg.vocab, 4, &lp);
  int32_t am = -1;
  if (type == napi_int32_array) {
    QH_CALL(qh_forward_tokens(m, c, static_cast<const int32_t*>(in), seq, static_cast<float*>(lp),
                              want ? &am : nullptr));
  } else {
    QH_CALL(qh_forward(m, c, static_cast<const float*>(in), seq, static_cast<float*>(lp), want ? &am : nullptr));
  }
  napi_value o, nul;
  napi_get_null(env, &nul);
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "logits", want ? logits : nul);
  napi_set_named_property(env, o, "argmax", want ? num(env, am) : nul);
  return o;
}

// (model, cache, Int32Array ids) -> Float64Array of ids.length - 1 negative log-likelihoods
// (qh_score: ids[t + 1] under the step that feeds ids[t], web/perplexity.html:146-170).
napi_value Score(napi_env env, napi_callback_info info) {
  Args a;
  qh_model* m;
  qh_cache* c;
  if (!get_args(env, info, a, 3) || !to_handle(env, a.v[0], &m) || !to_handle(env, a.v[1], &c)) return nullptr;
  bool is_ta = false;
  napi_is_typedarray(env, a.v[2], &is_ta);
  size_t n = 0;
  if (is_ta) {
    napi_typedarray_type type;
    void* data;
    napi_value ab;
    size_t off;
    napi_get_typedarray_info(env, a.v[2], &type, &n, &data, &ab, &off);
  }
  void* ids = nullptr;
  if (!to_array(env, a.v[2], napi_int32_array, "token ids", n, false, &ids)) return nullptr;
  void* out_data = nullptr;
  napi_value out = typed(env, napi_float64_array, n > 1 ? n - 1 : 0, 8, &out_data);
  QH_CALL(qh_score(m, c, static_cast<const int32_t*>(ids), (int32_t)n, static_cast<double*>(out_data)));
  return out;
}

napi_value Decode(napi_env env, napi_callback_info info) {  // (model, cache, firstToken, steps) -> Int32Array
  Args a;
  qh_model* m;
  qh_cache* c;
  int32_t first, steps;
  if (!get_args(env, info, a, 4) || !to_handle(env, a.v[0], &m) || !to_handle(env, a.v[1], &c) ||
      !to_i32(env, a.v[2], &first) || !to_i32(env, a.v[3], &steps))
    return nullptr;
  void* d;
  napi_value out = typed(env, napi_int32_array, (size_t)(steps > 0 ? steps : 0), 4, &d);
  QH_CALL(qh_decode(m, c, first, steps, static_cast<int32_t*>(d)));
  return out;
}

// (model, cache, layer) -> {key, value}: layer `layer`'s cache rows 0 .. length-1 as f32
// [kv_heads, length, head_dim] (qh_cache_present).
napi_value CachePresent(napi_env env, napi_callback_info info) {
  Args a;
  qh_model* m;
  qh_cache* c;
  int32_t layer, len = 0;
  if (!get_args(env, info, a, 3) || !to_handle(env, a.v[0], &m) || !to_handle(env, a.v[1], &c) ||
      !to_i32(env, a.v[2], &layer))
    return nullptr;
  qh_config cfg{};
  QH_CALL(qh_model_config(m, &cfg));
  QH_CALL(qh_cache_length(c, &len));
  const size_t n = (size_t)cfg.kv_heads * len * cfg.head_dim;
  void *k, *v;
  napi_value tk = typed(env, napi_float32_array, n, 4, &k);
  napi_value tv = typed(env, napi_float32_array, n, 4, &v);
  QH_CALL(qh_cache_present(c, layer, static_cast<float*>(k), static_cast<float*>(v)));
  napi_value o;
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "key", tk);
  napi_set_named_property(env, o, "value", tv);
  return o;
}

napi_value AbiVersion(napi_env env, napi_callback_info) { return num(env, qh_abi_version()); }

}  // namespace

static napi_value Init(napi_env env, napi_value exports) {
  const struct {
    const char* name;
    napi_callback fn;
  } fns[] = {{"abiVersion", AbiVersion},   {"open", Open},
             {"close", Close},             {"describe", Describe},
             {"synthBf16", SynthBf16},     {"synthTokens", SynthTokens},
             {"quantizeInt8", QuantizeInt8}, {"quantizeInt4", QuantizeInt4},
             {"modelCreate", ModelCreate}, {"modelSetMode", ModelSetMode},
             {"modelSetTensor", ModelSetTensor}, {"modelLoadTensor", ModelLoadTensor},
             {"modelFinalize", ModelFinalize},
             {"modelFree", ModelFree},     {"cacheCreate", CacheCreate},
             {"cacheFree", CacheFree},     {"cacheLength", CacheLength},
             {"cachePresent", CachePresent},
             {"forward", Forward},         {"decode", Decode},
             {"score", Score}};
  for (const auto& f : fns) {
    napi_value v;
    napi_create_function(env, f.name, NAPI_AUTO_LENGTH, f.fn, nullptr, &v);
    napi_set_named_property(env, exports, f.name, v);
  }
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
