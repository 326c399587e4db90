// Node-API binding of the gfx950 sampler's C ABI (include/hachiue_sampler.h).
//
// The JavaScript layer (../js/index.js) resolves SampleConfig defaults and the
// draw, then calls:
//   createContext(device)                               -> context handle
//   sampleRow(ctx, logits, vocab, history, config, u)   -> token (sync)
//   sampleBatch(ctx, logits, rows, stride, vocab, histIds, histOffsets,
//               configs, uniforms)                      -> Int32Array (sync)
//   sampleBatchAsync(...same...)                        -> Promise<Int32Array>
//   argmax(ctx, logits, rows, stride, vocab)            -> Int32Array (sync)
//   lastError()                                         -> string
// `config` / `configs` are Float64Arrays of 7 numbers per row in
// hs_sample_config field order.  Logits are Float32Arrays updated in place.
#include <node_api.h>

#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "hachiue_sampler.h"

namespace {

constexpr size_t kConfigFields = 7;

#define NAPI_OK(env, call)                                         \
  do {                                                             \
    if ((call) != napi_ok) {                                       \
      napi_throw_error((env), nullptr, "Node-API call failed: " #call); \
      return nullptr;                                              \
    }                                                              \
  } while (0)

napi_value throw_status(napi_env env, int status) {
  std::string msg = hs_last_error();
  if (msg.empty()) msg = "sampler call failed";
  if (status == HS_ERR_INVALID_ARGUMENT)
    napi_throw_range_error(env, "HS_ERR_INVALID_ARGUMENT", msg.c_str());
  else
    napi_throw_error(env, status == HS_ERR_HIP ? "HS_ERR_HIP"
                          : status == HS_ERR_OUT_OF_MEMORY ? "HS_ERR_OUT_OF_MEMORY"
                                                           : "HS_ERR_UNSUPPORTED",
                     msg.c_str());
  return nullptr;
}

void destroy_context(napi_env, void *data, void *) {
  hs_context_destroy(static_cast<hs_context *>(data));
}

bool get_ctx(napi_env env, napi_value v, hs_context **out) {
  void *p = nullptr;
  if (napi_get_value_external(env, v, &p) != napi_ok || !p) {
    napi_throw_type_error(env, nullptr, "expected a sampler context");
    return false;
  }
  *out = static_cast<hs_context *>(p);
  return true;
}

// Pointer and element count of a typed array of the given type (null -> null).
template <typename T>
bool get_typed(napi_env env, napi_value v, napi_typedarray_type want, T **data, size_t *len,
               bool allow_null, const char *what) {
  napi_valuetype vt;
  napi_typeof(env, v, &vt);
  if (allow_null && (vt == napi_null || vt == napi_undefined)) {
    *data = nullptr;
    *len = 0;
    return true;
  }
  bool is_ta = false;
  napi_is_typedarray(env, v, &is_ta);
  napi_typedarray_type type;
  void *raw = nullptr;
  size_t n = 0;
  if (!is_ta || napi_get_typedarray_info(env, v, &type, &n, &raw, nullptr, nullptr) != napi_ok ||
      type != want) {
    std::string m = std::string(what) + " has the wrong type";
    napi_throw_type_error(env, nullptr, m.c_str());
    return false;
  }
  *data = static_cast<T *>(raw);
  *len = n;
  return true;
}

bool get_double(napi_env env, napi_value v, double *out, const char *what) {
  if (napi_get_value_double(env, v, out) != napi_ok) {
    std::string m = std::string(what) + " must be a number";
    napi_throw_type_error(env, nullptr, m.c_str());
    return false;
  }
  return true;
}

bool to_config(const double *f, hs_sample_config *c) {
  c->temperature = f[0];
  c->top_k = f[1];
  c->top_p = f[2];
  c->min_p = f[3];
  c->repetition_penalty = f[4];
  c->presence_penalty = f[5];
  c->frequency_penalty = f[6];
  return true;
}

napi_value CreateContext(napi_env env, napi_callback_info info) {
  size_t argc = 1;
  napi_value argv[1];
  NAPI_OK(env, napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
  int32_t device = 0;
  if (argc >= 1) napi_get_value_int32(env, argv[0], &device);
  hs_context *ctx = nullptr;
  const int st = hs_context_create(device, &ctx);
  if (st != HS_OK) return throw_status(env, st);
  napi_value out;
  if (napi_create_external(env, ctx, destroy_context, nullptr, &out) != napi_ok) {
    hs_context_destroy(ctx);
    napi_throw_error(env, nullptr, "cannot wrap the sampler context");
    return nullptr;
  }
  return out;
}

napi_value LastError(napi_env env, napi_callback_info) {
  napi_value s;
  NAPI_OK(env, napi_create_string_utf8(env, hs_last_error(), NAPI_AUTO_LENGTH, &s));
  return s;
}

// sampleRow(ctx, logits: Float32Array, vocab, history: Int32Array, config: Float64Array(7), u)
napi_value SampleRow(napi_env env, napi_callback_info info) {
  size_t argc = 6;
  napi_value argv[6];
  NAPI_OK(env, napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
  if (argc < 6) {
    napi_throw_type_error(env, nullptr, "sampleRow needs 6 arguments");
    return nullptr;
  }
  hs_context *ctx;
  if (!get_ctx(env, argv[0], &ctx)) return nullptr;
  float *logits;
  size_t nl;
  if (!get_typed(env, argv[1], napi_float32_array, &logits, &nl, false, "logits")) return nullptr;
  int32_t vocab;
  NAPI_OK(env, napi_get_value_int32(env, argv[2], &vocab));
  int32_t *hist;
  size_t nh;
  if (!get_typed(env, argv[3], napi_int32_array, &hist, &nh, true, "history")) return nullptr;
  double *cf;
  size_t nc;
  if (!get_typed(env, argv[4], napi_float64_array, &cf, &nc, false, "config")) return nullptr;
  if (nc < kConfigFields) {
    napi_throw_range_error(env, nullptr, "config needs 7 fields");
    return nullptr;
  }
  double u;
  if (!get_double(env, argv[5], &u, "uniform")) return nullptr;
  if (vocab > 0 && (size_t)vocab > nl) {
    napi_throw_range_error(env, nullptr, "vocab exceeds the logits length");
    return nullptr;
  }
  hs_sample_config c;
  to_config(cf, &c);
  int32_t token = 0;
  const int st = hs_sample_logits(ctx, logits, vocab, hist, (int64_t)nh, &c, u, &token);
  if (st != HS_OK) return throw_status(env, st);
  napi_value out;
  NAPI_OK(env, napi_create_int32(env, token, &out));
  return out;
}

struct BatchArgs {
  hs_context *ctx = nullptr;
  float *logits = nullptr;
  int32_t rows = 0;
  int64_t stride = 0;
  int32_t vocab = 0;
  int32_t *hist = nullptr;
  std::vector<int64_t> offsets;
  std::vector<hs_sample_config> configs;
  double *uniforms = nullptr;
  int32_t *tokens = nullptr;
  napi_ref refs[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};
  int status = HS_OK;
  std::string error;
  napi_async_work work = nullptr;
  napi_deferred deferred = nullptr;
  napi_value tokens_value = nullptr;
};

// Parses sampleBatch's arguments; on failure a JS exception is pending.
bool parse_batch(napi_env env, napi_value *argv, size_t argc, BatchArgs &b,
                 napi_value *tokens_array) {
  if (argc < 9) {
    napi_throw_type_error(env, nullptr, "sampleBatch needs 9 arguments");
    return false;
  }
  if (!get_ctx(env, argv[0], &b.ctx)) return false;
  size_t nl;
  if (!get_typed(env, argv[1], napi_float32_array, &b.logits, &nl, false, "logits")) return false;
  double rows, stride, vocab;
  if (!get_double(env, argv[2], &rows, "rows") || !get_double(env, argv[3], &stride, "stride") ||
      !get_double(env, argv[4], &vocab, "vocab"))
    return false;
  b.rows = (int32_t)rows;
  b.stride = (int64_t)stride;
  b.vocab = (int32_t)vocab;
  if (b.rows < 0 || (b.rows > 0 && b.vocab > 0 &&
                     (size_t)((int64_t)(b.rows - 1) * b.stride + b.vocab) > nl)) {
    napi_throw_range_error(env, nullptr, "logits shorter than rows * stride");
    return false;
  }
  size_t nh, no;
  double *off;
  if (!get_typed(env, argv[5], napi_int32_array, &b.hist, &nh, true, "histIds")) return false;
  if (!get_typed(env, argv[6], napi_float64_array, &off, &no, true, "histOffsets")) return false;
  if ((b.hist == nullptr) != (off == nullptr) || (off && no != (size_t)b.rows + 1)) {
    napi_throw_range_error(env, nullptr, "histOffsets needs rows + 1 entries");
    return false;
  }
  if (off) {
    b.offsets.resize(no);
    for (size_t i = 0; i < no; ++i) {
      b.offsets[i] = (int64_t)off[i];
      if (b.offsets[i] < 0 || (size_t)b.offsets[i] > nh) {
        napi_throw_range_error(env, nullptr, "histOffsets out of range");
        return false;
      }
    }
  }
  double *cf;
  size_t nc;
  if (!get_typed(env, argv[7], napi_float64_array, &cf, &nc, false, "configs")) return false;
  if (nc < kConfigFields * (size_t)b.rows) {
    napi_throw_range_error(env, nullptr, "configs needs 7 numbers per row");
    return false;
  }
  b.configs.resize((size_t)b.rows);
  for (int32_t r = 0; r < b.rows; ++r) to_config(cf + kConfigFields * r, &b.configs[(size_t)r]);
  size_t nu;
  if (!get_typed(env, argv[8], napi_float64_array, &b.uniforms, &nu, false, "uniforms")) return false;
  if (nu < (size_t)b.rows) {
    napi_throw_range_error(env, nullptr, "uniforms needs one number per row");
    return false;
  }
  napi_value ab;
  void *tok = nullptr;
  if (napi_create_arraybuffer(env, sizeof(int32_t) * (size_t)(b.rows > 0 ? b.rows : 1), &tok, &ab) !=
          napi_ok ||
      napi_create_typedarray(env, napi_int32_array, (size_t)b.rows, ab, 0, tokens_array) != napi_ok) {
    napi_throw_error(env, nullptr, "cannot allocate the token array");
    return false;
  }
  b.tokens = static_cast<int32_t *>(tok);
  return true;
}

int run_batch(BatchArgs &b) {
  const int st = hs_sample_logits_batch(b.ctx, b.logits, b.rows, b.stride, b.vocab, b.hist,
                                        b.offsets.empty() ? nullptr : b.offsets.data(),
                                        b.configs.data(), b.uniforms, b.tokens);
  if (st != HS_OK) b.error = hs_last_error();
  return st;
}

napi_value SampleBatch(napi_env env, napi_callback_info info) {
  size_t argc = 9;
  napi_value argv[9];
  NAPI_OK(env, napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
  BatchArgs b;
  napi_value tokens;
  if (!parse_batch(env, argv, argc, b, &tokens)) return nullptr;
  const int st = run_batch(b);
  if (st != HS_OK) return throw_status(env, st);
  return tokens;
}

void batch_execute(napi_env, void *data) {
  BatchArgs *b = static_cast<BatchArgs *>(data);
  b->status = run_batch(*b);
}

void batch_complete(napi_env env, napi_status, void *data) {
  BatchArgs *b = static_cast<BatchArgs *>(data);
  if (b->status == HS_OK) {
    napi_value t;
    napi_get_reference_value(env, b->refs[4], &t);
    napi_resolve_deferred(env, b->deferred, t);
  } else {
    napi_value msg, err;
    napi_create_string_utf8(env, b->error.c_str(), NAPI_AUTO_LENGTH, &msg);
    napi_create_error(env, nullptr, msg, &err);
    napi_reject_deferred(env, b->deferred, err);
  }
  for (napi_ref &r : b->refs)
    if (r) napi_delete_reference(env, r);
  napi_delete_async_work(env, b->work);
  delete b;
}

// The context, logits, histories, uniforms and token array stay referenced
// until the work completes; the context must not be used meanwhile.
napi_value SampleBatchAsync(napi_env env, napi_callback_info info) {
  size_t argc = 9;
  napi_value argv[9];
  NAPI_OK(env, napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
  BatchArgs *b = new BatchArgs();
  napi_value tokens;
  if (!parse_batch(env, argv, argc, *b, &tokens)) {
    delete b;
    return nullptr;
  }
  napi_value promise, name;
  napi_create_reference(env, argv[0], 1, &b->refs[0]);
  napi_create_reference(env, argv[1], 1, &b->refs[1]);
  napi_valuetype vt;
  napi_typeof(env, argv[5], &vt);
  if (vt != napi_null && vt != napi_undefined) napi_create_reference(env, argv[5], 1, &b->refs[2]);
  napi_create_reference(env, argv[8], 1, &b->refs[3]);
  napi_create_reference(env, tokens, 1, &b->refs[4]);
  napi_create_promise(env, &b->deferred, &promise);
  napi_create_string_utf8(env, "hachiue_sample_batch", NAPI_AUTO_LENGTH, &name);
  if (napi_create_async_work(env, nullptr, name, batch_execute, batch_complete, b, &b->work) !=
          napi_ok ||
      napi_queue_async_work(env, b->work) != napi_ok) {
    napi_throw_error(env, nullptr, "cannot queue the sampling work");
    return nullptr;
  }
  return promise;
}

// argmax(ctx, logits: Float32Array, rows, stride, vocab): the engine's GPU
// greedy route (the WGSL argmax of src/kernels.ts:1613-1654); logits are
// read only.
napi_value Argmax(napi_env env, napi_callback_info info) {
  size_t argc = 5;
  napi_value argv[5];
  NAPI_OK(env, napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr));
  if (argc < 5) {
    napi_throw_type_error(env, nullptr, "argmax needs 5 arguments");
    return nullptr;
  }
  hs_context *ctx;
  if (!get_ctx(env, argv[0], &ctx)) return nullptr;
  float *logits;
  size_t nl;
  if (!get_typed(env, argv[1], napi_float32_array, &logits, &nl, false, "logits")) return nullptr;
  double rows_d, stride_d, vocab_d;
  if (!get_double(env, argv[2], &rows_d, "rows") || !get_double(env, argv[3], &stride_d, "stride") ||
      !get_double(env, argv[4], &vocab_d, "vocab"))
    return nullptr;
  const int32_t rows = (int32_t)rows_d, vocab = (int32_t)vocab_d;
  const int64_t stride = (int64_t)stride_d;
  if (rows < 0 || (rows > 0 && vocab > 0 && (size_t)((int64_t)(rows - 1) * stride + vocab) > nl)) {
    napi_throw_range_error(env, nullptr, "logits shorter than rows * stride");
    return nullptr;
  }
  napi_value ab, tokens;
  void *tok = nullptr;
  if (napi_create_arraybuffer(env, sizeof(int32_t) * (size_t)(rows > 0 ? rows : 1), &tok, &ab) !=
          napi_ok ||
      napi_create_typedarray(env, napi_int32_array, (size_t)rows, ab, 0, &tokens) != napi_ok) {
    napi_throw_error(env, nullptr, "cannot allocate the token array");
    return nullptr;
  }
  const int st = hs_argmax(ctx, logits, rows, stride, vocab, static_cast<int32_t *>(tok));
  if (st != HS_OK) return throw_status(env, st);
  return tokens;
}

napi_value Init(napi_env env, napi_value exports) {
  napi_property_descriptor props[] = {
      {"createContext", nullptr, CreateContext, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"sampleRow", nullptr, SampleRow, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"sampleBatch", nullptr, SampleBatch, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"sampleBatchAsync", nullptr, SampleBatchAsync, nullptr, nullptr, nullptr, napi_enumerable,
       nullptr},
      {"argmax", nullptr, Argmax, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"lastError", nullptr, LastError, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
  };
  napi_define_properties(env, exports, sizeof(props) / sizeof(props[0]), props);
  napi_value v;
  napi_create_int32(env, hs_abi_version(), &v);
  napi_set_named_property(env, exports, "abiVersion", v);
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
