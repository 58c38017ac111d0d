/* Node-API addon over the libnemo C ABI (include/nemo.h): the native half of
 * the JavaScript host (js/runtime.js), replacing the WebGPU calls of
 * src/webgpu/model.ts and src/webgpu/device.ts.
 *
 * Handles are externals wrapping a pointer. planRun executes nemo_plan_run on
 * the libuv thread pool (napi_async_work) and settles a Promise, like
 * EmbeddingPlan.run (src/webgpu/embedding-engine.ts:8); distinct plans may
 * run concurrently, runs of one plan are serialised by libnemo. A plan handle
 * counts its runs in flight: planDestroy closes it to new calls at once
 * (they throw 'plan was destroyed') and frees the plan when the last run has
 * settled, on the JS thread, so a pending run resolves normally (WebGPU's
 * destroy() is likewise safe with work already queued,
 * src/webgpu/model.ts:141-144). Every failure becomes a JS Error carrying
 * nemo_last_error(). */
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/nemo.h"

#define CHECK_NAPI(env, call)                                                 \
  do {                                                                        \
    if ((call) != napi_ok) {                                                  \
      napi_throw_error((env), NULL, "node-api call failed: " #call);          \
      return NULL;                                                            \
    }                                                                         \
  } while (0)

typedef struct {
  void* ptr;
  int kind;    /* 1 ctx, 2 model, 3 plan */
  int pending; /* plan runs queued or executing (touched on the JS thread only) */
  int closed;  /* planDestroy was called; the plan is freed once pending is 0 */
} handle_t;

static const char* kKindName[] = {"", "context", "model", "plan"};

static void handle_finalize(napi_env env, void* data, void* hint) {
  (void)env;
  (void)hint;
  free(data); /* the wrapper only; resources are released by destroy() */
}

static napi_value wrap(napi_env env, void* ptr, int kind) {
  handle_t* h = (handle_t*)malloc(sizeof(handle_t));
  napi_value out;
  if (!h) {
    napi_throw_error(env, NULL, "out of host memory");
    return NULL;
  }
  h->ptr = ptr;
  h->kind = kind;
  h->pending = 0;
  h->closed = 0;
  if (napi_create_external(env, h, handle_finalize, NULL, &out) != napi_ok) {
    free(h);
    napi_throw_error(env, NULL, "cannot create handle");
    return NULL;
  }
  return out;
}

static handle_t* unwrap(napi_env env, napi_value v, int kind) {
  handle_t* h = NULL;
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok || t != napi_external || napi_get_value_external(env, v, (void**)&h) != napi_ok ||
      !h || h->kind != kind) {
    char msg[64];
    snprintf(msg, sizeof msg, "expected a %s handle", kKindName[kind]);
    napi_throw_type_error(env, NULL, msg);
    return NULL;
  }
  if (!h->ptr || h->closed) {
    char msg[64];
    snprintf(msg, sizeof msg, "%s was destroyed", kKindName[kind]);
    napi_throw_error(env, NULL, msg);
    return NULL;
  }
  return h;
}

static napi_value throw_status(napi_env env, nemo_status s) {
  napi_value err, msg, code;
  const char* text = nemo_last_error();
  napi_create_string_utf8(env, text && *text ? text : "libnemo call failed", NAPI_AUTO_LENGTH, &msg);
  napi_create_error(env, NULL, msg, &err);
  napi_create_int32(env, s, &code);
  napi_set_named_property(env, err, "status", code);
  napi_throw(env, err);
  return NULL;
}

static int get_args(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, NULL, NULL) != napi_ok || argc < want) {
    napi_throw_type_error(env, NULL, "wrong number of arguments");
    return 0;
  }
  return 1;
}

static int get_i32(napi_env env, napi_value v, int32_t* out) {
  if (napi_get_value_int32(env, v, out) != napi_ok) {
    napi_throw_type_error(env, NULL, "expected a number");
    return 0;
  }
  return 1;
}

/* A typed array, DataView-free ArrayBuffer or Buffer: base pointer and bytes. */
static int get_bytes(napi_env env, napi_value v, void** data, size_t* n) {
  bool is;
  if (napi_is_typedarray(env, v, &is) == napi_ok && is) {
    napi_typedarray_type type;
    size_t length, offset;
    napi_value ab;
    if (napi_get_typedarray_info(env, v, &type, &length, data, &ab, &offset) != napi_ok) return 0;
    size_t elem = 1;
    switch (type) {
      case napi_int16_array: case napi_uint16_array: elem = 2; break;
      case napi_int32_array: case napi_uint32_array: case napi_float32_array: elem = 4; break;
      case napi_float64_array: elem = 8; break;
      default: elem = 1;
    }
    *n = length * elem;
    return 1;
  }
  if (napi_is_arraybuffer(env, v, &is) == napi_ok && is) return napi_get_arraybuffer_info(env, v, data, n) == napi_ok;
  if (napi_is_buffer(env, v, &is) == napi_ok && is) return napi_get_buffer_info(env, v, data, n) == napi_ok;
  napi_throw_type_error(env, NULL, "expected a typed array, ArrayBuffer or Buffer");
  return 0;
}

static int get_u32_array(napi_env env, napi_value v, const uint32_t** data, size_t* count) {
  bool is;
  napi_typedarray_type type;
  size_t length, offset;
  void* p;
  napi_value ab;
  if (napi_is_typedarray(env, v, &is) != napi_ok || !is ||
      napi_get_typedarray_info(env, v, &type, &length, &p, &ab, &offset) != napi_ok || type != napi_uint32_array) {
    napi_throw_type_error(env, NULL, "expected a Uint32Array");
    return 0;
  }
  *data = (const uint32_t*)p;
  *count = length;
  return 1;
}

/* ---- plain calls ---------------------------------------------------------- */

static napi_value js_version(napi_env env, napi_callback_info info) {
  napi_value out;
  (void)info;
  CHECK_NAPI(env, napi_create_string_utf8(env, nemo_version(), NAPI_AUTO_LENGTH, &out));
  return out;
}

static const char* kDimNames[] = {"hidden", "qHeads", "kvHeads", "headDim", "intermediate", "layers",
                                  "vocab", "mergeAfterLayer", "rmsEpsilon", "ropeTheta", "kvStrideThreshold",
                                  "kvStride", "kvDenseBeforeMerge"};

static napi_value dims_to_js(napi_env env, const nemo_dims* d) {
  napi_value o, v;
  const int32_t iv[] = {d->hidden, d->q_heads, d->kv_heads, d->head_dim, d->intermediate, d->layers,
                        d->vocab, d->merge_after_layer};
  CHECK_NAPI(env, napi_create_object(env, &o));
  for (int i = 0; i < 8; ++i) {
    CHECK_NAPI(env, napi_create_int32(env, iv[i], &v));
    CHECK_NAPI(env, napi_set_named_property(env, o, kDimNames[i], v));
  }
  CHECK_NAPI(env, napi_create_double(env, d->rms_epsilon, &v));
  CHECK_NAPI(env, napi_set_named_property(env, o, kDimNames[8], v));
  CHECK_NAPI(env, napi_create_double(env, d->rope_theta, &v));
  CHECK_NAPI(env, napi_set_named_property(env, o, kDimNames[9], v));
  CHECK_NAPI(env, napi_create_int32(env, d->kv_stride_threshold, &v));
  CHECK_NAPI(env, napi_set_named_property(env, o, kDimNames[10], v));
  CHECK_NAPI(env, napi_create_int32(env, d->kv_stride, &v));
  CHECK_NAPI(env, napi_set_named_property(env, o, kDimNames[11], v));
  CHECK_NAPI(env, napi_create_int32(env, d->kv_dense_before_merge, &v));
  CHECK_NAPI(env, napi_set_named_property(env, o, kDimNames[12], v));
  return o;
}

/* Every field must be present (the JS side fills defaults). */
static int dims_from_js(napi_env env, napi_value o, nemo_dims* d) {
  int32_t* iv[] = {&d->hidden, &d->q_heads, &d->kv_heads, &d->head_dim, &d->intermediate, &d->layers,
                   &d->vocab, &d->merge_after_layer};
  napi_value v;
  double x;
  for (int i = 0; i < 13; ++i) {
    if (napi_get_named_property(env, o, kDimNames[i], &v) != napi_ok || napi_get_value_double(env, v, &x) != napi_ok) {
      char msg[80];
      snprintf(msg, sizeof msg, "dims.%s must be a number", kDimNames[i]);
      napi_throw_type_error(env, NULL, msg);
      return 0;
    }
    if (i < 8) *iv[i] = (int32_t)x;
    else if (i == 8) d->rms_epsilon = (float)x;
    else if (i == 9) d->rope_theta = (float)x;
    else if (i == 10) d->kv_stride_threshold = (int32_t)x;
    else if (i == 11) d->kv_stride = (int32_t)x;
    else d->kv_dense_before_merge = (int32_t)x;
  }
  return 1;
}

static napi_value js_dims_reference(napi_env env, napi_callback_info info) {
  nemo_dims d;
  (void)info;
  nemo_dims_reference(&d);
  return dims_to_js(env, &d);
}

static napi_value js_stage_names(napi_env env, napi_callback_info info) {
  napi_value arr, s;
  (void)info;
  const int32_t n = nemo_profile_stage_count();
  CHECK_NAPI(env, napi_create_array_with_length(env, (size_t)n, &arr));
  for (int32_t i = 0; i < n; ++i) {
    CHECK_NAPI(env, napi_create_string_utf8(env, nemo_profile_stage_name(i), NAPI_AUTO_LENGTH, &s));
    CHECK_NAPI(env, napi_set_element(env, arr, (uint32_t)i, s));
  }
  return arr;
}

static napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

static napi_value js_init(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  int32_t device;
  nemo_ctx* ctx = NULL;
  if (!get_args(env, info, 1, argv) || !get_i32(env, argv[0], &device)) return NULL;
  nemo_status s = nemo_init(device, &ctx);
  if (s) return throw_status(env, s);
  return wrap(env, ctx, 1);
}

static napi_value js_shutdown(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  handle_t* h = unwrap(env, argv[0], 1);
  if (!h) return NULL;
  nemo_status s = nemo_shutdown((nemo_ctx*)h->ptr);
  h->ptr = NULL;
  if (s) return throw_status(env, s);
  return undefined(env);
}

static napi_value js_model_create(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  nemo_dims d;
  nemo_model* m = NULL;
  if (!get_args(env, info, 2, argv)) return NULL;
  handle_t* h = unwrap(env, argv[0], 1);
  if (!h || !dims_from_js(env, argv[1], &d)) return NULL;
  nemo_status s = nemo_model_create((nemo_ctx*)h->ptr, &d, &m);
  if (s) return throw_status(env, s);
  return wrap(env, m, 2);
}

static napi_value js_model_set_tensor(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  char name[256];
  size_t name_len;
  int32_t type;
  uint32_t n_dims;
  int64_t dims[4];
  void* data;
  size_t n;
  if (!get_args(env, info, 5, argv)) return NULL;
  handle_t* h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  if (napi_get_value_string_utf8(env, argv[1], name, sizeof name, &name_len) != napi_ok) {
    napi_throw_type_error(env, NULL, "tensor name must be a string");
    return NULL;
  }
  if (!get_i32(env, argv[2], &type)) return NULL;
  if (napi_get_array_length(env, argv[3], &n_dims) != napi_ok || n_dims < 1 || n_dims > 4) {
    napi_throw_type_error(env, NULL, "dimensions must be an array of 1 to 4 numbers");
    return NULL;
  }
  for (uint32_t i = 0; i < n_dims; ++i) {
    napi_value e;
    double x;
    if (napi_get_element(env, argv[3], i, &e) != napi_ok || napi_get_value_double(env, e, &x) != napi_ok) {
      napi_throw_type_error(env, NULL, "dimensions must be numbers");
      return NULL;
    }
    dims[i] = (int64_t)x;
  }
  if (!get_bytes(env, argv[4], &data, &n)) return NULL;
  nemo_status s = nemo_model_set_tensor((nemo_model*)h->ptr, name, type, dims, (int32_t)n_dims, data, n);
  if (s) return throw_status(env, s);
  return undefined(env);
}

static napi_value js_model_synthesize(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  double seed;
  int32_t emb;
  if (!get_args(env, info, 3, argv)) return NULL;
  handle_t* h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  if (napi_get_value_double(env, argv[1], &seed) != napi_ok || !get_i32(env, argv[2], &emb)) {
    napi_throw_type_error(env, NULL, "expected (model, seed, embeddingType)");
    return NULL;
  }
  nemo_status s = nemo_model_synthesize((nemo_model*)h->ptr, (uint64_t)seed, emb);
  if (s) return throw_status(env, s);
  return undefined(env);
}

static napi_value js_model_finalize(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  handle_t* h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  nemo_status s = nemo_model_finalize((nemo_model*)h->ptr);
  if (s) return throw_status(env, s);
  return undefined(env);
}

static napi_value js_model_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  handle_t* h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  nemo_status s = nemo_model_destroy((nemo_model*)h->ptr);
  h->ptr = NULL;
  if (s) return throw_status(env, s);
  return undefined(env);
}

static napi_value js_plan_create(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  int32_t batch, seq;
  nemo_plan* p = NULL;
  if (!get_args(env, info, 3, argv)) return NULL;
  handle_t* h = unwrap(env, argv[0], 2);
  if (!h || !get_i32(env, argv[1], &batch) || !get_i32(env, argv[2], &seq)) return NULL;
  nemo_status s = nemo_plan_create((nemo_model*)h->ptr, batch, seq, &p);
  if (s) return throw_status(env, s);
  return wrap(env, p, 3);
}

static napi_value js_plan_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  handle_t* h = unwrap(env, argv[0], 3);
  if (!h) return NULL;
  h->closed = 1;
  if (h->pending > 0) return undefined(env); /* freed by the last run_complete */
  nemo_status s = nemo_plan_destroy((nemo_plan*)h->ptr);
  h->ptr = NULL;
  if (s) return throw_status(env, s);
  return undefined(env);
}

/* ---- planRun: async ------------------------------------------------------- */

typedef struct {
  napi_async_work work;
  napi_deferred deferred;
  napi_ref plan_ref; /* keeps the plan handle alive while the work runs */
  handle_t* handle;
  nemo_plan* plan;
  uint32_t* ids;
  size_t n_ids;
  uint32_t* lengths;
  size_t n_lengths;
  float* out;
  size_t n_out;
  nemo_status status;
  char error[512];
} run_job_t;

static void run_execute(napi_env env, void* data) {
  run_job_t* j = (run_job_t*)data;
  (void)env;
  j->status = nemo_plan_run(j->plan, j->ids, j->n_ids, j->lengths, j->n_lengths, j->out);
  if (j->status) {
    /* nemo_last_error is per thread: read it on the thread that failed. */
    strncpy(j->error, nemo_last_error(), sizeof j->error - 1);
    j->error[sizeof j->error - 1] = 0;
  }
}

static void run_complete(napi_env env, napi_status status, void* data) {
  run_job_t* j = (run_job_t*)data;
  napi_value result;
  if (status != napi_ok || j->status) {
    napi_value err, msg, code;
    napi_create_string_utf8(env, status != napi_ok ? "plan run was cancelled" : j->error, NAPI_AUTO_LENGTH, &msg);
    napi_create_error(env, NULL, msg, &err);
    napi_create_int32(env, j->status, &code);
    napi_set_named_property(env, err, "status", code);
    napi_reject_deferred(env, j->deferred, err);
  } else {
    void* buf = NULL;
    napi_value ab;
    if (napi_create_arraybuffer(env, j->n_out * sizeof(float), &buf, &ab) == napi_ok) {
      memcpy(buf, j->out, j->n_out * sizeof(float));
      napi_create_typedarray(env, napi_float32_array, j->n_out, ab, 0, &result);
      napi_resolve_deferred(env, j->deferred, result);
    } else {
      napi_value err, msg;
      napi_create_string_utf8(env, "cannot allocate the embeddings", NAPI_AUTO_LENGTH, &msg);
      napi_create_error(env, NULL, msg, &err);
      napi_reject_deferred(env, j->deferred, err);
    }
  }
  /* On the JS thread, before the handle may be collected: a destroy that
   * arrived while runs were in flight frees the plan after the last. */
  handle_t* h = j->handle;
  if (--h->pending == 0 && h->closed && h->ptr) {
    (void)nemo_plan_destroy((nemo_plan*)h->ptr);
    h->ptr = NULL;
  }
  napi_delete_reference(env, j->plan_ref);
  napi_delete_async_work(env, j->work);
  free(j->ids);
  free(j->lengths);
  free(j->out);
  free(j);
}

/* planRun(plan, ids: Uint32Array, lengths: Uint32Array) ->
 * Promise<Float32Array(batch * hidden)>, batch and hidden taken from the
 * native plan (nemo_plan_shape). ids and lengths are copied at the call, as
 * the reference writes them into its buffers (model.ts:149-151). */
static napi_value js_plan_run(napi_env env, napi_callback_info info) {
  napi_value argv[3], promise, name;
  const uint32_t *ids, *lengths;
  size_t n_ids, n_lengths;
  int32_t batch = 0, hidden = 0;
  if (!get_args(env, info, 3, argv)) return NULL;
  handle_t* h = unwrap(env, argv[0], 3);
  if (!h || !get_u32_array(env, argv[1], &ids, &n_ids) || !get_u32_array(env, argv[2], &lengths, &n_lengths))
    return NULL;
  nemo_status st = nemo_plan_shape((nemo_plan*)h->ptr, &batch, NULL, &hidden);
  if (st) return throw_status(env, st);
  run_job_t* j = (run_job_t*)calloc(1, sizeof(run_job_t));
  if (!j) {
    napi_throw_error(env, NULL, "out of host memory");
    return NULL;
  }
  j->handle = h;
  j->plan = (nemo_plan*)h->ptr;
  j->n_ids = n_ids;
  j->n_lengths = n_lengths;
  j->n_out = (size_t)batch * (size_t)hidden;
  j->ids = (uint32_t*)malloc(n_ids * 4 + 4);
  j->lengths = (uint32_t*)malloc(n_lengths * 4 + 4);
  j->out = (float*)malloc(j->n_out * 4 + 4);
  if (!j->ids || !j->lengths || !j->out) {
    free(j->ids);
    free(j->lengths);
    free(j->out);
    free(j);
    napi_throw_error(env, NULL, "out of host memory");
    return NULL;
  }
  memcpy(j->ids, ids, n_ids * 4);
  memcpy(j->lengths, lengths, n_lengths * 4);
  CHECK_NAPI(env, napi_create_reference(env, argv[0], 1, &j->plan_ref));
  CHECK_NAPI(env, napi_create_promise(env, &j->deferred, &promise));
  CHECK_NAPI(env, napi_create_string_utf8(env, "nemo_plan_run", NAPI_AUTO_LENGTH, &name));
  CHECK_NAPI(env, napi_create_async_work(env, NULL, name, run_execute, run_complete, j, &j->work));
  CHECK_NAPI(env, napi_queue_async_work(env, j->work));
  h->pending++;
  return promise;
}

/* planProfile(plan, ids, lengths) -> { stageName: ms } (blocking). */
static napi_value js_plan_profile(napi_env env, napi_callback_info info) {
  napi_value argv[3], o, v;
  const uint32_t *ids, *lengths;
  size_t n_ids, n_lengths;
  float ms[32];
  if (!get_args(env, info, 3, argv)) return NULL;
  handle_t* h = unwrap(env, argv[0], 3);
  if (!h || !get_u32_array(env, argv[1], &ids, &n_ids) || !get_u32_array(env, argv[2], &lengths, &n_lengths))
    return NULL;
  const int32_t n = nemo_profile_stage_count();
  nemo_status s = nemo_plan_profile((nemo_plan*)h->ptr, ids, n_ids, lengths, n_lengths, ms, n < 32 ? n : 32);
  if (s) return throw_status(env, s);
  CHECK_NAPI(env, napi_create_object(env, &o));
  for (int32_t i = 0; i < n && i < 32; ++i) {
    CHECK_NAPI(env, napi_create_double(env, ms[i], &v));
    CHECK_NAPI(env, napi_set_named_property(env, o, nemo_profile_stage_name(i), v));
  }
  return o;
}

/* requantizeQ40(ctx, srcType, bytes, k, n) -> Uint8Array of n * k / 32
 * GGUF Q4_0 blocks (requantizeMatrixToQ40, src/gguf/quantization.ts:101-131,
 * on the GPU). Blocking. */
static napi_value js_requantize_q40(napi_env env, napi_callback_info info) {
  napi_value argv[5], ab, out;
  int32_t type;
  double kd, nd;
  void* src;
  size_t n_src;
  if (!get_args(env, info, 5, argv)) return NULL;
  handle_t* h = unwrap(env, argv[0], 1);
  if (!h || !get_i32(env, argv[1], &type) || !get_bytes(env, argv[2], &src, &n_src)) return NULL;
  if (napi_get_value_double(env, argv[3], &kd) != napi_ok || napi_get_value_double(env, argv[4], &nd) != napi_ok) {
    napi_throw_type_error(env, NULL, "k and n must be numbers");
    return NULL;
  }
  const int64_t k = (int64_t)kd, n = (int64_t)nd;
  const size_t need = k > 0 && n > 0 ? (size_t)n * (size_t)(k / 32) * 18 : 0;
  void* dst = NULL;
  CHECK_NAPI(env, napi_create_arraybuffer(env, need ? need : 1, &dst, &ab));
  nemo_status s = nemo_requantize_q40((nemo_ctx*)h->ptr, type, src, n_src, k, n, dst, need);
  if (s) return throw_status(env, s);
  CHECK_NAPI(env, napi_create_typedarray(env, napi_uint8_array, need, ab, 0, &out));
  return out;
}

static napi_value module_init(napi_env env, napi_value exports) {
  const napi_property_descriptor props[] = {
      {"version", NULL, js_version, NULL, NULL, NULL, napi_enumerable, NULL},
      {"dimsReference", NULL, js_dims_reference, NULL, NULL, NULL, napi_enumerable, NULL},
      {"profileStageNames", NULL, js_stage_names, NULL, NULL, NULL, napi_enumerable, NULL},
      {"init", NULL, js_init, NULL, NULL, NULL, napi_enumerable, NULL},
      {"shutdown", NULL, js_shutdown, NULL, NULL, NULL, napi_enumerable, NULL},
      {"modelCreate", NULL, js_model_create, NULL, NULL, NULL, napi_enumerable, NULL},
      {"modelSetTensor", NULL, js_model_set_tensor, NULL, NULL, NULL, napi_enumerable, NULL},
      {"modelSynthesize", NULL, js_model_synthesize, NULL, NULL, NULL, napi_enumerable, NULL},
      {"modelFinalize", NULL, js_model_finalize, NULL, NULL, NULL, napi_enumerable, NULL},
      {"modelDestroy", NULL, js_model_destroy, NULL, NULL, NULL, napi_enumerable, NULL},
      {"planCreate", NULL, js_plan_create, NULL, NULL, NULL, napi_enumerable, NULL},
      {"planRun", NULL, js_plan_run, NULL, NULL, NULL, napi_enumerable, NULL},
      {"planProfile", NULL, js_plan_profile, NULL, NULL, NULL, napi_enumerable, NULL},
      {"planDestroy", NULL, js_plan_destroy, NULL, NULL, NULL, napi_enumerable, NULL},
      {"requantizeQ40", NULL, js_requantize_q40, NULL, NULL, NULL, napi_enumerable, NULL},
  };
  if (napi_define_properties(env, exports, sizeof props / sizeof props[0], props) != napi_ok) return NULL;
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, module_init)
