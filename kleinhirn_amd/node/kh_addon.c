/*
 * kh_addon.node: Node-API binding of libkh_hip.so (include/kh_hip.h) for hip-backend.ts.
 *
 * Plain N-API C (no C++ wrapper, no node-gyp): every function maps one C-ABI entry point, takes
 * typed arrays as borrowed memory (the library copies what it keeps before returning) and throws a
 * JS Error carrying kh_last_error() when a call fails. Handles are napi externals; destroying them
 * twice is harmless. readOutputAsync waits for the device on a libuv worker thread and resolves a
 * Promise<Float32Array>, so the JS thread stays free while a forward runs, like the reference's
 * mapAsync readback (src/plan/executor.ts:395-408).
 */
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/kh_hip.h"

#define CHECK_NAPI(env, call)                                        \
  do {                                                               \
    if ((call) != napi_ok) {                                         \
      napi_throw_error((env), NULL, "kh_addon: N-API call failed"); \
      return NULL;                                                   \
    }                                                                \
  } while (0)

static napi_value throw_kh(napi_env env, int rc) {
  char msg[1024];
  snprintf(msg, sizeof msg, "kh status %d: %s", rc, kh_last_error());
  napi_throw_error(env, NULL, msg);
  return NULL;
}

typedef struct {
  void *ptr;
  int kind; /* 1 ctx, 2 plan, 3 scheduler */
} handle;

static void finalize_handle(napi_env env, void *data, void *hint) {
  (void)env;
  (void)hint;
  handle *h = (handle *)data;
  /* explicit destroy() is the contract; a garbage-collected handle frees its native object */
  if (h->ptr) {
    if (h->kind == 2) kh_plan_destroy((kh_plan *)h->ptr);
    else if (h->kind == 3) kh_sched_destroy((kh_sched *)h->ptr);
    else kh_ctx_destroy((kh_ctx *)h->ptr);
  }
  free(h);
}

static napi_value wrap(napi_env env, void *ptr, int kind) {
  handle *h = (handle *)malloc(sizeof(handle));
  h->ptr = ptr;
  h->kind = kind;
  napi_value v;
  CHECK_NAPI(env, napi_create_external(env, h, finalize_handle, NULL, &v));
  return v;
}

static handle *unwrap(napi_env env, napi_value v, int kind) {
  void *data = NULL;
  if (napi_get_value_external(env, v, &data) != napi_ok || !data || ((handle *)data)->kind != kind) {
    napi_throw_type_error(env, NULL, kind == 2   ? "expected a plan handle"
                                     : kind == 3 ? "expected a scheduler handle"
                                                 : "expected a context handle");
    return NULL;
  }
  return (handle *)data;
}

static int get_args(napi_env env, napi_callback_info info, size_t want, napi_value *argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, NULL, NULL) != napi_ok) return 0;
  for (size_t i = argc; i < want; i++) napi_get_undefined(env, &argv[i]);
  return 1;
}

/* bytes of a TypedArray / ArrayBuffer, or (NULL, 0) for null / undefined */
static int get_bytes(napi_env env, napi_value v, void **data, size_t *bytes) {
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_null || t == napi_undefined) {
    *data = NULL;
    *bytes = 0;
    return 1;
  }
  bool is_ta = false, is_ab = false;
  napi_is_typedarray(env, v, &is_ta);
  if (is_ta) {
    napi_typedarray_type tt;
    size_t len, off;
    napi_value ab;
    void *base;
    if (napi_get_typedarray_info(env, v, &tt, &len, &base, &ab, &off) != napi_ok) return 0;
    size_t el = (tt == napi_int8_array || tt == napi_uint8_array || tt == napi_uint8_clamped_array) ? 1
                : (tt == napi_int16_array || tt == napi_uint16_array) ? 2
                : (tt == napi_float64_array || tt == napi_bigint64_array || tt == napi_biguint64_array) ? 8 : 4;
    *data = base;
    *bytes = len * el;
    return 1;
  }
  napi_is_arraybuffer(env, v, &is_ab);
  if (is_ab) return napi_get_arraybuffer_info(env, v, data, bytes) == napi_ok;
  return 0;
}

static char *get_string(napi_env env, napi_value v, size_t *len) {
  size_t n = 0;
  if (napi_get_value_string_utf8(env, v, NULL, 0, &n) != napi_ok) return NULL;
  char *s = (char *)malloc(n + 1);
  napi_get_value_string_utf8(env, v, s, n + 1, &n);
  if (len) *len = n;
  return s;
}

static napi_value ctx_create(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  int32_t device = 0;
  napi_valuetype t;
  napi_typeof(env, argv[0], &t);
  if (t == napi_number) napi_get_value_int32(env, argv[0], &device);
  kh_ctx *ctx = NULL;
  int rc = kh_ctx_create(device, &ctx);
  if (rc) return throw_kh(env, rc);
  return wrap(env, ctx, 1);
}

static napi_value destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  void *data = NULL;
  if (napi_get_value_external(env, argv[0], &data) != napi_ok || !data) {
    napi_throw_type_error(env, NULL, "expected a handle");
    return NULL;
  }
  handle *h = (handle *)data;
  int rc = 0;
  if (h->ptr)
    rc = h->kind == 2   ? kh_plan_destroy((kh_plan *)h->ptr)
         : h->kind == 3 ? kh_sched_destroy((kh_sched *)h->ptr)
                        : kh_ctx_destroy((kh_ctx *)h->ptr);
  h->ptr = NULL;
  if (rc) return throw_kh(env, rc);
  return NULL;
}

/* weightAdd(ctx, name, dtype, shape: number[], data: TypedArray) */
static napi_value weight_add(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (!get_args(env, info, 5, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 1);
  if (!h) return NULL;
  char *name = get_string(env, argv[1], NULL);
  int32_t dtype = 0;
  napi_get_value_int32(env, argv[2], &dtype);
  uint32_t nd = 0;
  napi_get_array_length(env, argv[3], &nd);
  if (nd > 8) {
    free(name);
    napi_throw_range_error(env, NULL, "shape has more than 8 dimensions");
    return NULL;
  }
  int64_t shape[8];
  for (uint32_t i = 0; i < nd; i++) {
    napi_value e;
    napi_get_element(env, argv[3], i, &e);
    napi_get_value_int64(env, e, &shape[i]);
  }
  void *data;
  size_t bytes;
  if (!get_bytes(env, argv[4], &data, &bytes)) {
    free(name);
    napi_throw_type_error(env, NULL, "weight data must be a TypedArray or ArrayBuffer");
    return NULL;
  }
  int rc = kh_weight_add((kh_ctx *)h->ptr, name, dtype, shape, (int)nd, data, bytes);
  free(name);
  if (rc) return throw_kh(env, rc);
  return NULL;
}

static napi_value weight_bytes(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 1);
  if (!h) return NULL;
  uint64_t b = 0;
  int rc = kh_ctx_weight_bytes((kh_ctx *)h->ptr, &b);
  if (rc) return throw_kh(env, rc);
  napi_value v;
  napi_create_double(env, (double)b, &v);
  return v;
}

/* wordsSet(ctx, dtype, rows, width, data) */
static napi_value words_set(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  if (!get_args(env, info, 5, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 1);
  if (!h) return NULL;
  int32_t dtype = 0;
  int64_t rows = 0, width = 0;
  napi_get_value_int32(env, argv[1], &dtype);
  napi_get_value_int64(env, argv[2], &rows);
  napi_get_value_int64(env, argv[3], &width);
  void *data;
  size_t bytes;
  if (!get_bytes(env, argv[4], &data, &bytes)) {
    napi_throw_type_error(env, NULL, "word table must be a TypedArray");
    return NULL;
  }
  int rc = kh_words_set((kh_ctx *)h->ptr, dtype, rows, width, data, bytes);
  if (rc) return throw_kh(env, rc);
  return NULL;
}

/* planCheck(ctx | null, json) */
static napi_value plan_check(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  napi_valuetype t;
  napi_typeof(env, argv[0], &t);
  kh_ctx *ctx = NULL;
  if (t != napi_null && t != napi_undefined) {
    handle *h = unwrap(env, argv[0], 1);
    if (!h) return NULL;
    ctx = (kh_ctx *)h->ptr;
  }
  size_t n = 0;
  char *json = get_string(env, argv[1], &n);
  int rc = kh_plan_check(ctx, json, n);
  free(json);
  if (rc) return throw_kh(env, rc);
  return NULL;
}

static napi_value plan_create(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 1);
  if (!h) return NULL;
  size_t n = 0;
  char *json = get_string(env, argv[1], &n);
  kh_plan *plan = NULL;
  int rc = kh_plan_create((kh_ctx *)h->ptr, json, n, &plan);
  free(json);
  if (rc) return throw_kh(env, rc);
  return wrap(env, plan, 2);
}

static napi_value plan_init_buffer(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  char *id = get_string(env, argv[1], NULL);
  void *data;
  size_t bytes;
  if (!get_bytes(env, argv[2], &data, &bytes)) {
    free(id);
    napi_throw_type_error(env, NULL, "init data must be a TypedArray");
    return NULL;
  }
  int rc = kh_plan_init_buffer((kh_plan *)h->ptr, id, data, bytes);
  free(id);
  if (rc) return throw_kh(env, rc);
  return NULL;
}

static napi_value plan_info(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  kh_plan_info pi;
  int rc = kh_plan_info_get((kh_plan *)h->ptr, &pi);
  if (rc) return throw_kh(env, rc);
  napi_value o, v;
  napi_create_object(env, &o);
#define SET(name, val)                   \
  napi_create_double(env, (double)(val), &v); \
  napi_set_named_property(env, o, name, v);
  SET("length", pi.length);
  SET("batch", pi.batch);
  SET("markers", pi.markers);
  SET("f16", pi.f16);
  SET("bytes", pi.bytes);
  SET("outRows", pi.out_rows);
  SET("outCols", pi.out_cols);
  SET("launches", pi.launches);
  SET("streams", pi.streams);
#undef SET
  return o;
}

/* upload(plan, embeddings, mask: Float32Array, typeIds: Uint32Array | null) */
static napi_value upload(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!get_args(env, info, 4, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  void *emb, *mask, *tt;
  size_t eb, mb, tb;
  if (!get_bytes(env, argv[1], &emb, &eb) || !get_bytes(env, argv[2], &mask, &mb) || !get_bytes(env, argv[3], &tt, &tb)) {
    napi_throw_type_error(env, NULL, "upload takes TypedArrays");
    return NULL;
  }
  int rc = kh_upload((kh_plan *)h->ptr, emb, eb, (const float *)mask, mb / 4, (const uint32_t *)tt, tb / 4);
  if (rc) return throw_kh(env, rc);
  return NULL;
}

/* uploadIds(plan, ids: Int32Array, mask: Float32Array, typeIds: Uint32Array | null) */
static napi_value upload_ids(napi_env env, napi_callback_info info) {
  napi_value argv[4];
  if (!get_args(env, info, 4, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  void *ids, *mask, *tt;
  size_t ib, mb, tb;
  if (!get_bytes(env, argv[1], &ids, &ib) || !get_bytes(env, argv[2], &mask, &mb) || !get_bytes(env, argv[3], &tt, &tb)) {
    napi_throw_type_error(env, NULL, "uploadIds takes TypedArrays");
    return NULL;
  }
  int rc = kh_upload_ids((kh_plan *)h->ptr, (const int32_t *)ids, ib / 4, (const float *)mask, mb / 4,
                         (const uint32_t *)tt, tb / 4);
  if (rc) return throw_kh(env, rc);
  return NULL;
}

/* uploadMarkers(plan, packed: Uint32Array): RunInput.packedMarkers of a marker head */
static napi_value upload_markers(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  void *pk;
  size_t pb;
  if (!get_bytes(env, argv[1], &pk, &pb)) {
    napi_throw_type_error(env, NULL, "uploadMarkers takes a Uint32Array");
    return NULL;
  }
  int rc = kh_upload_markers((kh_plan *)h->ptr, (const uint32_t *)pk, pb / 4);
  if (rc) return throw_kh(env, rc);
  return NULL;
}

/* uploadQtypes(plan, qtype: Uint32Array): RunInput.qtype of a rowSelect (Julia) plan */
static napi_value upload_qtypes(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  void *q;
  size_t qb;
  if (!get_bytes(env, argv[1], &q, &qb)) {
    napi_throw_type_error(env, NULL, "uploadQtypes takes a Uint32Array");
    return NULL;
  }
  int rc = kh_upload_qtypes((kh_plan *)h->ptr, (const uint32_t *)q, qb / 4);
  if (rc) return throw_kh(env, rc);
  return NULL;
}

static napi_value run(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  int32_t rows = 0;
  napi_get_value_int32(env, argv[1], &rows);
  int rc = kh_run((kh_plan *)h->ptr, rows);
  if (rc) return throw_kh(env, rc);
  return NULL;
}

static napi_value read_output(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  kh_plan_info pi;
  int rc = kh_plan_info_get((kh_plan *)h->ptr, &pi);
  if (rc) return throw_kh(env, rc);
  size_t n = (size_t)pi.out_rows * (size_t)pi.out_cols;
  napi_value ab, out;
  void *data;
  CHECK_NAPI(env, napi_create_arraybuffer(env, n * 4, &data, &ab));
  rc = kh_read_output((kh_plan *)h->ptr, (float *)data, n);
  if (rc) return throw_kh(env, rc);
  CHECK_NAPI(env, napi_create_typedarray(env, napi_float32_array, n, ab, 0, &out));
  return out;
}

typedef struct {
  napi_async_work work;
  napi_deferred deferred;
  napi_ref plan_ref;
  kh_plan *plan;
  float *out;
  size_t n;
  int rc;
  char err[1024];
} read_job;

static void read_execute(napi_env env, void *data) {
  (void)env;
  read_job *j = (read_job *)data;
  j->rc = kh_read_output(j->plan, j->out, j->n);
  if (j->rc) snprintf(j->err, sizeof j->err, "kh status %d: %s", j->rc, kh_last_error());
}

static void read_complete(napi_env env, napi_status status, void *data) {
  read_job *j = (read_job *)data;
  if (status == napi_ok && j->rc == 0) {
    napi_value ab, out;
    void *buf;
    napi_create_arraybuffer(env, j->n * 4, &buf, &ab);
    memcpy(buf, j->out, j->n * 4);
    napi_create_typedarray(env, napi_float32_array, j->n, ab, 0, &out);
    napi_resolve_deferred(env, j->deferred, out);
  } else {
    napi_value msg, err;
    napi_create_string_utf8(env, j->rc ? j->err : "kh_addon: async read failed", NAPI_AUTO_LENGTH, &msg);
    napi_create_error(env, NULL, msg, &err);
    napi_reject_deferred(env, j->deferred, err);
  }
  napi_delete_reference(env, j->plan_ref);
  napi_delete_async_work(env, j->work);
  free(j->out);
  free(j);
}

static napi_value read_output_async(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  kh_plan_info pi;
  int rc = kh_plan_info_get((kh_plan *)h->ptr, &pi);
  if (rc) return throw_kh(env, rc);
  read_job *j = (read_job *)calloc(1, sizeof(read_job));
  j->plan = (kh_plan *)h->ptr;
  j->n = (size_t)pi.out_rows * (size_t)pi.out_cols;
  j->out = (float *)malloc(j->n * 4 + 4);
  napi_value promise, name;
  CHECK_NAPI(env, napi_create_promise(env, &j->deferred, &promise));
  napi_create_reference(env, argv[0], 1, &j->plan_ref);  /* keeps the plan alive while reading */
  napi_create_string_utf8(env, "kh_read_output", NAPI_AUTO_LENGTH, &name);
  CHECK_NAPI(env, napi_create_async_work(env, NULL, name, read_execute, read_complete, j, &j->work));
  CHECK_NAPI(env, napi_queue_async_work(env, j->work));
  return promise;
}

static napi_value last_run_ms(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 2);
  if (!h) return NULL;
  float ms = 0;
  int rc = kh_last_run_ms((kh_plan *)h->ptr, &ms);
  if (rc) return throw_kh(env, rc);
  napi_value v;
  napi_create_double(env, ms, &v);
  return v;
}

static napi_value manifest_info_object(napi_env env, const kh_manifest_info *mi) {
  napi_value o, v;
  napi_create_object(env, &o);
#define SET(name, val)                        \
  napi_create_double(env, (double)(val), &v); \
  napi_set_named_property(env, o, name, v);
  SET("version", mi->version);
  SET("tensors", mi->tensors);
  SET("shards", mi->shards);
  SET("wordsDtype", mi->words_dtype);
  SET("wordsRows", mi->words_rows);
  SET("wordsWidth", mi->words_width);
  SET("tensorBytes", mi->tensor_bytes);
  SET("fileBytes", mi->file_bytes);
  SET("readMs", mi->read_ms);
  SET("sha256Ms", mi->sha256_ms);
  SET("rowsMs", mi->rows_ms);
  SET("uploadMs", mi->upload_ms);
#undef SET
  return o;
}

/* manifestCheck(path: string, flags?: number) -> info (no device) */
static napi_value manifest_check(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  if (!get_args(env, info, 2, argv)) return NULL;
  int32_t flags = 0;
  napi_valuetype t;
  napi_typeof(env, argv[1], &t);
  if (t == napi_number) napi_get_value_int32(env, argv[1], &flags);
  char *path = get_string(env, argv[0], NULL);
  if (!path) return NULL;
  kh_manifest_info mi;
  int rc = kh_manifest_check(path, flags, &mi);
  free(path);
  if (rc) return throw_kh(env, rc);
  return manifest_info_object(env, &mi);
}

/* loadManifest(ctx, path: string, flags?: number) -> info */
static napi_value load_manifest(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 1);
  if (!h) return NULL;
  int32_t flags = 0;
  napi_valuetype t;
  napi_typeof(env, argv[2], &t);
  if (t == napi_number) napi_get_value_int32(env, argv[2], &flags);
  char *path = get_string(env, argv[1], NULL);
  if (!path) return NULL;
  kh_manifest_info mi;
  int rc = kh_load_manifest((kh_ctx *)h->ptr, path, flags, &mi);
  free(path);
  if (rc) return throw_kh(env, rc);
  return manifest_info_object(env, &mi);
}

/* scores(logits: Float32Array, cols: number, kind: number) -> { scores: Float32Array, index: Int32Array } */
static napi_value scores(napi_env env, napi_callback_info info) {
  napi_value argv[3];
  if (!get_args(env, info, 3, argv)) return NULL;
  void *data;
  size_t bytes;
  if (!get_bytes(env, argv[0], &data, &bytes)) {
    napi_throw_type_error(env, NULL, "logits must be a Float32Array");
    return NULL;
  }
  int32_t cols = 0, kind = 0;
  napi_get_value_int32(env, argv[1], &cols);
  napi_get_value_int32(env, argv[2], &kind);
  if (cols <= 0) {
    napi_throw_range_error(env, NULL, "cols must be positive");
    return NULL;
  }
  const size_t n = bytes / 4, rows = n / (size_t)cols;
  napi_value sab, iab, sarr, iarr, o;
  void *sp, *ip;
  CHECK_NAPI(env, napi_create_arraybuffer(env, n * 4, &sp, &sab));
  CHECK_NAPI(env, napi_create_arraybuffer(env, rows * 4 + 4, &ip, &iab));
  int rc = kh_scores((const float *)data, (int64_t)rows, cols, kind, (float *)sp, (int32_t *)ip);
  if (rc) return throw_kh(env, rc);
  CHECK_NAPI(env, napi_create_typedarray(env, napi_float32_array, n, sab, 0, &sarr));
  CHECK_NAPI(env, napi_create_typedarray(env, napi_int32_array, rows, iab, 0, &iarr));
  napi_create_object(env, &o);
  napi_set_named_property(env, o, "scores", sarr);
  napi_set_named_property(env, o, "index", iarr);
  return o;
}

/* rank(scores: Float32Array) -> Int32Array (highest first, ties in index order) */
static napi_value rank(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  void *data;
  size_t bytes;
  if (!get_bytes(env, argv[0], &data, &bytes)) {
    napi_throw_type_error(env, NULL, "scores must be a Float32Array");
    return NULL;
  }
  const size_t n = bytes / 4;
  napi_value ab, arr;
  void *op;
  CHECK_NAPI(env, napi_create_arraybuffer(env, n * 4 + 4, &op, &ab));
  int rc = kh_rank((const float *)data, (int64_t)n, (int32_t *)op);
  if (rc) return throw_kh(env, rc);
  CHECK_NAPI(env, napi_create_typedarray(env, napi_int32_array, n, ab, 0, &arr));
  return arr;
}

/* schedCreate(plans: handle[]) -> scheduler handle (the plans must outlive it) */
static napi_value sched_create(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  if (!get_args(env, info, 1, argv)) return NULL;
  uint32_t n = 0;
  if (napi_get_array_length(env, argv[0], &n) != napi_ok || n == 0) {
    napi_throw_type_error(env, NULL, "expected an array of plan handles");
    return NULL;
  }
  kh_plan **plans = (kh_plan **)malloc(n * sizeof(kh_plan *));
  for (uint32_t i = 0; i < n; i++) {
    napi_value e;
    napi_get_element(env, argv[0], i, &e);
    handle *h = unwrap(env, e, 2);
    if (!h) {
      free(plans);
      return NULL;
    }
    plans[i] = (kh_plan *)h->ptr;
  }
  kh_sched *s = NULL;
  int rc = kh_sched_create(plans, (int32_t)n, &s);
  free(plans);
  if (rc) return throw_kh(env, rc);
  return wrap(env, s, 3);
}

/* schedRun(s, ids: Int32Array, offsets: Float64Array, typeWords: Uint32Array | null, tokenBudget,
 *          cols) -> { out: Float32Array, stats } */
static napi_value sched_run(napi_env env, napi_callback_info info) {
  napi_value argv[6];
  if (!get_args(env, info, 6, argv)) return NULL;
  handle *h = unwrap(env, argv[0], 3);
  if (!h) return NULL;
  void *ids, *offs, *tw;
  size_t ids_b, offs_b, tw_b;
  if (!get_bytes(env, argv[1], &ids, &ids_b) || !get_bytes(env, argv[2], &offs, &offs_b) ||
      !get_bytes(env, argv[3], &tw, &tw_b) || offs_b < 8) {
    napi_throw_type_error(env, NULL, "schedRun(s, ids, offsets, typeWords, tokenBudget, cols)");
    return NULL;
  }
  double budget = 0;
  int32_t cols = 0;
  napi_get_value_double(env, argv[4], &budget);
  napi_get_value_int32(env, argv[5], &cols);
  const size_t nseq = offs_b / 8 - 1;
  int64_t *o64 = (int64_t *)malloc((nseq + 1) * 8);
  for (size_t i = 0; i <= nseq; i++) o64[i] = (int64_t)((const double *)offs)[i];
  napi_value ab, arr, res, st, v;
  void *op;
  CHECK_NAPI(env, napi_create_arraybuffer(env, nseq * (size_t)cols * 4 + 4, &op, &ab));
  kh_sched_stats ss;
  int rc = kh_sched_run((kh_sched *)h->ptr, (const int32_t *)ids, o64, (int64_t)nseq, (const uint32_t *)tw,
                        (int64_t)budget, (float *)op, nseq * (size_t)cols, &ss);
  free(o64);
  if (rc) return throw_kh(env, rc);
  CHECK_NAPI(env, napi_create_typedarray(env, napi_float32_array, nseq * (size_t)cols, ab, 0, &arr));
  napi_create_object(env, &st);
#define SET(name, val)                        \
  napi_create_double(env, (double)(val), &v); \
  napi_set_named_property(env, st, name, v);
  SET("chunks", ss.chunks);
  SET("sequences", ss.sequences);
  SET("tokens", ss.tokens);
  SET("wallMs", ss.wall_ms);
  SET("gpuMs", ss.gpu_ms);
  SET("hostMs", ss.host_ms);
#undef SET
  napi_create_object(env, &res);
  napi_set_named_property(env, res, "out", arr);
  napi_set_named_property(env, res, "stats", st);
  return res;
}

static napi_value abi_version(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value v;
  napi_create_int32(env, kh_abi_version(), &v);
  return v;
}

static napi_value init(napi_env env, napi_value exports) {
  const napi_property_descriptor props[] = {
      {"abiVersion", 0, abi_version, 0, 0, 0, napi_default, 0},
      {"ctxCreate", 0, ctx_create, 0, 0, 0, napi_default, 0},
      {"ctxDestroy", 0, destroy, 0, 0, 0, napi_default, 0},
      {"weightAdd", 0, weight_add, 0, 0, 0, napi_default, 0},
      {"weightBytes", 0, weight_bytes, 0, 0, 0, napi_default, 0},
      {"wordsSet", 0, words_set, 0, 0, 0, napi_default, 0},
      {"planCheck", 0, plan_check, 0, 0, 0, napi_default, 0},
      {"planCreate", 0, plan_create, 0, 0, 0, napi_default, 0},
      {"planInitBuffer", 0, plan_init_buffer, 0, 0, 0, napi_default, 0},
      {"planInfo", 0, plan_info, 0, 0, 0, napi_default, 0},
      {"planDestroy", 0, destroy, 0, 0, 0, napi_default, 0},
      {"upload", 0, upload, 0, 0, 0, napi_default, 0},
      {"uploadIds", 0, upload_ids, 0, 0, 0, napi_default, 0},
      {"uploadMarkers", 0, upload_markers, 0, 0, 0, napi_default, 0},
      {"uploadQtypes", 0, upload_qtypes, 0, 0, 0, napi_default, 0},
      {"run", 0, run, 0, 0, 0, napi_default, 0},
      {"readOutput", 0, read_output, 0, 0, 0, napi_default, 0},
      {"readOutputAsync", 0, read_output_async, 0, 0, 0, napi_default, 0},
      {"lastRunMs", 0, last_run_ms, 0, 0, 0, napi_default, 0},
      {"manifestCheck", 0, manifest_check, 0, 0, 0, napi_default, 0},
      {"loadManifest", 0, load_manifest, 0, 0, 0, napi_default, 0},
      {"scores", 0, scores, 0, 0, 0, napi_default, 0},
      {"rank", 0, rank, 0, 0, 0, napi_default, 0},
      {"schedCreate", 0, sched_create, 0, 0, 0, napi_default, 0},
      {"schedRun", 0, sched_run, 0, 0, 0, napi_default, 0},
      {"schedDestroy", 0, destroy, 0, 0, 0, napi_default, 0},
  };
  napi_define_properties(env, exports, sizeof props / sizeof props[0], props);
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init)
