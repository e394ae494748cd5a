/*
 * q8hip_napi.c -- Node N-API addon over the C ABI of libq8hip.so
 * (include/q8hip.h).  This is the thin native layer the reference's
 * TypeScript runtime would load in place of its koffi bindings to libcuda
 * (src/runtime/node/cuda/ffi.ts:53-97): the JS side (hip_backend.js)
 * registers a runtime backend, an external-codegen entry and a dispatcher
 * library on top of it.
 *
 * Conventions:
 *   - device buffers are napi externals wrapping {device pointer, bytes};
 *     they are released by free() or, as a backstop, by the garbage
 *     collector (the reference's terac runtime module keeps the same
 *     explicit-release-plus-finalizer rule,
 *     src/backend/terac/runtime_module.ts:22,37,89-94);
 *   - host memory stays owned by JS: upload()/download() copy between a
 *     typed array (or ArrayBuffer) and a device buffer and block;
 *   - ops enqueue on the addon's one stream (created by init()) and return
 *     immediately; sync() waits, syncAsync() returns a promise of the same
 *     wait made on a worker thread; captureBegin() / captureEnd() record a
 *     launch sequence on it as a graph that graphLaunch() replays;
 *   - every device buffer an op names is checked against the bytes its
 *     shape arguments imply before the C ABI is called;
 *   - a non-zero status from the C ABI becomes a thrown Error whose message
 *     is q8_last_error() (the reference maps driver codes to JS errors the
 *     same way, src/runtime/node/cuda/ffi.ts:102-104).
 */
#define NAPI_VERSION 8
#include <node_api.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "q8hip.h"

typedef struct {
  void* ptr;
  size_t bytes;
} DevBuf;

/* The addon's one stream (the reference runtime keeps one per process,
 * src/runtime/node/cuda/device.ts:14-35): created by init(), used by every
 * op, upload, download and sync, and the stream plans are captured on.
 * NULL (the null stream) until init(). */
static void* g_stream = NULL;

#define NAPI_CALL(env, call)                                      \
  do {                                                            \
    if ((call) != napi_ok) {                                      \
      napi_throw_error((env), NULL, "q8hip: N-API call failed");  \
      return NULL;                                                \
    }                                                             \
  } while (0)

static napi_value throw_q8(napi_env env, int rc) {
  char code[16];
  snprintf(code, sizeof(code), "Q8_ERR_%d", rc);
  const char* msg = q8_last_error();
  napi_throw_error(env, code, (msg && msg[0]) ? msg : "q8hip: operation failed");
  return NULL;
}

#define Q8_CHECK(env, expr)              \
  do {                                   \
    int rc_ = (expr);                    \
    if (rc_ != Q8_OK) return throw_q8((env), rc_); \
  } while (0)

static napi_value undefined(napi_env env) {
  napi_value u;
  napi_get_undefined(env, &u);
  return u;
}

static int get_args(napi_env env, napi_callback_info info, size_t want, napi_value* argv) {
  size_t argc = want;
  if (napi_get_cb_info(env, info, &argc, argv, NULL, NULL) != napi_ok) return 0;
  if (argc < want) {
    napi_throw_type_error(env, NULL, "q8hip: too few arguments");
    return 0;
  }
  return 1;
}

static int arg_i64(napi_env env, napi_value v, int64_t* out) {
  if (napi_get_value_int64(env, v, out) != napi_ok) {
    napi_throw_type_error(env, NULL, "q8hip: expected a number");
    return 0;
  }
  return 1;
}

static int arg_f64(napi_env env, napi_value v, double* out) {
  if (napi_get_value_double(env, v, out) != napi_ok) {
    napi_throw_type_error(env, NULL, "q8hip: expected a number");
    return 0;
  }
  return 1;
}

/* A device buffer argument; null / undefined give NULL when allowed. */
static int arg_buf(napi_env env, napi_value v, int nullable, void** out) {
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok) return 0;
  if (t == napi_null || t == napi_undefined) {
    if (nullable) {
      *out = NULL;
      return 1;
    }
    napi_throw_type_error(env, NULL, "q8hip: device buffer required");
    return 0;
  }
  if (t != napi_external) {
    napi_throw_type_error(env, NULL, "q8hip: expected a device buffer from alloc()");
    return 0;
  }
  DevBuf* b = NULL;
  if (napi_get_value_external(env, v, (void**)&b) != napi_ok || b == NULL) return 0;
  if (b->ptr == NULL && b->bytes != 0) {
    napi_throw_error(env, NULL, "q8hip: device buffer was freed");
    return 0;
  }
  *out = b->ptr;
  return 1;
}

static int arg_devbuf(napi_env env, napi_value v, DevBuf** out) {
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok || t != napi_external) {
    napi_throw_type_error(env, NULL, "q8hip: expected a device buffer from alloc()");
    return 0;
  }
  return napi_get_value_external(env, v, (void**)out) == napi_ok && *out != NULL;
}

/* Bytes of a*b*c (elements times element size): 0 when a factor is
 * negative (the C ABI rejects the shape itself), -1 on overflow. */
static int64_t nbytes(int64_t a, int64_t b, int64_t c) {
  if (a < 0 || b < 0 || c < 0) return 0;
  if (a == 0 || b == 0 || c == 0) return 0;
  if (a > INT64_MAX / b) return -1;
  const int64_t ab = a * b;
  if (ab > INT64_MAX / c) return -1;
  return ab * c;
}

/* Element bytes of a Q8_I8 / Q8_U8 / Q8_I32 / Q8_F32 / Q8_F64 code (0 for
 * an unknown code, which the C ABI rejects). */
static int64_t elem_bytes(int64_t code) {
  switch (code) {
    case Q8_I8: case Q8_U8: return 1;
    case Q8_I32: case Q8_F32: return 4;
    case Q8_F64: return 8;
    default: return 0;
  }
}

/* A device buffer argument that must hold `need` bytes: every op checks its
 * buffers against the sizes its shape arguments imply before the C ABI
 * launches anything, so an undersized buffer is a JS RangeError, never an
 * out-of-bounds access on the device.  null / undefined give NULL when
 * `nullable` (the C ABI then rejects a NULL that the call needs). */
static int arg_buf_n(napi_env env, napi_value v, int nullable, int64_t need, const char* what, void** out) {
  if (!arg_buf(env, v, nullable, out)) return 0;
  if (*out == NULL) return 1;
  DevBuf* b = NULL;
  if (!arg_devbuf(env, v, &b)) return 0;
  char msg[160];
  if (need < 0) {
    snprintf(msg, sizeof(msg), "q8hip: %s: size overflows", what);
    napi_throw_range_error(env, NULL, msg);
    return 0;
  }
  if ((uint64_t)need > (uint64_t)b->bytes) {
    snprintf(msg, sizeof(msg), "q8hip: %s device buffer holds %zu bytes, the call needs %lld", what, b->bytes,
             (long long)need);
    napi_throw_range_error(env, NULL, msg);
    return 0;
  }
  return 1;
}

/* Host bytes of a typed array, DataView or ArrayBuffer. */
static int arg_host(napi_env env, napi_value v, void** data, size_t* bytes) {
  bool is;
  if (napi_is_typedarray(env, v, &is) == napi_ok && is) {
    napi_typedarray_type tt;
    size_t len, off;
    napi_value ab;
    if (napi_get_typedarray_info(env, v, &tt, &len, data, &ab, &off) != napi_ok) return 0;
    static const size_t esz[] = {1, 1, 1, 2, 2, 4, 4, 4, 8, 8, 8};
    *bytes = len * (tt < (int)(sizeof(esz) / sizeof(esz[0])) ? esz[tt] : 1);
    return 1;
  }
  if (napi_is_arraybuffer(env, v, &is) == napi_ok && is)
    return napi_get_arraybuffer_info(env, v, data, bytes) == napi_ok;
  napi_throw_type_error(env, NULL, "q8hip: expected a typed array or ArrayBuffer");
  return 0;
}

/* A JS array of at most `max` integers. */
static int arg_i64_array(napi_env env, napi_value v, int64_t* out, uint32_t max, uint32_t* n) {
  bool is;
  if (napi_is_array(env, v, &is) != napi_ok || !is) {
    napi_throw_type_error(env, NULL, "q8hip: expected an array of numbers");
    return 0;
  }
  uint32_t len;
  if (napi_get_array_length(env, v, &len) != napi_ok) return 0;
  if (len > max) {
    napi_throw_range_error(env, NULL, "q8hip: array too long");
    return 0;
  }
  for (uint32_t i = 0; i < len; i++) {
    napi_value e;
    if (napi_get_element(env, v, i, &e) != napi_ok || !arg_i64(env, e, &out[i])) return 0;
  }
  *n = len;
  return 1;
}

/* ---------------------------------------------------------------- runtime */

static napi_value js_version(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value r;
  NAPI_CALL(env, napi_create_int32(env, q8_version(), &r));
  return r;
}

static napi_value js_last_error(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value r;
  NAPI_CALL(env, napi_create_string_utf8(env, q8_last_error(), NAPI_AUTO_LENGTH, &r));
  return r;
}

static napi_value js_device_count(napi_env env, napi_callback_info info) {
  (void)info;
  int n = 0;
  Q8_CHECK(env, q8_device_count(&n));
  napi_value r;
  NAPI_CALL(env, napi_create_int32(env, n, &r));
  return r;
}

static napi_value js_init(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  int64_t dev;
  if (!get_args(env, info, 1, argv) || !arg_i64(env, argv[0], &dev)) return NULL;
  Q8_CHECK(env, q8_init((int)dev));
  if (g_stream == NULL) Q8_CHECK(env, q8_stream_create(&g_stream));
  return undefined(env);
}

/* ---------------------------------------------------------------- graphs */

static void finalize_graph(napi_env env, void* data, void* hint) {
  (void)env;
  (void)hint;
  void** g = (void**)data;
  if (*g) q8_graph_destroy(*g);
  free(g);
}

/* captureBegin(): launches on the addon's stream are recorded from here on
 * (the reference's beginEagerCapture, eager_graph.ts). */
static napi_value js_capture_begin(napi_env env, napi_callback_info info) {
  (void)info;
  Q8_CHECK(env, q8_graph_capture_begin(g_stream));
  return undefined(env);
}

/* captureEnd() -> graph: the recorded launches, instantiated; freed by
 * graphDestroy() or, as a backstop, by the garbage collector. */
static napi_value js_capture_end(napi_env env, napi_callback_info info) {
  (void)info;
  void** g = (void**)calloc(1, sizeof(void*));
  if (!g) {
    napi_throw_error(env, NULL, "q8hip.captureEnd: out of host memory");
    return NULL;
  }
  int rc = q8_graph_capture_end(g_stream, g);
  if (rc != Q8_OK) {
    free(g);
    return throw_q8(env, rc);
  }
  napi_value ext;
  if (napi_create_external(env, g, finalize_graph, NULL, &ext) != napi_ok) {
    q8_graph_destroy(*g);
    free(g);
    napi_throw_error(env, NULL, "q8hip.captureEnd: napi_create_external failed");
    return NULL;
  }
  return ext;
}

static int arg_graph(napi_env env, napi_value v, void*** out) {
  napi_valuetype t;
  if (napi_typeof(env, v, &t) != napi_ok || t != napi_external ||
      napi_get_value_external(env, v, (void**)out) != napi_ok || *out == NULL) {
    napi_throw_type_error(env, NULL, "q8hip: expected a graph from captureEnd()");
    return 0;
  }
  return 1;
}

/* graphLaunch(graph): replay on the addon's stream (returns immediately). */
static napi_value js_graph_launch(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  void** g;
  if (!get_args(env, info, 1, argv) || !arg_graph(env, argv[0], &g)) return NULL;
  if (*g == NULL) {
    napi_throw_error(env, NULL, "q8hip.graphLaunch: graph was destroyed");
    return NULL;
  }
  Q8_CHECK(env, q8_graph_launch(*g, g_stream));
  return undefined(env);
}

static napi_value js_graph_destroy(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  void** g;
  if (!get_args(env, info, 1, argv) || !arg_graph(env, argv[0], &g)) return NULL;
  void* x = *g;
  *g = NULL;
  Q8_CHECK(env, q8_graph_destroy(x));
  return undefined(env);
}

static void finalize_buf(napi_env env, void* data, void* hint) {
  (void)env;
  (void)hint;
  DevBuf* b = (DevBuf*)data;
  if (b->ptr) q8_free(b->ptr);
  free(b);
}

static napi_value js_alloc(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  int64_t bytes;
  if (!get_args(env, info, 1, argv) || !arg_i64(env, argv[0], &bytes)) return NULL;
  if (bytes < 0) {
    napi_throw_range_error(env, NULL, "q8hip.alloc: negative size");
    return NULL;
  }
  DevBuf* b = (DevBuf*)calloc(1, sizeof(DevBuf));
  if (!b) {
    napi_throw_error(env, NULL, "q8hip.alloc: out of host memory");
    return NULL;
  }
  int rc = q8_alloc(&b->ptr, (size_t)bytes);
  if (rc != Q8_OK) {
    free(b);
    return throw_q8(env, rc);
  }
  b->bytes = (size_t)bytes;
  napi_value ext;
  if (napi_create_external(env, b, finalize_buf, NULL, &ext) != napi_ok) {
    q8_free(b->ptr);
    free(b);
    napi_throw_error(env, NULL, "q8hip.alloc: napi_create_external failed");
    return NULL;
  }
  return ext;
}

static napi_value js_free(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  DevBuf* b;
  if (!get_args(env, info, 1, argv) || !arg_devbuf(env, argv[0], &b)) return NULL;
  void* p = b->ptr;
  b->ptr = NULL;
  b->bytes = 0;
  Q8_CHECK(env, q8_free(p));
  return undefined(env);
}

static napi_value js_bytes(napi_env env, napi_callback_info info) {
  napi_value argv[1];
  DevBuf* b;
  if (!get_args(env, info, 1, argv) || !arg_devbuf(env, argv[0], &b)) return NULL;
  napi_value r;
  NAPI_CALL(env, napi_create_double(env, (double)b->bytes, &r));
  return r;
}

/* upload(dev, hostArray): host -> device, blocking; sizes must fit. */
static napi_value js_upload(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  DevBuf* b;
  void* host;
  size_t n;
  if (!get_args(env, info, 2, argv) || !arg_devbuf(env, argv[0], &b) ||
      !arg_host(env, argv[1], &host, &n))
    return NULL;
  if (n > b->bytes) {
    napi_throw_range_error(env, NULL, "q8hip.upload: host array larger than the device buffer");
    return NULL;
  }
  Q8_CHECK(env, q8_h2d(b->ptr, host, n, g_stream));
  return undefined(env);
}

/* download(hostArray, dev): device -> host, blocking; copies hostArray's size. */
static napi_value js_download(napi_env env, napi_callback_info info) {
  napi_value argv[2];
  DevBuf* b;
  void* host;
  size_t n;
  if (!get_args(env, info, 2, argv) || !arg_host(env, argv[0], &host, &n) ||
      !arg_devbuf(env, argv[1], &b))
    return NULL;
  if (n > b->bytes) {
    napi_throw_range_error(env, NULL, "q8hip.download: host array larger than the device buffer");
    return NULL;
  }
  Q8_CHECK(env, q8_d2h(host, b->ptr, n, g_stream));
  return undefined(env);
}

static napi_value js_sync(napi_env env, napi_callback_info info) {
  (void)info;
  Q8_CHECK(env, q8_stream_sync(g_stream));
  return undefined(env);
}

/* syncAsync(): a promise that settles when the stream's work has finished.
 * The wait runs on a libuv worker thread (napi_async_work), so the JS thread
 * stays free while the device works; the promise rejects with the coded
 * error of a failed wait.  The error text is the worker thread's own
 * (q8_last_error is thread-local), copied before the thread moves on. */
typedef struct {
  napi_async_work work;
  napi_deferred deferred;
  int rc;
  char msg[1024];
} SyncWork;

static void sync_execute(napi_env env, void* data) {
  (void)env;
  SyncWork* w = (SyncWork*)data;
  w->rc = q8_stream_sync(g_stream);
  if (w->rc != Q8_OK) snprintf(w->msg, sizeof(w->msg), "%s", q8_last_error());
}

static void sync_complete(napi_env env, napi_status status, void* data) {
  SyncWork* w = (SyncWork*)data;
  if (status == napi_ok && w->rc == Q8_OK) {
    napi_resolve_deferred(env, w->deferred, undefined(env));
  } else {
    char code[16];
    snprintf(code, sizeof(code), "Q8_ERR_%d", w->rc != Q8_OK ? w->rc : Q8_ERR_DEVICE);
    napi_value c, m, e;
    napi_create_string_utf8(env, code, NAPI_AUTO_LENGTH, &c);
    napi_create_string_utf8(env, w->rc != Q8_OK && w->msg[0] ? w->msg : "q8hip.syncAsync: the wait did not run",
                            NAPI_AUTO_LENGTH, &m);
    napi_create_error(env, c, m, &e);
    napi_reject_deferred(env, w->deferred, e);
  }
  napi_delete_async_work(env, w->work);
  free(w);
}

static napi_value js_sync_async(napi_env env, napi_callback_info info) {
  (void)info;
  SyncWork* w = (SyncWork*)calloc(1, sizeof(SyncWork));
  napi_value promise, name;
  if (!w) {
    napi_throw_error(env, NULL, "q8hip.syncAsync: out of host memory");
    return NULL;
  }
  if (napi_create_promise(env, &w->deferred, &promise) != napi_ok ||
      napi_create_string_utf8(env, "q8hip.syncAsync", NAPI_AUTO_LENGTH, &name) != napi_ok ||
      napi_create_async_work(env, NULL, name, sync_execute, sync_complete, w, &w->work) != napi_ok ||
      napi_queue_async_work(env, w->work) != napi_ok) {
    free(w);
    napi_throw_error(env, NULL, "q8hip.syncAsync: could not queue the wait");
    return NULL;
  }
  return promise;
}

/* ---------------------------------------------------------------- ops */

/* fillNormal(t, n, seed, offset, mean, std) / fillUniform(t, n, seed, offset, a, b) */
static napi_value fill(napi_env env, napi_callback_info info, int normal) {
  napi_value argv[6];
  void* t;
  int64_t n, seed, offset;
  double a, b;
  if (!get_args(env, info, 6, argv) || !arg_i64(env, argv[1], &n) ||
      !arg_i64(env, argv[2], &seed) || !arg_i64(env, argv[3], &offset) || !arg_f64(env, argv[4], &a) ||
      !arg_f64(env, argv[5], &b) || !arg_buf_n(env, argv[0], 0, nbytes(n, 4, 1), "fill output", &t))
    return NULL;
  if (normal)
    Q8_CHECK(env, q8_fill_normal((float*)t, n, (uint32_t)seed, (uint64_t)offset, a, b, g_stream));
  else
    Q8_CHECK(env, q8_fill_uniform((float*)t, n, (uint32_t)seed, (uint64_t)offset, a, b, g_stream));
  return undefined(env);
}
static napi_value js_fill_normal(napi_env env, napi_callback_info info) { return fill(env, info, 1); }
static napi_value js_fill_uniform(napi_env env, napi_callback_info info) { return fill(env, info, 0); }

/* quantizeStatic(x, n, scale, zeroPoint, target, q) */
static napi_value js_quantize_static(napi_env env, napi_callback_info info) {
  napi_value argv[6];
  void *x, *q;
  int64_t n, target;
  double s, zp;
  if (!get_args(env, info, 6, argv) || !arg_i64(env, argv[1], &n) ||
      !arg_f64(env, argv[2], &s) || !arg_f64(env, argv[3], &zp) || !arg_i64(env, argv[4], &target) ||
      !arg_buf_n(env, argv[0], 1, nbytes(n, 4, 1), "quantizeStatic x", &x) ||
      !arg_buf_n(env, argv[5], 1, nbytes(n, 1, 1), "quantizeStatic q", &q))
    return NULL;
  Q8_CHECK(env, q8_quantize_static((const float*)x, n, s, zp, (int)target, q, g_stream));
  return undefined(env);
}

/* quantizeRows(x, M, K, mode, q, scales) */
static napi_value js_quantize_rows(napi_env env, napi_callback_info info) {
  napi_value argv[6];
  void *x, *q, *sc;
  int64_t M, K, mode;
  if (!get_args(env, info, 6, argv) || !arg_i64(env, argv[1], &M) ||
      !arg_i64(env, argv[2], &K) || !arg_i64(env, argv[3], &mode) ||
      !arg_buf_n(env, argv[0], 1, nbytes(M, K, 4), "quantizeRows x", &x) ||
      !arg_buf_n(env, argv[4], 1, nbytes(M, K, 1), "quantizeRows q", &q) ||
      !arg_buf_n(env, argv[5], 1, nbytes(mode == Q8_PER_TOKEN ? M : 1, 8, 1), "quantizeRows scales", &sc))
    return NULL;
  Q8_CHECK(env, q8_quantize_rows((const float*)x, M, K, (int)mode, (int8_t*)q, (double*)sc, g_stream));
  return undefined(env);
}

/* dequantize(q, src, M, K, scales, granularity, zeroPoint, y) */
static napi_value js_dequantize(napi_env env, napi_callback_info info) {
  napi_value argv[8];
  void *q, *sc, *y;
  int64_t src, M, K, gran;
  double zp;
  if (!get_args(env, info, 8, argv) || !arg_i64(env, argv[1], &src) ||
      !arg_i64(env, argv[2], &M) || !arg_i64(env, argv[3], &K) ||
      !arg_i64(env, argv[5], &gran) || !arg_f64(env, argv[6], &zp) ||
      !arg_buf_n(env, argv[0], 1, nbytes(M, K, elem_bytes(src)), "dequantize q", &q) ||
      !arg_buf_n(env, argv[4], 1, nbytes(gran == Q8_PER_TOKEN ? M : 1, 8, 1), "dequantize scales", &sc) ||
      !arg_buf_n(env, argv[7], 1, nbytes(M, K, 4), "dequantize y", &y))
    return NULL;
  Q8_CHECK(env, q8_dequantize(q, (int)src, M, K, (const double*)sc, (int)gran, zp, (float*)y, g_stream));
  return undefined(env);
}

/* packWeight(W, rows, cols, axis, granularity, Wq, scales) */
static napi_value js_pack_weight(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  void *w, *wq, *sc;
  int64_t rows, cols, axis, gran;
  if (!get_args(env, info, 7, argv) || !arg_i64(env, argv[1], &rows) ||
      !arg_i64(env, argv[2], &cols) || !arg_i64(env, argv[3], &axis) || !arg_i64(env, argv[4], &gran) ||
      !arg_buf_n(env, argv[0], 1, nbytes(rows, cols, 4), "packWeight W", &w) ||
      !arg_buf_n(env, argv[5], 1, nbytes(rows, cols, 1), "packWeight Wq", &wq) ||
      !arg_buf_n(env, argv[6], 1, nbytes(gran == Q8_PER_TENSOR ? 1 : (axis == 0 ? rows : cols), 8, 1),
                 "packWeight scales", &sc))
    return NULL;
  Q8_CHECK(env, q8_pack_weight((const float*)w, rows, cols, (int)axis, (int)gran, (int8_t*)wq,
                               (double*)sc, g_stream));
  return undefined(env);
}

/* gemm(A, B, M, N, K, zpA, zpB, sA, sAmode, sB, sBmode, epi, sOut, bias, act, outKind, out) */
static napi_value js_gemm(napi_env env, napi_callback_info info) {
  napi_value argv[17];
  void *A, *B, *sA, *sB, *bias, *out;
  int64_t M, N, K, zpA, zpB, sAm, sBm, epi, act, ok;
  double sOut;
  if (!get_args(env, info, 17, argv) ||
      !arg_i64(env, argv[2], &M) || !arg_i64(env, argv[3], &N) || !arg_i64(env, argv[4], &K) ||
      !arg_i64(env, argv[5], &zpA) || !arg_i64(env, argv[6], &zpB) ||
      !arg_i64(env, argv[8], &sAm) || !arg_i64(env, argv[10], &sBm) ||
      !arg_i64(env, argv[11], &epi) || !arg_f64(env, argv[12], &sOut) ||
      !arg_i64(env, argv[14], &act) || !arg_i64(env, argv[15], &ok) ||
      !arg_buf_n(env, argv[0], 1, nbytes(M, K, 1), "gemm A", &A) ||
      !arg_buf_n(env, argv[1], 1, nbytes(N, K, 1), "gemm B", &B) ||
      !arg_buf_n(env, argv[7], 1, nbytes(sAm == Q8_PER_TOKEN ? M : 1, 8, 1), "gemm sA", &sA) ||
      !arg_buf_n(env, argv[9], 1, nbytes(sBm == Q8_PER_CHANNEL ? N : 1, 8, 1), "gemm sB", &sB) ||
      !arg_buf_n(env, argv[13], 1, nbytes(N, 4, 1), "gemm bias", &bias) ||
      !arg_buf_n(env, argv[16], 1, nbytes(M, N, 4), "gemm out", &out))
    return NULL;
  Q8_CHECK(env, q8_gemm((const int8_t*)A, (const int8_t*)B, M, N, K, (int32_t)zpA, (int32_t)zpB,
                        (const double*)sA, (int)sAm, (const double*)sB, (int)sBm, (int)epi, sOut,
                        (const float*)bias, (int)act, (int)ok, out, g_stream));
  return undefined(env);
}

/* gemmRequant(A, B, M, N, K, sA, sAMode, sB, sBMode, epi, sOut, bias, act, sNext, out):
 * the epilogue value requantized with the next layer's static scale (int8 out). */
static napi_value js_gemm_requant(napi_env env, napi_callback_info info) {
  napi_value argv[15];
  void *A, *B, *sA, *sB, *bias, *out;
  int64_t M, N, K, sAm, sBm, epi, act;
  double sOut, sNext;
  if (!get_args(env, info, 15, argv) ||
      !arg_i64(env, argv[2], &M) || !arg_i64(env, argv[3], &N) || !arg_i64(env, argv[4], &K) ||
      !arg_i64(env, argv[6], &sAm) || !arg_i64(env, argv[8], &sBm) || !arg_i64(env, argv[9], &epi) ||
      !arg_f64(env, argv[10], &sOut) || !arg_i64(env, argv[12], &act) || !arg_f64(env, argv[13], &sNext) ||
      !arg_buf_n(env, argv[0], 1, nbytes(M, K, 1), "gemmRequant A", &A) ||
      !arg_buf_n(env, argv[1], 1, nbytes(N, K, 1), "gemmRequant B", &B) ||
      !arg_buf_n(env, argv[5], 1, nbytes(sAm == Q8_PER_TOKEN ? M : 1, 8, 1), "gemmRequant sA", &sA) ||
      !arg_buf_n(env, argv[7], 1, nbytes(sBm == Q8_PER_CHANNEL ? N : 1, 8, 1), "gemmRequant sB", &sB) ||
      !arg_buf_n(env, argv[11], 1, nbytes(N, 4, 1), "gemmRequant bias", &bias) ||
      !arg_buf_n(env, argv[14], 1, nbytes(M, N, 1), "gemmRequant out", &out))
    return NULL;
  Q8_CHECK(env, q8_gemm_requant((const int8_t*)A, (const int8_t*)B, M, N, K, (const double*)sA, (int)sAm,
                                (const double*)sB, (int)sBm, (int)epi, sOut, (const float*)bias, (int)act,
                                sNext, (int8_t*)out, g_stream));
  return undefined(env);
}

/* qlinearDynamic(x, M, K, xMode, wq, sW, sWMode, N, bias, act, out, xq, sx) */
static napi_value js_qlinear_dynamic(napi_env env, napi_callback_info info) {
  napi_value argv[13];
  void *x, *wq, *sw, *bias, *out, *xq, *sx;
  int64_t M, K, xm, swm, N, act;
  if (!get_args(env, info, 13, argv) || !arg_i64(env, argv[1], &M) ||
      !arg_i64(env, argv[2], &K) || !arg_i64(env, argv[3], &xm) ||
      !arg_i64(env, argv[6], &swm) || !arg_i64(env, argv[7], &N) || !arg_i64(env, argv[9], &act) ||
      !arg_buf_n(env, argv[0], 1, nbytes(M, K, 4), "qlinearDynamic x", &x) ||
      !arg_buf_n(env, argv[4], 1, nbytes(N, K, 1), "qlinearDynamic wq", &wq) ||
      !arg_buf_n(env, argv[5], 1, nbytes(swm == Q8_PER_CHANNEL ? N : 1, 8, 1), "qlinearDynamic sW", &sw) ||
      !arg_buf_n(env, argv[8], 1, nbytes(N, 4, 1), "qlinearDynamic bias", &bias) ||
      !arg_buf_n(env, argv[10], 1, nbytes(M, N, 4), "qlinearDynamic out", &out) ||
      !arg_buf_n(env, argv[11], 1, nbytes(M, K, 1), "qlinearDynamic xq", &xq) ||
      !arg_buf_n(env, argv[12], 1, nbytes(xm == Q8_PER_TOKEN ? M : 1, 8, 1), "qlinearDynamic sx", &sx))
    return NULL;
  Q8_CHECK(env, q8_qlinear_dynamic((const float*)x, M, K, (int)xm, (const int8_t*)wq, (const double*)sw,
                                   (int)swm, N, (const float*)bias, (int)act, (float*)out, (int8_t*)xq,
                                   (double*)sx, g_stream));
  return undefined(env);
}

/* packWeightInt4(W, N, K, groupSize, wq4, scales) */
static napi_value js_pack_weight_int4(napi_env env, napi_callback_info info) {
  napi_value argv[6];
  void *W, *wq, *s;
  int64_t N, K, g;
  if (!get_args(env, info, 6, argv) || !arg_i64(env, argv[1], &N) ||
      !arg_i64(env, argv[2], &K) || !arg_i64(env, argv[3], &g) ||
      !arg_buf_n(env, argv[0], 1, nbytes(N, K, 4), "packWeightInt4 W", &W) ||
      !arg_buf_n(env, argv[4], 1, nbytes(N, K / 2, 1), "packWeightInt4 packed weights", &wq) ||
      !arg_buf_n(env, argv[5], 1, g > 0 ? nbytes(N, K / g, 8) : 0, "packWeightInt4 scales", &s))
    return NULL;
  Q8_CHECK(env, q8_pack_weight_int4((const float*)W, N, K, g, (uint8_t*)wq, (double*)s, g_stream));
  return undefined(env);
}

/* gemvW4(xq, sx, sxMode, wq4, sw, M, N, K, groupSize, bias, act, out) */
static napi_value js_gemv_w4(napi_env env, napi_callback_info info) {
  napi_value argv[12];
  void *xq, *sx, *wq, *sw, *bias, *out;
  int64_t sxm, M, N, K, g, act;
  if (!get_args(env, info, 12, argv) || !arg_i64(env, argv[2], &sxm) ||
      !arg_i64(env, argv[5], &M) || !arg_i64(env, argv[6], &N) || !arg_i64(env, argv[7], &K) ||
      !arg_i64(env, argv[8], &g) || !arg_i64(env, argv[10], &act) ||
      !arg_buf_n(env, argv[0], 1, nbytes(M, K, 1), "gemvW4 xq", &xq) ||
      !arg_buf_n(env, argv[1], 1, nbytes(sxm == Q8_PER_TOKEN ? M : 1, 8, 1), "gemvW4 sx", &sx) ||
      !arg_buf_n(env, argv[3], 1, nbytes(N, K / 2, 1), "gemvW4 packed weights", &wq) ||
      !arg_buf_n(env, argv[4], 1, g > 0 ? nbytes(N, K / g, 8) : 0, "gemvW4 group scales", &sw) ||
      !arg_buf_n(env, argv[9], 1, nbytes(N, 4, 1), "gemvW4 bias", &bias) ||
      !arg_buf_n(env, argv[11], 1, nbytes(M, N, 4), "gemvW4 out", &out))
    return NULL;
  Q8_CHECK(env, q8_gemv_w4((const int8_t*)xq, (const double*)sx, (int)sxm, (const uint8_t*)wq,
                           (const double*)sw, M, N, K, g, (const float*)bias, (int)act, (float*)out, g_stream));
  return undefined(env);
}

/* Shape arguments of the conv entry points: xShape, wShape, strides, padLo,
 * padHi, dilation as JS arrays (argv[0..5]) for `d` spatial dims. */
typedef struct {
  int64_t xs[5], ws[5], st[3], lo[3], hi[3], dl[3];
} ConvArgs;
static int conv_args(napi_env env, napi_value* argv, int64_t d, ConvArgs* c) {
  uint32_t n[6];
  if (d < 1 || d > 3) {
    napi_throw_range_error(env, NULL, "q8hip: spatial dims must be 1, 2 or 3");
    return 0;
  }
  if (!arg_i64_array(env, argv[0], c->xs, 5, &n[0]) || !arg_i64_array(env, argv[1], c->ws, 5, &n[1]) ||
      !arg_i64_array(env, argv[2], c->st, 3, &n[2]) || !arg_i64_array(env, argv[3], c->lo, 3, &n[3]) ||
      !arg_i64_array(env, argv[4], c->hi, 3, &n[4]) || !arg_i64_array(env, argv[5], c->dl, 3, &n[5]))
    return 0;
  if (n[0] != 2 + d || n[1] != 2 + d || n[2] != d || n[3] != d || n[4] != d || n[5] != d) {
    napi_throw_range_error(env, NULL, "q8hip: conv shape arrays do not match the spatial rank");
    return 0;
  }
  return 1;
}

/* Bytes of x, w and the int32 / fp32 output a conv call reads and writes
 * (the output extent of spatial dim i is
 * floor((x_i + lo_i + hi_i - dl_i * (k_i - 1) - 1) / st_i) + 1; shapes the
 * C ABI rejects give 0). */
static void conv_bytes(const ConvArgs* c, int64_t d, int64_t xe, int64_t we, int64_t* xb, int64_t* wb,
                       int64_t* ob) {
  int64_t xn = 1, wn = 1, on = c->xs[0] * c->ws[0];
  for (int64_t i = 0; i < 2 + d; ++i) {
    xn = nbytes(xn, c->xs[i], 1);
    wn = nbytes(wn, c->ws[i], 1);
  }
  for (int64_t i = 0; i < d; ++i) {
    int64_t o = 0;
    if (c->st[i] > 0 && c->dl[i] > 0 && c->ws[2 + i] > 0) {
      const int64_t span = c->xs[2 + i] + c->lo[i] + c->hi[i] - c->dl[i] * (c->ws[2 + i] - 1) - 1;
      o = span >= 0 ? span / c->st[i] + 1 : 0;
    }
    on = nbytes(on, o, 1);
  }
  *xb = nbytes(xn, xe, 1);
  *wb = nbytes(wn, we, 1);
  *ob = nbytes(on, 4, 1);
}

/* convWorkspace(d, xShape, wShape, strides, padLo, padHi, dilation, groups) -> bytes */
static napi_value js_conv_workspace(napi_env env, napi_callback_info info) {
  napi_value argv[8], r;
  int64_t d, groups;
  ConvArgs c;
  size_t bytes = 0;
  if (!get_args(env, info, 8, argv) || !arg_i64(env, argv[0], &d) || !conv_args(env, argv + 1, d, &c) ||
      !arg_i64(env, argv[7], &groups))
    return NULL;
  Q8_CHECK(env, q8_quantized_conv_workspace((int)d, c.xs, c.ws, c.st, c.lo, c.hi, c.dl, groups, &bytes));
  napi_create_double(env, (double)bytes, &r);
  return r;
}

/* quantizedConv(x, w, d, xShape, wShape, strides, padLo, padHi, dilation, groups,
 *               zpX, zpW, outKind, sOut, workspace, out) */
static napi_value js_quantized_conv(napi_env env, napi_callback_info info) {
  napi_value argv[16];
  void *x, *w, *ws, *out;
  int64_t d, groups, zpx, zpw, ok;
  double sOut;
  ConvArgs c;
  DevBuf* wsb = NULL;
  int64_t xb, wb, ob;
  if (!get_args(env, info, 16, argv) ||
      !arg_i64(env, argv[2], &d) || !conv_args(env, argv + 3, d, &c) || !arg_i64(env, argv[9], &groups) ||
      !arg_i64(env, argv[10], &zpx) || !arg_i64(env, argv[11], &zpw) || !arg_i64(env, argv[12], &ok) ||
      !arg_f64(env, argv[13], &sOut) || !arg_buf(env, argv[14], 1, &ws))
    return NULL;
  conv_bytes(&c, d, 1, 1, &xb, &wb, &ob);
  if (!arg_buf_n(env, argv[0], 1, xb, "quantizedConv x", &x) || !arg_buf_n(env, argv[1], 1, wb, "quantizedConv w", &w) ||
      !arg_buf_n(env, argv[15], 1, ob, "quantizedConv out", &out))
    return NULL;
  size_t ws_bytes = 0;
  if (ws != NULL && arg_devbuf(env, argv[14], &wsb)) ws_bytes = wsb->bytes;
  Q8_CHECK(env, q8_quantized_conv((const int8_t*)x, (const int8_t*)w, (int)d, c.xs, c.ws, c.st, c.lo,
                                  c.hi, c.dl, groups, (int32_t)zpx, (int32_t)zpw, (int)ok, sOut, ws,
                                  ws_bytes, out, g_stream));
  return undefined(env);
}

/* convWeightTaps(w, d, wShape, groups, wTaps): the tap-major copy of a conv
 * weight (q8_conv_weight_taps) */
static napi_value js_conv_weight_taps(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  void *w, *wt;
  int64_t d, groups, ws[5];
  uint32_t n = 0;
  if (!get_args(env, info, 5, argv) || !arg_i64(env, argv[1], &d) || !arg_i64_array(env, argv[2], ws, 5, &n) ||
      !arg_i64(env, argv[3], &groups))
    return NULL;
  if (n != (uint32_t)(2 + d)) {
    napi_throw_range_error(env, NULL, "q8hip.convWeightTaps: wShape does not match the spatial rank");
    return NULL;
  }
  int64_t wb = 1;
  for (uint32_t i = 0; i < n; ++i) wb = nbytes(wb, ws[i], 1);
  if (!arg_buf_n(env, argv[0], 1, wb, "convWeightTaps w", &w) || !arg_buf_n(env, argv[4], 1, wb, "convWeightTaps wTaps", &wt))
    return NULL;
  Q8_CHECK(env, q8_conv_weight_taps((const int8_t*)w, (int)d, ws, groups, (int8_t*)wt, g_stream));
  return undefined(env);
}

/* quantizedConvPrepacked(x, w, wTaps, d, xShape, wShape, strides, padLo, padHi,
 *                        dilation, groups, zpX, zpW, outKind, sOut, workspace, out) */
static napi_value js_quantized_conv_prepacked(napi_env env, napi_callback_info info) {
  napi_value argv[17];
  void *x, *w, *wt, *ws, *out;
  int64_t d, groups, zpx, zpw, ok;
  double sOut;
  ConvArgs c;
  DevBuf* wsb = NULL;
  int64_t xb, wb, ob;
  if (!get_args(env, info, 17, argv) || !arg_i64(env, argv[3], &d) || !conv_args(env, argv + 4, d, &c) ||
      !arg_i64(env, argv[10], &groups) || !arg_i64(env, argv[11], &zpx) || !arg_i64(env, argv[12], &zpw) ||
      !arg_i64(env, argv[13], &ok) || !arg_f64(env, argv[14], &sOut) || !arg_buf(env, argv[15], 1, &ws))
    return NULL;
  conv_bytes(&c, d, 1, 1, &xb, &wb, &ob);
  if (!arg_buf_n(env, argv[0], 1, xb, "quantizedConvPrepacked x", &x) ||
      !arg_buf_n(env, argv[1], 1, wb, "quantizedConvPrepacked w", &w) ||
      !arg_buf_n(env, argv[2], 1, wb, "quantizedConvPrepacked wTaps", &wt) ||
      !arg_buf_n(env, argv[16], 1, ob, "quantizedConvPrepacked out", &out))
    return NULL;
  size_t ws_bytes = 0;
  if (ws != NULL && arg_devbuf(env, argv[15], &wsb)) ws_bytes = wsb->bytes;
  Q8_CHECK(env, q8_quantized_conv_prepacked((const int8_t*)x, (const int8_t*)w, (const int8_t*)wt, (int)d, c.xs,
                                            c.ws, c.st, c.lo, c.hi, c.dl, groups, (int32_t)zpx, (int32_t)zpw,
                                            (int)ok, sOut, ws, ws_bytes, out, g_stream));
  return undefined(env);
}

/* siluMulQuantizeRows(g, u, M, K, h, q, scales) */
/* quantizedConvEx(x, xDtype, w, wDtype, d, xShape, wShape, strides, padLo, padHi, dilation,
 *                 groups, zpX, zpW, outKind, sOut, workspace, out) */
static napi_value js_quantized_conv_ex(napi_env env, napi_callback_info info) {
  napi_value argv[18];
  void *x, *w, *ws, *out;
  int64_t xd, wd, d, groups, zpx, zpw, ok;
  double sOut;
  ConvArgs c;
  DevBuf* wsb = NULL;
  int64_t xb, wb, ob;
  if (!get_args(env, info, 18, argv) || !arg_i64(env, argv[1], &xd) ||
      !arg_i64(env, argv[3], &wd) || !arg_i64(env, argv[4], &d) ||
      !conv_args(env, argv + 5, d, &c) || !arg_i64(env, argv[11], &groups) ||
      !arg_i64(env, argv[12], &zpx) || !arg_i64(env, argv[13], &zpw) || !arg_i64(env, argv[14], &ok) ||
      !arg_f64(env, argv[15], &sOut) || !arg_buf(env, argv[16], 1, &ws))
    return NULL;
  conv_bytes(&c, d, elem_bytes(xd), elem_bytes(wd), &xb, &wb, &ob);
  if (!arg_buf_n(env, argv[0], 1, xb, "quantizedConvEx x", &x) ||
      !arg_buf_n(env, argv[2], 1, wb, "quantizedConvEx w", &w) ||
      !arg_buf_n(env, argv[17], 1, ob, "quantizedConvEx out", &out))
    return NULL;
  size_t ws_bytes = 0;
  if (ws != NULL && arg_devbuf(env, argv[16], &wsb)) ws_bytes = wsb->bytes;
  Q8_CHECK(env, q8_quantized_conv_ex(x, (int)xd, w, (int)wd, (int)d, c.xs, c.ws, c.st, c.lo, c.hi, c.dl,
                                     groups, (int32_t)zpx, (int32_t)zpw, (int)ok, sOut, ws, ws_bytes, out,
                                     g_stream));
  return undefined(env);
}

/* quantizedDotWorkspace(M, N, K, aDtype, bDtype, zpA, zpB) -> bytes */
static napi_value js_quantized_dot_workspace(napi_env env, napi_callback_info info) {
  napi_value argv[7], r;
  int64_t M, N, K, ad, bd, za, zb;
  size_t bytes = 0;
  if (!get_args(env, info, 7, argv) || !arg_i64(env, argv[0], &M) || !arg_i64(env, argv[1], &N) ||
      !arg_i64(env, argv[2], &K) || !arg_i64(env, argv[3], &ad) || !arg_i64(env, argv[4], &bd) ||
      !arg_i64(env, argv[5], &za) || !arg_i64(env, argv[6], &zb))
    return NULL;
  Q8_CHECK(env, q8_quantized_dot_workspace(M, N, K, (int)ad, (int)bd, (int32_t)za, (int32_t)zb, &bytes));
  napi_create_double(env, (double)bytes, &r);
  return r;
}

/* quantizedDot(A, aDtype, B, bDtype, M, N, K, zpA, zpB, workspace, out) */
static napi_value js_quantized_dot(napi_env env, napi_callback_info info) {
  napi_value argv[11];
  void *A, *B, *ws, *out;
  int64_t ad, bd, M, N, K, za, zb;
  DevBuf* wsb = NULL;
  if (!get_args(env, info, 11, argv) || !arg_i64(env, argv[1], &ad) ||
      !arg_i64(env, argv[3], &bd) || !arg_i64(env, argv[4], &M) ||
      !arg_i64(env, argv[5], &N) || !arg_i64(env, argv[6], &K) || !arg_i64(env, argv[7], &za) ||
      !arg_i64(env, argv[8], &zb) || !arg_buf(env, argv[9], 1, &ws) ||
      !arg_buf_n(env, argv[0], 1, nbytes(M, K, 1), "quantizedDot A", &A) ||
      !arg_buf_n(env, argv[2], 1, nbytes(N, K, 1), "quantizedDot B", &B) ||
      !arg_buf_n(env, argv[10], 1, nbytes(M, N, 4), "quantizedDot out", &out))
    return NULL;
  size_t ws_bytes = 0;
  if (ws != NULL && arg_devbuf(env, argv[9], &wsb)) ws_bytes = wsb->bytes;
  Q8_CHECK(env, q8_quantized_dot(A, (int)ad, B, (int)bd, M, N, K, (int32_t)za, (int32_t)zb, ws, ws_bytes,
                                 (int32_t*)out, g_stream));
  return undefined(env);
}

static napi_value js_silu_mul_quantize_rows(napi_env env, napi_callback_info info) {
  napi_value argv[7];
  void *g, *u, *h, *q, *sc;
  int64_t M, K;
  if (!get_args(env, info, 7, argv) || !arg_i64(env, argv[2], &M) || !arg_i64(env, argv[3], &K) ||
      !arg_buf_n(env, argv[0], 1, nbytes(M, K, 4), "siluMulQuantizeRows g", &g) ||
      !arg_buf_n(env, argv[1], 1, nbytes(M, K, 4), "siluMulQuantizeRows u", &u) ||
      !arg_buf_n(env, argv[4], 1, nbytes(M, K, 4), "siluMulQuantizeRows h", &h) ||
      !arg_buf_n(env, argv[5], 1, nbytes(M, K, 1), "siluMulQuantizeRows q", &q) ||
      !arg_buf_n(env, argv[6], 1, nbytes(M, 8, 1), "siluMulQuantizeRows scales", &sc))
    return NULL;
  Q8_CHECK(env, q8_silu_mul_quantize_rows((const float*)g, (const float*)u, M, K, (float*)h,
                                          (int8_t*)q, (double*)sc, g_stream));
  return undefined(env);
}

/* ---------------------------------------------------------------- module */

/* ewise(progBytes, [inputs], [inNumel], out, outNumel): one elementwise loop
 * nest (q8_ewise); progBytes holds a q8_ew_prog exactly (ewise.js packs it). */
static napi_value js_ewise(napi_env env, napi_callback_info info) {
  napi_value argv[5];
  void* pb = NULL;
  size_t pbytes = 0;
  void* out = NULL;
  int64_t onum = 0;
  if (!get_args(env, info, 5, argv) || !arg_host(env, argv[0], &pb, &pbytes) || !arg_i64(env, argv[4], &onum))
    return NULL;
  if (pbytes != sizeof(q8_ew_prog)) {
    napi_throw_range_error(env, NULL, "q8hip: program bytes differ from sizeof(q8_ew_prog)");
    return NULL;
  }
  q8_ew_prog prog;
  memcpy(&prog, pb, sizeof(prog));
  if (!arg_buf_n(env, argv[3], 1, nbytes(onum, elem_bytes(prog.out_dtype), 1), "ewise out", &out)) return NULL;
  bool is;
  uint32_t n = 0;
  if (napi_is_array(env, argv[1], &is) != napi_ok || !is || napi_get_array_length(env, argv[1], &n) != napi_ok ||
      n > Q8_EW_MAX_INPUTS) {
    napi_throw_type_error(env, NULL, "q8hip: inputs must be an array of at most 8 device buffers");
    return NULL;
  }
  const void* ins[Q8_EW_MAX_INPUTS] = {0};
  int64_t nums[Q8_EW_MAX_INPUTS] = {0};
  uint32_t nn = 0;
  if (!arg_i64_array(env, argv[2], nums, Q8_EW_MAX_INPUTS, &nn)) return NULL;
  if (nn != n || (int64_t)n != prog.ninputs) {
    napi_throw_range_error(env, NULL, "q8hip: inputs / inNumel do not match the program");
    return NULL;
  }
  for (uint32_t i = 0; i < n; i++) {
    napi_value e;
    void* p = NULL;
    if (napi_get_element(env, argv[1], i, &e) != napi_ok ||
        !arg_buf_n(env, e, 0, nbytes(nums[i], elem_bytes(prog.in_dtype[i]), 1), "ewise input", &p))
      return NULL;
    ins[i] = p;
  }
  Q8_CHECK(env, q8_ewise(&prog, ins, nums, out, onum, g_stream));
  return undefined(env);
}

static napi_value js_ewise_prog_bytes(napi_env env, napi_callback_info info) {
  (void)info;
  napi_value r;
  NAPI_CALL(env, napi_create_int32(env, (int32_t)sizeof(q8_ew_prog), &r));
  return r;
}

static napi_value init_module(napi_env env, napi_value exports) {
  const struct {
    const char* name;
    napi_callback fn;
  } fns[] = {
      {"version", js_version},
      {"lastError", js_last_error},
      {"deviceCount", js_device_count},
      {"init", js_init},
      {"captureBegin", js_capture_begin},
      {"captureEnd", js_capture_end},
      {"graphLaunch", js_graph_launch},
      {"graphDestroy", js_graph_destroy},
      {"alloc", js_alloc},
      {"free", js_free},
      {"bytes", js_bytes},
      {"upload", js_upload},
      {"download", js_download},
      {"sync", js_sync},
      {"syncAsync", js_sync_async},
      {"fillNormal", js_fill_normal},
      {"fillUniform", js_fill_uniform},
      {"quantizeStatic", js_quantize_static},
      {"quantizeRows", js_quantize_rows},
      {"dequantize", js_dequantize},
      {"packWeight", js_pack_weight},
      {"gemm", js_gemm},
      {"gemmRequant", js_gemm_requant},
      {"qlinearDynamic", js_qlinear_dynamic},
      {"packWeightInt4", js_pack_weight_int4},
      {"gemvW4", js_gemv_w4},
      {"siluMulQuantizeRows", js_silu_mul_quantize_rows},
      {"convWorkspace", js_conv_workspace},
      {"quantizedConv", js_quantized_conv},
      {"quantizedConvEx", js_quantized_conv_ex},
      {"convWeightTaps", js_conv_weight_taps},
      {"quantizedConvPrepacked", js_quantized_conv_prepacked},
      {"quantizedDotWorkspace", js_quantized_dot_workspace},
      {"quantizedDot", js_quantized_dot},
      {"ewise", js_ewise},
      {"ewiseProgBytes", js_ewise_prog_bytes},
  };
  for (size_t i = 0; i < sizeof(fns) / sizeof(fns[0]); ++i) {
    napi_value f;
    NAPI_CALL(env, napi_create_function(env, fns[i].name, NAPI_AUTO_LENGTH, fns[i].fn, NULL, &f));
    NAPI_CALL(env, napi_set_named_property(env, exports, fns[i].name, f));
  }
  const struct {
    const char* name;
    int value;
  } consts[] = {
      {"Q8_I8", Q8_I8}, {"Q8_U8", Q8_U8}, {"Q8_I32", Q8_I32}, {"Q8_F32", Q8_F32}, {"Q8_F64", Q8_F64},
      {"Q8_PER_TENSOR", Q8_PER_TENSOR}, {"Q8_PER_TOKEN", Q8_PER_TOKEN},
      {"Q8_PER_CHANNEL", Q8_PER_CHANNEL}, {"Q8_EPI_PT", Q8_EPI_PT}, {"Q8_EPI_ROWCOL", Q8_EPI_ROWCOL},
      {"Q8_ACT_NONE", Q8_ACT_NONE}, {"Q8_ACT_RELU", Q8_ACT_RELU}, {"Q8_ACT_SILU", Q8_ACT_SILU},
  };
  for (size_t i = 0; i < sizeof(consts) / sizeof(consts[0]); ++i) {
    napi_value v;
    NAPI_CALL(env, napi_create_int32(env, consts[i].value, &v));
    NAPI_CALL(env, napi_set_named_property(env, exports, consts[i].name, v));
  }
  return exports;
}

NAPI_MODULE(NODE_GYP_MODULE_NAME, init_module)
