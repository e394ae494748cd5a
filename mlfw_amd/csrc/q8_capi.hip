// q8_capi.hip -- the extern "C" boundary (include/q8hip.h).
//
// Every entry point validates its arguments on the host before launching
// anything, reports failures as a status code plus a thread-local message
// (the terac convention, terac/include/Tera/CAPI/Execution.h:55), and
// enqueues its kernels on the caller's stream.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

#include "../../include/q8hip.h"
#include "q8_internal.h"

namespace {

thread_local char g_err[1024] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(e == hipErrorOutOfMemory ? Q8_ERR_OOM : Q8_ERR_DEVICE, "%s: %s (%d)", what,
              hipGetErrorString(e), (int)e);
}

// Per-device state: initialised once.  The library allocates no device
// memory for the ops: per-tensor reductions keep their keys in the caller's
// scales output and workspaces come from the caller.  The one exception is
// `scratch` below, a file-scope device array (no allocation call) that only
// q8_qlinear_dynamic_noalloc uses.
constexpr int kMaxDevices = 64;
struct DevState {
  std::atomic<int> ready{0};
  unsigned char* scratch = nullptr;   // this device's copy of `scratch`
};
DevState g_dev[kMaxDevices];
std::mutex g_init_mu;

// Staging of q8_qlinear_dynamic_noalloc: the int8 codes of x and their f64
// scales.  Every device the library runs on holds its own copy until the
// process ends.  In host code the name is only a stand-in for the symbol:
// its device address comes from hipGetSymbolAddress (g_dev[dev].scratch).
static __device__ __align__(256) unsigned char scratch[Q8_NOALLOC_SCRATCH_BYTES];

int init_device(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return fail(Q8_ERR_INVALID, "device %d out of range", dev);
  if (g_dev[dev].ready.load(std::memory_order_acquire)) return Q8_OK;
  std::lock_guard<std::mutex> lk(g_init_mu);
  if (g_dev[dev].ready.load(std::memory_order_relaxed)) return Q8_OK;
  hipDeviceProp_t prop;
  hipError_t e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(Q8_ERR_DEVICE, "device %d is %s; this library is built for gfx950 only", dev,
                prop.gcnArchName);
  int cur = 0;
  e = hipGetDevice(&cur);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return hip_fail(e, "hipSetDevice");
  e = q8::setup_kernel_attributes();
  if (e == hipSuccess) e = q8::setup_w4_attributes();
  (void)q8::cu_count();
  void* sp = nullptr;
  if (e == hipSuccess) e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
  if (cur != dev) (void)hipSetDevice(cur);
  if (e != hipSuccess) return hip_fail(e, "device set-up");
  if (sp == nullptr) return fail(Q8_ERR_DEVICE, "device %d: no address for the scratch array", dev);
  g_dev[dev].scratch = static_cast<unsigned char*>(sp);
  g_dev[dev].ready.store(1, std::memory_order_release);
  return Q8_OK;
}

// Initialise the calling thread's current device on first use; `scratch`
// (may be NULL) receives that device's address of the scratch array.
int ensure_current(unsigned char** scratch_out = nullptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice (no HIP device?)");
  int rc = init_device(dev);
  if (rc != Q8_OK) return rc;
  if (scratch_out) *scratch_out = g_dev[dev].scratch;
  return Q8_OK;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return hip_fail(e, what);
  g_err[0] = '\0';
  return Q8_OK;
}

bool mul_ok(int64_t a, int64_t b) { return a >= 0 && b >= 0 && (b == 0 || a <= INT64_MAX / b); }

#define Q8_REQUIRE(cond, ...) \
  do {                        \
    if (!(cond)) return fail(Q8_ERR_INVALID, __VA_ARGS__); \
  } while (0)

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ---- calibration scale selection (host side of the observer) ----

// JS Math.max / Math.min on doubles (NaN wins; max(-0,+0) = +0).
double js_max(double a, double b) {
  if (std::isnan(a) || std::isnan(b)) return NAN;
  if (a == b) return std::signbit(a) ? b : a;
  return a > b ? a : b;
}
double js_min(double a, double b) {
  if (std::isnan(a) || std::isnan(b)) return NAN;
  if (a == b) return std::signbit(a) ? a : b;
  return a < b ? a : b;
}
// `v || 1e-10` for a number.
double or_tiny(double v) { return (v == 0.0 || std::isnan(v)) ? 1e-10 : v; }
// Math.round: floor(y + 0.5) computed without the double-rounding of y + 0.5.
double js_round(double y) {
  if (!std::isfinite(y)) return y;
  const double f = std::floor(y);
  const double r = (y - f >= 0.5) ? f + 1.0 : f;
  return (r == 0.0 && std::signbit(y)) ? -0.0 : r;
}

// QuantizationParams.fromRange, 8 bits (quantization_types.ts:248-263).
void params_from_range(double mn, double mx, bool symmetric, bool is_u8, double* scale,
                       double* zp) {
  if (symmetric) {
    *scale = or_tiny(js_max(std::fabs(mn), std::fabs(mx)) / 127.0);
    *zp = 0.0;
    return;
  }
  const double cmin = is_u8 ? 0.0 : -128.0, cmax = is_u8 ? 255.0 : 127.0;
  const double s = or_tiny(mx - mn) / (cmax - cmin);
  *scale = s;
  *zp = js_max(cmin, js_min(cmax, js_round(cmin - mn / s)));
}

// computePercentileThreshold (calibration.ts:128-139).
double hist_percentile(const double* bins, int nb, double lo, double hi, double total, double p) {
  const double target = total * p, w = (hi - lo) / nb;
  double cum = 0.0;
  for (int i = 0; i < nb; ++i) {
    cum += bins[i];
    if (cum >= target) return lo + (i + 1) * w;
  }
  return hi;
}

// computeEntropyThreshold (calibration.ts:141-187): the threshold bin count
// t in [nq, nb] whose nq-level requantisation of bins[0..t) has the least
// KL divergence from the normalised histogram.  Every sum is formed left to
// right, in the reference's order, so the chosen t matches it exactly.
double hist_entropy(const double* bins, int nb, double lo, double hi, double total, int nq) {
  if (total == 0.0) return hi;
  std::vector<double> ref(nb), q(nb);
  for (int i = 0; i < nb; ++i) ref[i] = bins[i] / total;
  int best_t = nb;
  double best_kl = INFINITY;
  for (int t = nq; t <= nb; ++t) {
    const double qw = (double)t / nq;
    for (int j = 0; j < t; ++j) q[j] = 0.0;
    for (int i = 0; i < nq; ++i) {
      const int start = (int)std::floor(i * qw);
      const double e = std::floor((i + 1) * qw);
      const int end = e < t ? (int)e : t;
      double sum = 0.0;
      for (int j = start; j < end; ++j) sum += ref[j];
      if (end > start) {
        const double avg = sum / (end - start);
        for (int j = start; j < end; ++j) q[j] = avg;
      }
    }
    double kl = 0.0;
    for (int i = 0; i < t; ++i)
      if (ref[i] > 0.0 && q[i] > 0.0) kl += ref[i] * std::log(ref[i] / q[i]);
    if (kl < best_kl) {
      best_kl = kl;
      best_t = t;
    }
  }
  return lo + best_t * ((hi - lo) / nb);
}

}  // namespace

extern "C" {

int q8_version(void) { return Q8HIP_VERSION; }

const char* q8_last_error(void) { return g_err; }

int q8_device_count(int* count) {
  Q8_REQUIRE(count != nullptr, "q8_device_count: count is NULL");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) n = 0;
  else if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  *count = n;
  return Q8_OK;
}

int q8_init(int device) {
  int n = 0;
  int rc = q8_device_count(&n);
  if (rc != Q8_OK) return rc;
  if (n == 0) return fail(Q8_ERR_DEVICE, "q8_init: no HIP device is visible");
  if (device < 0 || device >= n)
    return fail(Q8_ERR_INVALID, "q8_init: device %d out of range (%d visible)", device, n);
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  return init_device(device);
}

int q8_alloc(void** dptr, size_t bytes) {
  Q8_REQUIRE(dptr != nullptr, "q8_alloc: dptr is NULL");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  *dptr = nullptr;
  if (bytes == 0) return Q8_OK;
  hipError_t e = hipMalloc(dptr, bytes);
  return launched(e, "hipMalloc");
}

int q8_free(void* dptr) {
  if (dptr == nullptr) return Q8_OK;
  return launched(hipFree(dptr), "hipFree");
}

int q8_h2d(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return Q8_OK;
  Q8_REQUIRE(dst && src, "q8_h2d: NULL pointer");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream));
  if (e == hipSuccess) e = hipStreamSynchronize(as_stream(stream));
  return launched(e, "q8_h2d");
}

int q8_d2h(void* dst, const void* src, size_t bytes, void* stream) {
  if (bytes == 0) return Q8_OK;
  Q8_REQUIRE(dst && src, "q8_d2h: NULL pointer");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream));
  if (e == hipSuccess) e = hipStreamSynchronize(as_stream(stream));
  return launched(e, "q8_d2h");
}

int q8_memset(void* dst, int value, size_t bytes, void* stream) {
  if (bytes == 0) return Q8_OK;
  Q8_REQUIRE(dst != nullptr, "q8_memset: dst is NULL");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  // a fill kernel, not hipMemsetAsync: callers may capture this in a HIP graph
  return launched(q8::launch_fill_u8(dst, value, (int64_t)bytes, as_stream(stream)), "q8_memset");
}

int q8_stream_sync(void* stream) {
  return launched(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
}

int q8_stream_create(void** stream) {
  Q8_REQUIRE(stream != nullptr, "q8_stream_create: stream is NULL");
  *stream = nullptr;
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  hipStream_t s = nullptr;
  // default priority; non-blocking so the legacy null stream never joins it
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_fail(e, "hipStreamCreateWithFlags");
  *stream = s;
  return launched(hipSuccess, "q8_stream_create");
}

int q8_stream_destroy(void* stream) {
  if (stream == nullptr) return Q8_OK;
  return launched(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
}

int q8_graph_capture_begin(void* stream) {
  Q8_REQUIRE(stream != nullptr, "q8_graph_capture_begin: capture needs a created stream, not the null stream");
  return launched(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal),
                  "hipStreamBeginCapture");
}

int q8_graph_capture_end(void* stream, void** graph_exec) {
  Q8_REQUIRE(stream != nullptr && graph_exec != nullptr, "q8_graph_capture_end: NULL argument");
  *graph_exec = nullptr;
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(as_stream(stream), &g);
  if (e != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    return hip_fail(e, "hipStreamEndCapture");
  }
  hipGraphExec_t x = nullptr;
  e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
  *graph_exec = x;
  return launched(hipSuccess, "q8_graph_capture_end");
}

int q8_graph_launch(void* graph_exec, void* stream) {
  Q8_REQUIRE(graph_exec != nullptr, "q8_graph_launch: graph_exec is NULL");
  return launched(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), as_stream(stream)), "hipGraphLaunch");
}

int q8_graph_destroy(void* graph_exec) {
  if (graph_exec == nullptr) return Q8_OK;
  return launched(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)), "hipGraphExecDestroy");
}

int q8_fill_normal(float* out, int64_t n, uint32_t seed, uint64_t offset, double mean,
                   double std, void* stream) {
  Q8_REQUIRE(n >= 0, "q8_fill_normal: n < 0");
  Q8_REQUIRE(n == 0 || out, "q8_fill_normal: out is NULL");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_fill_normal(out, n, seed, offset, mean, std, as_stream(stream)),
                  "q8_fill_normal launch");
}

int q8_fill_uniform(float* out, int64_t n, uint32_t seed, uint64_t offset, double a, double b,
                    void* stream) {
  Q8_REQUIRE(n >= 0, "q8_fill_uniform: n < 0");
  Q8_REQUIRE(n == 0 || out, "q8_fill_uniform: out is NULL");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_fill_uniform(out, n, seed, offset, a, b, as_stream(stream)),
                  "q8_fill_uniform launch");
}

int q8_apply_outliers(float* x, int64_t n, uint32_t seed, double p, double factor, void* stream) {
  Q8_REQUIRE(n >= 0, "q8_apply_outliers: n < 0");
  Q8_REQUIRE(n == 0 || x, "q8_apply_outliers: x is NULL");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_apply_outliers(x, n, seed, p, factor, as_stream(stream)),
                  "q8_apply_outliers launch");
}

int q8_quantize_static(const float* x, int64_t n, double scale, double zero_point, int target,
                       void* q, void* stream) {
  Q8_REQUIRE(n >= 0, "q8_quantize_static: n < 0");
  Q8_REQUIRE(n == 0 || (x && q), "q8_quantize_static: NULL pointer");
  Q8_REQUIRE(target == Q8_I8 || target == Q8_U8,
             "q8_quantize_static: target must be Q8_I8 or Q8_U8 (got %d)", target);
  // quantize op verifier: `scale <= 0` is rejected (ops/quantization.ts:44-47)
  Q8_REQUIRE(!(scale <= 0.0), "q8_quantize_static: quantize scale must be positive (got %g)", scale);
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_quant_static(x, n, scale, zero_point, target == Q8_U8, q,
                                          as_stream(stream)),
                  "q8_quantize_static launch");
}

int q8_quantize_rows(const float* x, int64_t M, int64_t K, int mode, int8_t* q, double* scales,
                     void* stream) {
  Q8_REQUIRE(M >= 0 && K >= 0 && mul_ok(M, K), "q8_quantize_rows: bad shape [%lld,%lld]",
             (long long)M, (long long)K);
  Q8_REQUIRE(mode == Q8_PER_TOKEN || mode == Q8_PER_TENSOR,
             "q8_quantize_rows: mode must be Q8_PER_TOKEN or Q8_PER_TENSOR (got %d)", mode);
  Q8_REQUIRE(scales != nullptr || (mode == Q8_PER_TOKEN && M == 0), "q8_quantize_rows: scales is NULL");
  Q8_REQUIRE(M * K == 0 || (x && q), "q8_quantize_rows: NULL pointer");
  Q8_REQUIRE((reinterpret_cast<uintptr_t>(scales) & 7) == 0,
             "q8_quantize_rows: scales must be 8-byte aligned");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  hipError_t e = mode == Q8_PER_TOKEN
                     ? q8::launch_quant_rows(x, K, M, K, q, scales, as_stream(stream))
                     : q8::launch_quant_tensor(x, M * K, q, scales, as_stream(stream));
  return launched(e, "q8_quantize_rows launch");
}

int q8_quantize_rows_ld(const float* x, int64_t ldx, int64_t M, int64_t K, int8_t* q,
                        double* scales, void* stream) {
  Q8_REQUIRE(M >= 0 && K >= 0 && mul_ok(M, K), "q8_quantize_rows_ld: bad shape [%lld,%lld]",
             (long long)M, (long long)K);
  Q8_REQUIRE(ldx >= K && mul_ok(M, ldx), "q8_quantize_rows_ld: row stride %lld must be >= K (%lld)",
             (long long)ldx, (long long)K);
  Q8_REQUIRE(M == 0 || scales, "q8_quantize_rows_ld: scales is NULL");
  Q8_REQUIRE(M * K == 0 || (x && q), "q8_quantize_rows_ld: NULL pointer");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_quant_rows(x, ldx, M, K, q, scales, as_stream(stream)),
                  "q8_quantize_rows_ld launch");
}

int q8_dequantize(const void* q, int src, int64_t M, int64_t K, const double* scales,
                  int granularity, double zero_point, float* y, void* stream) {
  Q8_REQUIRE(M >= 0 && K >= 0 && mul_ok(M, K), "q8_dequantize: bad shape [%lld,%lld]",
             (long long)M, (long long)K);
  Q8_REQUIRE(src == Q8_I8 || src == Q8_U8 || src == Q8_I32,
             "q8_dequantize: src must be Q8_I8, Q8_U8 or Q8_I32 (got %d)", src);
  Q8_REQUIRE(granularity == Q8_PER_TENSOR || granularity == Q8_PER_TOKEN,
             "q8_dequantize: granularity must be Q8_PER_TENSOR or Q8_PER_TOKEN (got %d)", granularity);
  Q8_REQUIRE(M * K == 0 || (q && y && scales), "q8_dequantize: NULL pointer");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_dequant(q, src, M, K, scales, granularity == Q8_PER_TOKEN,
                                     zero_point, y, as_stream(stream)),
                  "q8_dequantize launch");
}

int q8_pack_weight(const float* W, int64_t rows, int64_t cols, int axis, int granularity,
                   int8_t* Wq, double* scales, void* stream) {
  Q8_REQUIRE(rows >= 0 && cols >= 0 && mul_ok(rows, cols), "q8_pack_weight: bad shape [%lld,%lld]",
             (long long)rows, (long long)cols);
  Q8_REQUIRE(axis == 0 || axis == 1, "q8_pack_weight: axis must be 0 or 1 (got %d)", axis);
  Q8_REQUIRE(granularity == Q8_PER_CHANNEL || granularity == Q8_PER_TENSOR,
             "q8_pack_weight: granularity must be Q8_PER_CHANNEL or Q8_PER_TENSOR (got %d)",
             granularity);
  Q8_REQUIRE(rows * cols == 0 || (W && Wq), "q8_pack_weight: NULL pointer");
  Q8_REQUIRE(scales != nullptr, "q8_pack_weight: scales is NULL");
  Q8_REQUIRE((reinterpret_cast<uintptr_t>(scales) & 7) == 0,
             "q8_pack_weight: scales must be 8-byte aligned");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_pack_weight(W, rows, cols, axis, granularity == Q8_PER_TENSOR, Wq,
                                         scales, as_stream(stream)),
                  "q8_pack_weight launch");
}

static int gemm_common(const char* who, const int8_t* A, const int8_t* B, int64_t M, int64_t N,
                       int64_t K, int32_t zpA, int32_t zpB, const double* sA, int sA_mode,
                       const double* sB, int sB_mode, int epi, double s_out, const float* bias,
                       int act, int out_kind, void* out, q8::GemmEpi* e) {
  Q8_REQUIRE(M >= 0 && N >= 0 && K >= 0 && mul_ok(M, N) && mul_ok(M, K) && mul_ok(N, K),
             "%s: bad shape M=%lld N=%lld K=%lld", who, (long long)M, (long long)N, (long long)K);
  Q8_REQUIRE(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31),
             "%s: dimensions must be below 2^31", who);
  Q8_REQUIRE(out_kind == Q8_F32 || out_kind == Q8_I32, "%s: out_kind must be Q8_F32 or Q8_I32", who);
  Q8_REQUIRE(act == Q8_ACT_NONE || act == Q8_ACT_RELU || act == Q8_ACT_SILU, "%s: bad act %d", who, act);
  Q8_REQUIRE(epi == Q8_EPI_PT || epi == Q8_EPI_ROWCOL, "%s: bad epi %d", who, epi);
  Q8_REQUIRE(M * N == 0 || out, "%s: out is NULL", who);
  Q8_REQUIRE(M * N * K == 0 || (A && B), "%s: NULL operand", who);
  if (zpA != 0 || zpB != 0)
    return fail(Q8_ERR_UNSUPPORTED, "%s: non-zero zero points are not supported by this build", who);
  e->sA = sA;
  e->sB = sB;
  e->sA_stride = 0;
  e->sB_stride = 0;
  e->s_out = s_out;
  e->bias = bias;
  e->mode = epi == Q8_EPI_ROWCOL ? 1 : 0;
  e->act = act;
  e->out_i32 = out_kind == Q8_I32;
  e->out_q8 = 0;
  e->s_q = 0.0;
  e->rq32 = 0.0f;
  e->q_fast = 0;
  if (out_kind == Q8_F32 && epi == Q8_EPI_ROWCOL) {
    Q8_REQUIRE(sA && sB, "%s: ROWCOL epilogue needs sA and sB", who);
    Q8_REQUIRE(sA_mode == Q8_PER_TENSOR || sA_mode == Q8_PER_TOKEN, "%s: bad sA_mode %d", who, sA_mode);
    Q8_REQUIRE(sB_mode == Q8_PER_TENSOR || sB_mode == Q8_PER_CHANNEL, "%s: bad sB_mode %d", who, sB_mode);
    e->sA_stride = sA_mode == Q8_PER_TOKEN ? 1 : 0;
    e->sB_stride = sB_mode == Q8_PER_CHANNEL ? 1 : 0;
  }
  if (out_kind == Q8_I32)
    Q8_REQUIRE(bias == nullptr && act == Q8_ACT_NONE, "%s: Q8_I32 output takes no bias or activation", who);
  return Q8_OK;
}

int q8_gemm(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K, int32_t zpA,
            int32_t zpB, const double* sA, int sA_mode, const double* sB, int sB_mode, int epi,
            double s_out, const float* bias, int act, int out_kind, void* out, void* stream) {
  q8::GemmEpi e{};
  int rc = gemm_common("q8_gemm", A, B, M, N, K, zpA, zpB, sA, sA_mode, sB, sB_mode, epi, s_out,
                       bias, act, out_kind, out, &e);
  if (rc != Q8_OK) return rc;
  rc = ensure_current();
  if (rc != Q8_OK) return rc;
  hipError_t err = (M <= 16) ? q8::launch_gemv(A, B, M, N, K, e, out, as_stream(stream))
                             : q8::launch_gemm(A, B, M, N, K, e, out, as_stream(stream));
  return launched(err, "q8_gemm launch");
}

int q8_glu_interleave(const int8_t* Wg, const double* sg, const float* bg, const int8_t* Wu,
                      const double* su, const float* bu, int64_t F, int64_t K, int8_t* W, double* s,
                      float* b, void* stream) {
  Q8_REQUIRE(F >= 0 && K >= 0 && mul_ok(2 * F, K), "q8_glu_interleave: bad shape F=%lld K=%lld",
             (long long)F, (long long)K);
  Q8_REQUIRE(F % 32 == 0, "q8_glu_interleave: F (%lld) must be a multiple of 32", (long long)F);
  Q8_REQUIRE(F == 0 || (sg && su && s && (K == 0 || (Wg && Wu && W))), "q8_glu_interleave: NULL pointer");
  Q8_REQUIRE((bg == nullptr) == (bu == nullptr) && (bg == nullptr) == (b == nullptr),
             "q8_glu_interleave: give both biases and the output bias, or none");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_glu_interleave(Wg, Wu, sg, su, bg, bu, F, K, W, s, b, as_stream(stream)),
                  "q8_glu_interleave launch");
}

int q8_gemm_glu_workspace(int64_t M, int64_t F, int64_t K, size_t* bytes) {
  Q8_REQUIRE(M >= 0 && F >= 0 && K >= 0 && mul_ok(M, 8 * F), "q8_gemm_glu_workspace: bad shape");
  Q8_REQUIRE(bytes != nullptr, "q8_gemm_glu_workspace: bytes is NULL");
  *bytes = q8::gemm_glu_ws_bytes(M, F, K);
  return Q8_OK;
}

int q8_gemm_glu(const int8_t* A, const int8_t* B, int64_t M, int64_t F, int64_t K, const double* sA,
                int sA_mode, const double* sB, int sB_mode, const float* bias, float* h, void* workspace,
                size_t workspace_bytes, void* stream) {
  Q8_REQUIRE(F >= 0 && F % 32 == 0, "q8_gemm_glu: F (%lld) must be a multiple of 32", (long long)F);
  Q8_REQUIRE(mul_ok(M, 2 * F), "q8_gemm_glu: bad shape");
  q8::GemmEpi e{};
  int rc = gemm_common("q8_gemm_glu", A, B, M, 2 * F, K, 0, 0, sA, sA_mode, sB, sB_mode, Q8_EPI_ROWCOL, 0.0,
                       bias, Q8_ACT_NONE, Q8_F32, h, &e);
  if (rc != Q8_OK) return rc;
  const size_t need = q8::gemm_glu_ws_bytes(M, F, K);
  Q8_REQUIRE(need == 0 || (workspace && workspace_bytes >= need),
             "q8_gemm_glu: needs a workspace of %zu bytes (got %zu)", need, workspace_bytes);
  rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_gemm_glu(A, B, M, F, K, e, h, workspace, as_stream(stream)), "q8_gemm_glu launch");
}

int q8_generic_gemm_launches(int64_t* count) {
  Q8_REQUIRE(count != nullptr, "q8_generic_gemm_launches: count is NULL");
  *count = (int64_t)q8::g_generic_gemm_launches.load(std::memory_order_relaxed);
  return Q8_OK;
}

int q8_gemv(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K, const double* sA,
            int sA_mode, const double* sB, int sB_mode, int epi, double s_out, const float* bias,
            int act, int out_kind, void* out, void* stream) {
  Q8_REQUIRE(M >= 0 && M <= 16, "q8_gemv: M must be in [0, 16] (got %lld)", (long long)M);
  q8::GemmEpi e{};
  int rc = gemm_common("q8_gemv", A, B, M, N, K, 0, 0, sA, sA_mode, sB, sB_mode, epi, s_out, bias,
                       act, out_kind, out, &e);
  if (rc != Q8_OK) return rc;
  rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_gemv(A, B, M, N, K, e, out, as_stream(stream)), "q8_gemv launch");
}

// Workspace of q8_quantized_dot: int8 copies of ui8 operands, then the
// row sums the zero-point correction needs, each 256-byte aligned.
namespace {
struct QdotPlan {
  size_t a_off, b_off, rs_off, cs_off, bytes;
  bool a_u8, b_u8, need_rs, need_cs;
  int32_t cA, cB;
};
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
QdotPlan qdot_plan(int64_t M, int64_t N, int64_t K, int a_dtype, int b_dtype, int32_t zpA,
                   int32_t zpB) {
  QdotPlan p{};
  p.a_u8 = a_dtype == Q8_U8;
  p.b_u8 = b_dtype == Q8_U8;
  p.cA = (p.a_u8 ? 128 : 0) - zpA;
  p.cB = (p.b_u8 ? 128 : 0) - zpB;
  p.need_rs = p.cB != 0;
  p.need_cs = p.cA != 0;
  size_t off = 0;
  p.a_off = off; if (p.a_u8) off = align256(off + (size_t)(M * K));
  p.b_off = off; if (p.b_u8) off = align256(off + (size_t)(N * K));
  p.rs_off = off; if (p.need_rs) off = align256(off + 4 * (size_t)M);
  p.cs_off = off; if (p.need_cs) off = align256(off + 4 * (size_t)N);
  p.bytes = off;
  return p;
}
}  // namespace

int q8_quantized_dot_workspace(int64_t M, int64_t N, int64_t K, int a_dtype, int b_dtype,
                               int32_t zpA, int32_t zpB, size_t* bytes) {
  Q8_REQUIRE(M >= 0 && N >= 0 && K >= 0 && mul_ok(M, K) && mul_ok(N, K) && mul_ok(M, N),
             "q8_quantized_dot_workspace: bad shape M=%lld N=%lld K=%lld", (long long)M,
             (long long)N, (long long)K);
  Q8_REQUIRE((a_dtype == Q8_I8 || a_dtype == Q8_U8) && (b_dtype == Q8_I8 || b_dtype == Q8_U8),
             "q8_quantized_dot_workspace: operands must be Q8_I8 or Q8_U8");
  Q8_REQUIRE(bytes != nullptr, "q8_quantized_dot_workspace: bytes is NULL");
  *bytes = qdot_plan(M, N, K, a_dtype, b_dtype, zpA, zpB).bytes;
  return Q8_OK;
}

int q8_quantized_dot(const void* A, int a_dtype, const void* B, int b_dtype, int64_t M,
                     int64_t N, int64_t K, int32_t zpA, int32_t zpB, void* workspace,
                     size_t workspace_bytes, int32_t* out, void* stream) {
  Q8_REQUIRE((a_dtype == Q8_I8 || a_dtype == Q8_U8) && (b_dtype == Q8_I8 || b_dtype == Q8_U8),
             "q8_quantized_dot: operands must be Q8_I8 or Q8_U8 (got %d, %d)", a_dtype, b_dtype);
  q8::GemmEpi e{};
  int rc = gemm_common("q8_quantized_dot", (const int8_t*)A, (const int8_t*)B, M, N, K, 0, 0,
                       nullptr, Q8_PER_TENSOR, nullptr, Q8_PER_TENSOR, Q8_EPI_PT, 0.0, nullptr,
                       Q8_ACT_NONE, Q8_I32, out, &e);
  if (rc != Q8_OK) return rc;
  const QdotPlan p = qdot_plan(M, N, K, a_dtype, b_dtype, zpA, zpB);
  Q8_REQUIRE(p.bytes == 0 || (workspace && workspace_bytes >= p.bytes),
             "q8_quantized_dot: needs a workspace of %zu bytes (got %zu)", p.bytes, workspace_bytes);
  rc = ensure_current();
  if (rc != Q8_OK) return rc;
  if (M * N == 0) return Q8_OK;
  hipStream_t st = as_stream(stream);
  int8_t* ws = static_cast<int8_t*>(workspace);
  const int8_t* a = static_cast<const int8_t*>(A);
  const int8_t* b = static_cast<const int8_t*>(B);
  hipError_t err = hipSuccess;
  if (p.a_u8 && err == hipSuccess) {
    err = q8::launch_flip_u8(static_cast<const uint8_t*>(A), ws + p.a_off, M * K, st);
    a = ws + p.a_off;
  }
  if (p.b_u8 && err == hipSuccess) {
    err = q8::launch_flip_u8(static_cast<const uint8_t*>(B), ws + p.b_off, N * K, st);
    b = ws + p.b_off;
  }
  int32_t* rs = p.need_rs ? reinterpret_cast<int32_t*>(ws + p.rs_off) : nullptr;
  int32_t* cs = p.need_cs ? reinterpret_cast<int32_t*>(ws + p.cs_off) : nullptr;
  if (rs && err == hipSuccess) err = q8::launch_row_sums_i8(a, M, K, rs, st);
  if (cs && err == hipSuccess) err = q8::launch_row_sums_i8(b, N, K, cs, st);
  if (err == hipSuccess)
    err = (M <= 16) ? q8::launch_gemv(a, b, M, N, K, e, out, st) : q8::launch_gemm(a, b, M, N, K, e, out, st);
  if (err == hipSuccess && (p.cA != 0 || p.cB != 0))
    err = q8::launch_zp_correct(out, M, N, rs, cs, p.cA, p.cB, K, st);
  return launched(err, "q8_quantized_dot launch");
}

// Body of the dynamic linear once the arguments are checked; xq / sx are
// the caller's outputs (q8_qlinear_dynamic) or the scratch staging
// (q8_qlinear_dynamic_noalloc).
static hipError_t qlinear_dynamic_run(const float* x, int64_t M, int64_t K, int x_mode,
                                      const int8_t* Wq, const double* sW, int64_t N,
                                      const float* bias, int act, float* out, int8_t* xq,
                                      double* sx, q8::GemmEpi& e, hipStream_t st) {
  if (M * N == 0 && M * K == 0) return hipSuccess;
  if (N > 0 && q8::qlinear_fused_ok(x, Wq, M, K))
    return q8::launch_qlinear_fused(x, M, K, x_mode == Q8_PER_TENSOR ? 1 : 0, Wq, sW,
                                    e.sB_stride, N, bias, act, out, sx, xq, st);
  hipError_t err = x_mode == Q8_PER_TOKEN ? q8::launch_quant_rows(x, K, M, K, xq, sx, st)
                                          : q8::launch_quant_tensor(x, M * K, xq, sx, st);
  if (err != hipSuccess || M * N == 0) return err;
  e.sA = sx;
  return (M <= 16) ? q8::launch_gemv(xq, Wq, M, N, K, e, out, st)
                   : q8::launch_gemm(xq, Wq, M, N, K, e, out, st);
}

int q8_qlinear_dynamic(const float* x, int64_t M, int64_t K, int x_mode, const int8_t* Wq,
                       const double* sW, int sW_mode, int64_t N, const float* bias, int act,
                       float* out, int8_t* xq, double* sx, void* stream) {
  Q8_REQUIRE(x_mode == Q8_PER_TOKEN || x_mode == Q8_PER_TENSOR,
             "q8_qlinear_dynamic: x_mode must be Q8_PER_TOKEN or Q8_PER_TENSOR (got %d)", x_mode);
  q8::GemmEpi e{};
  int rc = gemm_common("q8_qlinear_dynamic", xq, Wq, M, N, K, 0, 0, sx, x_mode, sW, sW_mode,
                       Q8_EPI_ROWCOL, 0.0, bias, act, Q8_F32, out, &e);
  if (rc != Q8_OK) return rc;
  Q8_REQUIRE(M * K == 0 || x, "q8_qlinear_dynamic: x is NULL");
  Q8_REQUIRE((reinterpret_cast<uintptr_t>(sx) & 7) == 0,
             "q8_qlinear_dynamic: sx must be 8-byte aligned");
  rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(qlinear_dynamic_run(x, M, K, x_mode, Wq, sW, N, bias, act, out, xq, sx, e,
                                      as_stream(stream)),
                  "q8_qlinear_dynamic launch");
}

int q8_qlinear_dynamic_noalloc(const float* x, int64_t M, int64_t K, int x_mode,
                               const int8_t* Wq, const double* sW, int sW_mode, int64_t N,
                               const float* bias, int act, float* out, void* stream) {
  Q8_REQUIRE(x_mode == Q8_PER_TOKEN || x_mode == Q8_PER_TENSOR,
             "q8_qlinear_dynamic_noalloc: x_mode must be Q8_PER_TOKEN or Q8_PER_TENSOR (got %d)",
             x_mode);
  Q8_REQUIRE(M >= 0 && K >= 0 && mul_ok(M, K), "q8_qlinear_dynamic_noalloc: bad shape [%lld,%lld]",
             (long long)M, (long long)K);
  // staging: codes at offset 0, scales at the next 256-byte boundary
  const int64_t codes = (M * K + 255) / 256 * 256;
  const int64_t nsc = x_mode == Q8_PER_TOKEN ? M : 1;
  Q8_REQUIRE(M <= (int64_t)Q8_NOALLOC_SCRATCH_BYTES &&
                 codes + 8 * nsc <= (int64_t)Q8_NOALLOC_SCRATCH_BYTES,
             "q8_qlinear_dynamic_noalloc: x of [%lld,%lld] needs %lld bytes of staging; the "
             "scratch holds %lld (use q8_qlinear_dynamic with caller buffers)",
             (long long)M, (long long)K, (long long)(codes + 8 * nsc),
             (long long)Q8_NOALLOC_SCRATCH_BYTES);
  // a stand-in, non-NULL, 8-aligned pointer lets gemm_common check the
  // other arguments; the real staging addresses are set below
  int8_t* const fake_xq = reinterpret_cast<int8_t*>(static_cast<uintptr_t>(256));
  double* const fake_sx = reinterpret_cast<double*>(static_cast<uintptr_t>(256));
  q8::GemmEpi e{};
  int rc = gemm_common("q8_qlinear_dynamic_noalloc", fake_xq, Wq, M, N, K, 0, 0, fake_sx, x_mode,
                       sW, sW_mode, Q8_EPI_ROWCOL, 0.0, bias, act, Q8_F32, out, &e);
  if (rc != Q8_OK) return rc;
  Q8_REQUIRE(M * K == 0 || x, "q8_qlinear_dynamic_noalloc: x is NULL");
  unsigned char* sp = nullptr;
  rc = ensure_current(&sp);
  if (rc != Q8_OK) return rc;
  int8_t* xq = reinterpret_cast<int8_t*>(sp);
  double* sx = reinterpret_cast<double*>(sp + codes);
  return launched(qlinear_dynamic_run(x, M, K, x_mode, Wq, sW, N, bias, act, out, xq, sx, e,
                                      as_stream(stream)),
                  "q8_qlinear_dynamic_noalloc launch");
}

int q8_gemm_requant(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                    const double* sA, int sA_mode, const double* sB, int sB_mode, int epi,
                    double s_out, const float* bias, int act, double s_next, int8_t* out,
                    void* stream) {
  q8::GemmEpi e{};
  int rc = gemm_common("q8_gemm_requant", A, B, M, N, K, 0, 0, sA, sA_mode, sB, sB_mode, epi,
                       s_out, bias, act, Q8_F32, out, &e);
  if (rc != Q8_OK) return rc;
  // the `quantize` op's verifier (ops/quantization.ts:44-47): scale > 0
  Q8_REQUIRE(s_next > 0.0 && std::isfinite(s_next),
             "q8_gemm_requant: s_next must be a finite scale > 0 (got %g)", s_next);
  e.out_q8 = 1;
  e.s_q = s_next;
  e.rq32 = (float)(1.0 / s_next);
  e.q_fast = (s_next >= 0x1p-100 && s_next <= 0x1p100) ? 1 : 0;
  rc = ensure_current();
  if (rc != Q8_OK) return rc;
  hipError_t err = (M <= 16) ? q8::launch_gemv(A, B, M, N, K, e, out, as_stream(stream))
                             : q8::launch_gemm(A, B, M, N, K, e, out, as_stream(stream));
  return launched(err, "q8_gemm_requant launch");
}

// Route of q8_gemm_requant_dynamic: the fused kernel needs the
// MFMA GEMM (M > 16, K a multiple of 16, 256-row tile offsets in 32 bits)
// and every 256 x 256 tile resident at once.
static bool dq_fused_route(int64_t M, int64_t N, int64_t K) {
  return M > 16 && K > 0 && K % 16 == 0 && 256 * K < (1LL << 31) && q8::gemm_dq_fits(M, N);
}

static size_t dq_fallback_bytes(int64_t M, int64_t N) { return (size_t)((M * N * 4 + 255) / 256 * 256); }

int q8_gemm_requant_dynamic_workspace(int64_t M, int64_t N, int64_t K, size_t* bytes, int* fused) {
  Q8_REQUIRE(M >= 0 && N >= 0 && K >= 0 && mul_ok(M, N) && mul_ok(M, 4 * N),
             "q8_gemm_requant_dynamic_workspace: bad shape M=%lld N=%lld K=%lld", (long long)M,
             (long long)N, (long long)K);
  Q8_REQUIRE(bytes != nullptr, "q8_gemm_requant_dynamic_workspace: bytes is NULL");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  const bool f = dq_fused_route(M, N, K);
  *bytes = f ? q8::gemm_dq_ws_bytes(M) : dq_fallback_bytes(M, N);
  if (fused) *fused = f ? 1 : 0;
  return Q8_OK;
}

int q8_gemm_requant_dynamic(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                            const double* sA, int sA_mode, const double* sB, int sB_mode, int epi,
                            double s_out, const float* bias, int act, int8_t* out,
                            double* out_scales, void* workspace, size_t workspace_bytes,
                            void* stream) {
  q8::GemmEpi e{};
  int rc = gemm_common("q8_gemm_requant_dynamic", A, B, M, N, K, 0, 0, sA, sA_mode, sB, sB_mode, epi,
                       s_out, bias, act, Q8_F32, out, &e);
  if (rc != Q8_OK) return rc;
  Q8_REQUIRE(M == 0 || out_scales, "q8_gemm_requant_dynamic: out_scales is NULL");
  Q8_REQUIRE(mul_ok(M, 4 * N), "q8_gemm_requant_dynamic: bad shape");
  rc = ensure_current();
  if (rc != Q8_OK) return rc;
  if (M == 0) return Q8_OK;
  const bool fused = dq_fused_route(M, N, K);
  const size_t need = fused ? q8::gemm_dq_ws_bytes(M) : dq_fallback_bytes(M, N);
  Q8_REQUIRE(workspace && workspace_bytes >= need,
             "q8_gemm_requant_dynamic: needs a workspace of %zu bytes (got %zu)", need, workspace_bytes);
  hipStream_t st = as_stream(stream);
  if (fused) {
    Q8_REQUIRE((reinterpret_cast<uintptr_t>(A) & 15) == 0 && (reinterpret_cast<uintptr_t>(B) & 15) == 0,
               "q8_gemm_requant_dynamic: the fused route needs 16-byte aligned A and B");
    return launched(q8::launch_gemm_dq(A, B, M, N, K, e, out, out_scales, workspace, st),
                    "q8_gemm_requant_dynamic launch");
  }
  // fp32 result in the workspace, then the per-token quantize of it
  float* y = static_cast<float*>(workspace);
  hipError_t err = (M <= 16) ? q8::launch_gemv(A, B, M, N, K, e, y, st) : q8::launch_gemm(A, B, M, N, K, e, y, st);
  if (err == hipSuccess) err = q8::launch_quant_rows(y, N, M, N, out, out_scales, st);
  return launched(err, "q8_gemm_requant_dynamic launch");
}

int q8_gemm_requant_dynamic_status(const void* workspace, int64_t M, int* timed_out, void* stream) {
  Q8_REQUIRE(workspace && timed_out && M >= 0, "q8_gemm_requant_dynamic_status: NULL argument");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  hipStream_t st = as_stream(stream);
  hipError_t e = hipStreamSynchronize(st);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  const size_t off = q8::gemm_dq_ws_bytes(M) - 256 + 4;
  int v = 0;
  e = hipMemcpy(&v, static_cast<const char*>(workspace) + off, sizeof(int), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpy");
  *timed_out = v;
  return Q8_OK;
}

int q8_debug_ewise_jit(int mode, int64_t* compiled, int64_t* launches) {
  Q8_REQUIRE(mode <= 2, "q8_debug_ewise_jit: mode must be 0, 1 or 2 (or negative to read only)");
  if (mode >= 0) q8::g_ewise_jit_mode.store(mode, std::memory_order_relaxed);
  if (compiled) *compiled = (int64_t)q8::g_ewise_jit_compiled.load(std::memory_order_relaxed);
  if (launches) *launches = (int64_t)q8::g_ewise_jit_launches.load(std::memory_order_relaxed);
  return Q8_OK;
}

int q8_debug_ewise_jit_error(char* buf, size_t cap, size_t* len) {
  const size_t n = q8::ewise_jit_error(buf, cap);
  if (len) *len = n;
  return Q8_OK;
}

int q8_debug_dq_force_timeout(int on) {
  q8::g_dq_force_timeout.store(on ? 1 : 0, std::memory_order_relaxed);
  return Q8_OK;
}

int q8_pack_weight_int4(const float* W, int64_t N, int64_t K, int64_t group_size,
                        uint8_t* Wq4, double* scales, void* stream) {
  Q8_REQUIRE(N >= 0 && K >= 0 && mul_ok(N, K), "q8_pack_weight_int4: bad shape [%lld,%lld]",
             (long long)N, (long long)K);
  Q8_REQUIRE(group_size >= 2 && group_size % 2 == 0 && K % group_size == 0,
             "q8_pack_weight_int4: group_size (%lld) must be even and divide K (%lld)",
             (long long)group_size, (long long)K);
  Q8_REQUIRE(N * (K / 2) < (1LL << 31), "q8_pack_weight_int4: weight too large (%lld x %lld; "
             "q8_gemv_w4 addresses N * K / 2 bytes with 32-bit offsets)", (long long)N, (long long)K);
  Q8_REQUIRE(N * K == 0 || (W && Wq4 && scales), "q8_pack_weight_int4: NULL pointer");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_pack_w4(W, N, K, group_size, Wq4, scales, as_stream(stream)),
                  "q8_pack_weight_int4 launch");
}

int q8_gemv_w4(const int8_t* xq, const double* sx, int sx_mode, const uint8_t* Wq4,
               const double* sw, int64_t M, int64_t N, int64_t K, int64_t group_size,
               const float* bias, int act, float* out, void* stream) {
  Q8_REQUIRE(M >= 0 && N >= 0 && K >= 0 && mul_ok(M, N) && mul_ok(M, K) && mul_ok(N, K),
             "q8_gemv_w4: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  Q8_REQUIRE(M * K < (1LL << 31) && N * (K / 2) < (1LL << 31) && M * N < (1LL << 39),
             "q8_gemv_w4: tensors too large for 32-bit offsets");
  Q8_REQUIRE(group_size >= 2 && group_size % 2 == 0 && K % group_size == 0,
             "q8_gemv_w4: group_size (%lld) must be even and divide K (%lld)",
             (long long)group_size, (long long)K);
  Q8_REQUIRE(sx_mode == Q8_PER_TENSOR || sx_mode == Q8_PER_TOKEN, "q8_gemv_w4: bad sx_mode %d", sx_mode);
  Q8_REQUIRE(act == Q8_ACT_NONE || act == Q8_ACT_RELU || act == Q8_ACT_SILU, "q8_gemv_w4: bad act %d", act);
  Q8_REQUIRE(M * N == 0 || (xq && sx && Wq4 && sw && out), "q8_gemv_w4: NULL pointer");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_gemv_w4(xq, sx, sx_mode == Q8_PER_TOKEN ? 1 : 0, Wq4, sw, M, N, K,
                                     group_size, bias, act, out, as_stream(stream)),
                  "q8_gemv_w4 launch");
}

static int conv_geom(const char* who, int d, const int64_t* xs, const int64_t* ws,
                     const int64_t* strides, const int64_t* pad_lo, const int64_t* pad_hi,
                     const int64_t* dilation, int64_t groups, q8::ConvGeom* G) {
  Q8_REQUIRE(d >= 1 && d <= 3, "%s: spatial_dims must be 1, 2 or 3 (got %d)", who, d);
  Q8_REQUIRE(xs && ws && strides && pad_lo && pad_hi && dilation, "%s: NULL shape array", who);
  constexpr int64_t LIM = (1LL << 31) - 1;
  Q8_REQUIRE(xs[0] >= 0 && xs[1] >= 1 && ws[0] >= 1 && ws[1] >= 1 && xs[0] <= LIM &&
                 xs[1] <= LIM && ws[0] <= LIM && ws[1] <= LIM,
             "%s: bad channel or batch sizes", who);
  Q8_REQUIRE(groups >= 1 && xs[1] % groups == 0 && ws[0] % groups == 0 && ws[1] * groups == xs[1],
             "%s: groups=%lld must divide C=%lld and O=%lld with kernel I = C / groups (I=%lld)", who,
             (long long)groups, (long long)xs[1], (long long)ws[0], (long long)ws[1]);
  G->d = d;
  G->N = xs[0];
  G->C = xs[1];
  G->O = ws[0];
  G->groups = groups;
  G->Cg = (int)ws[1];
  G->Og = (int)(ws[0] / groups);
  int64_t Sn = 1, Kn = 1, Pn = 1;
  for (int i = 0; i < 3; ++i) {
    if (i >= d) {
      G->S[i] = G->K[i] = G->P[i] = 1;
      G->st[i] = 1;
      G->lo[i] = 0;
      G->dl[i] = 1;
      continue;
    }
    const int64_t S = xs[2 + i], K = ws[2 + i];
    Q8_REQUIRE(S >= 1 && S <= LIM && K >= 1 && K <= LIM, "%s: bad spatial size in dim %d", who, i);
    Q8_REQUIRE(strides[i] >= 1 && strides[i] <= LIM && dilation[i] >= 1 && dilation[i] <= LIM,
               "%s: stride and dilation must be >= 1 (dim %d)", who, i);
    Q8_REQUIRE(pad_lo[i] >= 0 && pad_hi[i] >= 0 && pad_lo[i] <= LIM && pad_hi[i] <= LIM,
               "%s: padding must be >= 0 (dim %d)", who, i);
    const int64_t eff = (K - 1) * dilation[i] + 1;
    const int64_t span = S + pad_lo[i] + pad_hi[i] - eff;
    Q8_REQUIRE(span >= 0, "%s: kernel extent %lld exceeds the padded input %lld in dim %d", who,
               (long long)eff, (long long)(S + pad_lo[i] + pad_hi[i]), i);
    const int64_t P = span / strides[i] + 1;
    G->S[i] = (int)S;
    G->K[i] = (int)K;
    G->P[i] = (int)P;
    G->st[i] = strides[i];
    G->lo[i] = pad_lo[i];
    G->dl[i] = dilation[i];
    Q8_REQUIRE(mul_ok(Sn, S) && mul_ok(Kn, K) && mul_ok(Pn, P), "%s: size overflow", who);
    Sn *= S;
    Kn *= K;
    Pn *= P;
  }
  Q8_REQUIRE(Kn <= LIM && mul_ok(Kn, G->Cg) && Kn * G->Cg <= LIM - 16, "%s: contraction too long", who);
  Q8_REQUIRE(mul_ok(G->N * G->C, Sn) && mul_ok(G->N * G->O, Pn) && G->N * G->O * Pn < (1LL << 39) &&
                 mul_ok(Pn, Kn * G->Cg + 16) && Pn * (Kn * G->Cg + 16) < (1LL << 39),
             "%s: tensor too large", who);
  G->Sn = Sn;
  G->Pn = Pn;
  G->Kn = (int)Kn;
  G->Kc = (int)(Kn * G->Cg);
  G->Kc16 = (G->Kc + 15) & ~15;
  return Q8_OK;
}

int q8_quantized_conv_workspace(int spatial_dims, const int64_t* x_shape, const int64_t* w_shape,
                                const int64_t* strides, const int64_t* pad_lo,
                                const int64_t* pad_hi, const int64_t* dilation, int64_t groups,
                                size_t* bytes) {
  Q8_REQUIRE(bytes != nullptr, "q8_quantized_conv_workspace: bytes is NULL");
  q8::ConvGeom G;
  int rc = conv_geom("q8_quantized_conv_workspace", spatial_dims, x_shape, w_shape, strides,
                     pad_lo, pad_hi, dilation, groups, &G);
  if (rc != Q8_OK) return rc;
  *bytes = q8::conv_workspace_bytes(G);
  g_err[0] = '\0';
  return Q8_OK;
}

static int conv_impl(const char* who, const void* x, int x_dtype, const void* w, int w_dtype,
                     const int8_t* w_taps, int spatial_dims, const int64_t* x_shape, const int64_t* w_shape,
                     const int64_t* strides, const int64_t* pad_lo, const int64_t* pad_hi,
                     const int64_t* dilation, int64_t groups, int32_t zp_x, int32_t zp_w,
                     int out_kind, double s_out, void* workspace, size_t workspace_bytes, void* out,
                     void* stream) {
  q8::ConvGeom G;
  int rc = conv_geom(who, spatial_dims, x_shape, w_shape, strides, pad_lo, pad_hi, dilation, groups,
                     &G);
  if (rc != Q8_OK) return rc;
  Q8_REQUIRE(out_kind == Q8_F32 || out_kind == Q8_I32, "%s: out_kind must be Q8_F32 or Q8_I32", who);
  Q8_REQUIRE((x_dtype == Q8_I8 || x_dtype == Q8_U8) && (w_dtype == Q8_I8 || w_dtype == Q8_U8),
             "%s: operands must be Q8_I8 or Q8_U8 (got %d, %d)", who, x_dtype, w_dtype);
  G.zpx = zp_x;
  G.zpw = zp_w;
  G.x_u8 = x_dtype == Q8_U8;
  G.w_u8 = w_dtype == Q8_U8;
  const bool empty = G.N * G.O * G.Pn == 0;
  Q8_REQUIRE(empty || (x && w && out), "%s: NULL pointer", who);
  const size_t need = q8::conv_direct(G) ? 0 : q8::conv_workspace_bytes(G);
  Q8_REQUIRE(empty || workspace_bytes >= need,
             "%s: workspace of %zu bytes is smaller than the %zu bytes required "
             "(q8_quantized_conv_workspace)", who, workspace_bytes, need);
  Q8_REQUIRE(empty || need == 0 || workspace, "%s: workspace is NULL", who);
  q8::GemmEpi e{};
  e.mode = 0;
  e.s_out = s_out;
  e.out_i32 = out_kind == Q8_I32;
  rc = ensure_current();
  if (rc != Q8_OK) return rc;
  if (w_taps) {
    Q8_REQUIRE(q8::conv_taps_used(G), "%s: this weight shape has no tap-major form (q8_conv_weight_taps)", who);
    Q8_REQUIRE((reinterpret_cast<uintptr_t>(w_taps) & 15) == 0, "%s: w_taps must be 16-byte aligned", who);
  }
  return launched(q8::launch_conv(static_cast<const int8_t*>(x), static_cast<const int8_t*>(w), w_taps, G,
                                  e, workspace, out, as_stream(stream)),
                  "quantized_conv launch");
}

int q8_conv_weight_taps(const int8_t* w, int spatial_dims, const int64_t* w_shape, int64_t groups,
                        int8_t* w_taps, void* stream) {
  Q8_REQUIRE(w_shape != nullptr && spatial_dims >= 1 && spatial_dims <= 3,
             "q8_conv_weight_taps: spatial_dims must be 1, 2 or 3 (got %d)", spatial_dims);
  Q8_REQUIRE(groups >= 1 && w_shape[0] > 0 && w_shape[0] % groups == 0 && w_shape[1] > 0,
             "q8_conv_weight_taps: bad weight shape or groups");
  // the geometry of a 1-image input that the kernel fits exactly (only the
  // weight's dimensions matter for the permutation)
  int64_t xs[5] = {1, w_shape[1] * groups, 1, 1, 1}, st[3] = {1, 1, 1}, lo[3] = {0, 0, 0}, dl[3] = {1, 1, 1};
  for (int i = 0; i < spatial_dims; ++i) xs[2 + i] = w_shape[2 + i];
  q8::ConvGeom G;
  int rc = conv_geom("q8_conv_weight_taps", spatial_dims, xs, w_shape, st, lo, lo, dl, groups, &G);
  if (rc != Q8_OK) return rc;
  if (!q8::conv_taps_used(G))
    return fail(Q8_ERR_UNSUPPORTED, "q8_conv_weight_taps: weights of this shape are used as given "
                "(the tap-major form needs channels per group a multiple of 16 and 2..1024 kernel positions)");
  Q8_REQUIRE(w && w_taps && ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(w_taps)) & 15) == 0,
             "q8_conv_weight_taps: w and w_taps must be 16-byte aligned device pointers");
  rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_conv_weight_taps(w, G, w_taps, as_stream(stream)), "q8_conv_weight_taps launch");
}

int q8_quantized_conv(const int8_t* x, const int8_t* w, int spatial_dims, const int64_t* x_shape,
                      const int64_t* w_shape, const int64_t* strides, const int64_t* pad_lo,
                      const int64_t* pad_hi, const int64_t* dilation, int64_t groups,
                      int32_t zp_x, int32_t zp_w, int out_kind, double s_out, void* workspace,
                      size_t workspace_bytes, void* out, void* stream) {
  return conv_impl("q8_quantized_conv", x, Q8_I8, w, Q8_I8, nullptr, spatial_dims, x_shape, w_shape, strides,
                   pad_lo, pad_hi, dilation, groups, zp_x, zp_w, out_kind, s_out, workspace,
                   workspace_bytes, out, stream);
}

int q8_quantized_conv_prepacked(const int8_t* x, const int8_t* w, const int8_t* w_taps, int spatial_dims,
                                const int64_t* x_shape, const int64_t* w_shape, const int64_t* strides,
                                const int64_t* pad_lo, const int64_t* pad_hi, const int64_t* dilation,
                                int64_t groups, int32_t zp_x, int32_t zp_w, int out_kind, double s_out,
                                void* workspace, size_t workspace_bytes, void* out, void* stream) {
  Q8_REQUIRE(w_taps != nullptr, "q8_quantized_conv_prepacked: w_taps is NULL (use q8_quantized_conv)");
  return conv_impl("q8_quantized_conv_prepacked", x, Q8_I8, w, Q8_I8, w_taps, spatial_dims, x_shape, w_shape,
                   strides, pad_lo, pad_hi, dilation, groups, zp_x, zp_w, out_kind, s_out, workspace,
                   workspace_bytes, out, stream);
}

int q8_quantized_conv_ex(const void* x, int x_dtype, const void* w, int w_dtype, int spatial_dims,
                         const int64_t* x_shape, const int64_t* w_shape, const int64_t* strides,
                         const int64_t* pad_lo, const int64_t* pad_hi, const int64_t* dilation,
                         int64_t groups, int32_t zp_x, int32_t zp_w, int out_kind, double s_out,
                         void* workspace, size_t workspace_bytes, void* out, void* stream) {
  return conv_impl("q8_quantized_conv_ex", x, x_dtype, w, w_dtype, nullptr, spatial_dims, x_shape, w_shape,
                   strides, pad_lo, pad_hi, dilation, groups, zp_x, zp_w, out_kind, s_out, workspace,
                   workspace_bytes, out, stream);
}

int q8_silu_mul_quantize_rows_ld(const float* g, int64_t ldg, const float* u, int64_t ldu,
                                 int64_t M, int64_t K, float* h_out, int8_t* q, double* scales,
                                 void* stream) {
  Q8_REQUIRE(M >= 0 && K >= 0 && mul_ok(M, K), "q8_silu_mul_quantize_rows: bad shape");
  Q8_REQUIRE(ldg >= K && ldu >= K && mul_ok(M, ldg) && mul_ok(M, ldu),
             "q8_silu_mul_quantize_rows: row strides (%lld, %lld) must be >= K (%lld)",
             (long long)ldg, (long long)ldu, (long long)K);
  Q8_REQUIRE(M == 0 || scales, "q8_silu_mul_quantize_rows: scales is NULL");
  Q8_REQUIRE(M * K == 0 || (g && u && q), "q8_silu_mul_quantize_rows: NULL pointer");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_silu_mul_quant_rows(g, ldg, u, ldu, M, K, h_out, q, scales,
                                                 as_stream(stream)),
                  "q8_silu_mul_quantize_rows launch");
}

int q8_silu_mul_quantize_rows(const float* g, const float* u, int64_t M, int64_t K, float* h_out,
                              int8_t* q, double* scales, void* stream) {
  return q8_silu_mul_quantize_rows_ld(g, K, u, K, M, K, h_out, q, scales, stream);
}

int q8_ewise(const q8_ew_prog* prog, const void* const* inputs, const int64_t* in_numel,
             void* out, int64_t out_numel, void* stream) {
  Q8_REQUIRE(prog != nullptr, "q8_ewise: prog is NULL");
  Q8_REQUIRE(out_numel >= 0, "q8_ewise: negative out_numel");
  Q8_REQUIRE(prog->ninputs == 0 || (inputs && in_numel), "q8_ewise: inputs / in_numel is NULL");
  const char* why = q8::ewise_check(*prog, in_numel, out_numel);
  Q8_REQUIRE(why == nullptr, "q8_ewise: %s", why);
  if (out_numel > 0) {
    Q8_REQUIRE(out != nullptr, "q8_ewise: out is NULL");
    for (int j = 0; j < prog->ninputs; ++j)
      Q8_REQUIRE(inputs[j] != nullptr, "q8_ewise: input %d is NULL", j);
  }
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_ewise(*prog, inputs, out, out_numel, as_stream(stream)),
                  "q8_ewise launch");
}

int q8_observer_state_bytes(int num_bins, size_t* bytes) {
  Q8_REQUIRE(num_bins >= 1 && num_bins <= Q8_OBS_MAX_BINS,
             "q8_observer_state_bytes: num_bins must be in [1, %d] (got %d)", Q8_OBS_MAX_BINS,
             num_bins);
  Q8_REQUIRE(bytes != nullptr, "q8_observer_state_bytes: bytes is NULL");
  *bytes = q8::obs_state_bytes(num_bins);
  return Q8_OK;
}

int q8_observer_reset(void* state, int num_bins, int histogram, void* stream) {
  Q8_REQUIRE(state != nullptr, "q8_observer_reset: state is NULL");
  Q8_REQUIRE((reinterpret_cast<uintptr_t>(state) & 7) == 0, "q8_observer_reset: state must be 8-byte aligned");
  Q8_REQUIRE(num_bins >= 1 && num_bins <= Q8_OBS_MAX_BINS,
             "q8_observer_reset: num_bins must be in [1, %d] (got %d)", Q8_OBS_MAX_BINS, num_bins);
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_obs_reset(static_cast<q8::ObsState*>(state), num_bins,
                                       histogram ? 1 : 0, as_stream(stream)),
                  "q8_observer_reset launch");
}

int q8_observer_update(void* state, const float* x, int64_t n, void* stream) {
  Q8_REQUIRE(state != nullptr, "q8_observer_update: state is NULL");
  Q8_REQUIRE((reinterpret_cast<uintptr_t>(state) & 7) == 0, "q8_observer_update: state must be 8-byte aligned");
  Q8_REQUIRE(n >= 0, "q8_observer_update: n must be >= 0");
  Q8_REQUIRE(n == 0 || x != nullptr, "q8_observer_update: x is NULL");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  return launched(q8::launch_obs_update(static_cast<q8::ObsState*>(state), x, n, as_stream(stream)),
                  "q8_observer_update launch");
}

int q8_observer_read(const void* state, double* summary, double* bins, void* stream) {
  Q8_REQUIRE(state != nullptr && summary != nullptr, "q8_observer_read: NULL pointer");
  int rc = ensure_current();
  if (rc != Q8_OK) return rc;
  q8::ObsState h;
  hipStream_t s = as_stream(stream);
  hipError_t e = hipMemcpyAsync(&h, state, sizeof(h), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(e, "q8_observer_read");
  if (h.num_bins < 1 || h.num_bins > Q8_OBS_MAX_BINS)
    return fail(Q8_ERR_INVALID, "q8_observer_read: state was not set up by q8_observer_reset");
  const bool any = h.min_key != 0x7fffffff;
  auto key_to_double = [](int k) {
    const int bits = k < 0 ? (k ^ 0x7fffffff) : k;
    float f;
    std::memcpy(&f, &bits, 4);
    return (double)f;
  };
  summary[0] = any ? key_to_double(h.min_key) : INFINITY;
  summary[1] = any ? key_to_double(h.max_key) : -INFINITY;
  summary[2] = (double)h.count;
  summary[3] = h.has_hist;
  summary[4] = h.initialized;
  summary[5] = h.range_min;
  summary[6] = h.range_max;
  summary[7] = (double)h.total_count;
  summary[8] = h.num_bins;
  if (bins) {
    std::vector<unsigned long long> b(h.num_bins);
    const char* src = static_cast<const char*>(state) + q8::Q8_OBS_HEADER;
    e = hipMemcpyAsync(b.data(), src, b.size() * 8, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "q8_observer_read bins");
    for (int i = 0; i < h.num_bins; ++i) bins[i] = (double)b[i];
  }
  g_err[0] = '\0';
  return Q8_OK;
}

static int hist_args(const char* who, const double* summary, const double* bins) {
  Q8_REQUIRE(summary && bins, "%s: NULL pointer", who);
  const double nb = summary[8];
  Q8_REQUIRE(nb >= 1 && nb <= Q8_OBS_MAX_BINS && nb == (int)nb,
             "%s: summary does not come from q8_observer_read", who);
  return Q8_OK;
}

int q8_hist_percentile(const double* summary, const double* bins, double percentile,
                       double* threshold) {
  int rc = hist_args("q8_hist_percentile", summary, bins);
  if (rc != Q8_OK) return rc;
  Q8_REQUIRE(threshold != nullptr, "q8_hist_percentile: threshold is NULL");
  *threshold = hist_percentile(bins, (int)summary[8], summary[5], summary[6], summary[7], percentile);
  return Q8_OK;
}

int q8_hist_entropy(const double* summary, const double* bins, int num_quant_bins,
                    double* threshold) {
  int rc = hist_args("q8_hist_entropy", summary, bins);
  if (rc != Q8_OK) return rc;
  Q8_REQUIRE(threshold != nullptr, "q8_hist_entropy: threshold is NULL");
  Q8_REQUIRE(num_quant_bins >= 1, "q8_hist_entropy: num_quant_bins must be >= 1");
  *threshold = hist_entropy(bins, (int)summary[8], summary[5], summary[6], summary[7], num_quant_bins);
  return Q8_OK;
}

int q8_calib_params(const double* summary, const double* bins, int mode, int scheme,
                    int unsigned_, double* scale, double* zero_point, int* has_params) {
  Q8_REQUIRE(summary && scale && zero_point && has_params, "q8_calib_params: NULL pointer");
  Q8_REQUIRE(mode == Q8_CALIB_MINMAX || mode == Q8_CALIB_PERCENTILE || mode == Q8_CALIB_ENTROPY,
             "q8_calib_params: bad mode %d", mode);
  Q8_REQUIRE(scheme == Q8_SCHEME_PER_TENSOR_SYMMETRIC || scheme == Q8_SCHEME_PER_TENSOR_ASYMMETRIC ||
                 scheme == Q8_SCHEME_PER_CHANNEL,
             "q8_calib_params: bad scheme %d", scheme);
  *has_params = 0;
  if (summary[2] == 0.0) return Q8_OK;                      // getRange -> null
  const bool hist = summary[3] != 0.0 && mode != Q8_CALIB_MINMAX &&
                    scheme != Q8_SCHEME_PER_TENSOR_ASYMMETRIC;
  double lo = summary[0], hi = summary[1];
  if (hist) {
    int rc = hist_args("q8_calib_params", summary, bins);
    if (rc != Q8_OK) return rc;
    const int nb = (int)summary[8];
    const double t = mode == Q8_CALIB_PERCENTILE
                         ? hist_percentile(bins, nb, summary[5], summary[6], summary[7], 0.999)
                         : hist_entropy(bins, nb, summary[5], summary[6], summary[7],
                                        unsigned_ ? 256 : 255);
    lo = -t;
    hi = t;
  }
  params_from_range(lo, hi, scheme == Q8_SCHEME_PER_TENSOR_SYMMETRIC, unsigned_ != 0, scale,
                    zero_point);
  *has_params = 1;
  return Q8_OK;
}

}  // extern "C"
