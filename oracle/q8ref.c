/*
 * q8ref.c -- CPU oracle (plain C restatement) of mlfw's int8 inference path.
 * TEST INFRASTRUCTURE ONLY; see q8ref.h for the rules and the notation.
 *
 * Reference files followed (paths relative to the reference checkout):
 *   src/util/random.ts:5-14                    mulberry32
 *   src/nn/init.ts:31-52                       uniform_, normal_ (Box-Muller)
 *   src/compiler/analysis/calibration.ts:24-34 ValueObserver min/max
 *   src/compiler/ir/graph/quantization_types.ts scales (S-*), R2, clampRange
 *   src/compiler/passes/lowering/quant_math.ts R1 (:16-27), D1 (:29-34)
 *   src/compiler/passes/lowering/rules/quantization.ts:57-76  M1
 *   src/backend/cpu/codegen.ts                 fround / Math.round / |0 rules
 *   src/compiler/passes/quantization/quantization_pass.ts:335-355, :431-456
 *   src/compiler/passes/decompose/decomposition_pass.ts:197-203, :224-230
 */
#include "q8ref.h"

#include <math.h>
#include <stddef.h>
#include <stdlib.h>

/* ------------------------------------------------------------------ */
/* rounding primitives                                                 */
/* ------------------------------------------------------------------ */

/* Math.fround: binary32 round-to-nearest-even of a double. */
float q8r_fround(double v) { return (float)v; }

/* ECMA-262 Math.round: nearest integer, ties toward +infinity.
 * floor(y) + (y - floor(y) >= 0.5); y - floor(y) is exact for every double
 * (the fraction keeps y's low bits), and NaN / +-inf fall through
 * unchanged because the comparison with NaN is false.  A zero result keeps
 * the sign of y (Math.round(-0.3) is -0). */
double q8r_js_round(double y) {
  double r = floor(y);
  r = (y - r >= 0.5) ? r + 1.0 : r;
  return r == 0.0 ? copysign(0.0, y) : r;
}

/* ------------------------------------------------------------------ */
/* seeded inputs                                                       */
/* ------------------------------------------------------------------ */

/* makeRng(seed): a = seed >>> 0  (random.ts:5-6) */
void q8r_rng_seed(q8r_rng* r, uint32_t seed) { r->a = seed; }

/* next() (random.ts:7-13).  Math.imul and `| 0` are multiplication and
 * addition modulo 2^32, `>>>` is a logical shift of the 32-bit pattern. */
double q8r_rng_next(q8r_rng* r) {
  r->a += 0x6D2B79F5u;
  uint32_t a = r->a;
  uint32_t t = (a ^ (a >> 15)) * (1u | a);
  t = (t + ((t ^ (t >> 7)) * (61u | t))) ^ t;
  return (double)(t ^ (t >> 14)) / 4294967296.0;
}

/* normal_(tensor, mean, std) (init.ts:40-52): pairs of draws, the second
 * draw of an odd tail is consumed and its sine discarded. */
void q8r_fill_normal(q8r_rng* r, float* out, int64_t n, double mean, double std) {
  for (int64_t i = 0; i < n; i += 2) {
    double u1 = q8r_rng_next(r);
    if (u1 == 0.0) u1 = 1e-10;                  /* random() || 1e-10 */
    double u2 = q8r_rng_next(r);
    double rad = sqrt(-2.0 * log(u1));
    double theta = 6.283185307179586 * u2;
    out[i] = (float)(mean + std * rad * cos(theta));
    if (i + 1 < n) out[i + 1] = (float)(mean + std * rad * sin(theta));
  }
}

/* uniform_(tensor, a, b) (init.ts:31-37) */
void q8r_fill_uniform(q8r_rng* r, float* out, int64_t n, double a, double b) {
  double range = b - a;
  for (int64_t i = 0; i < n; i++) out[i] = (float)(a + q8r_rng_next(r) * range);
}

void q8r_apply_outliers(float* x, int64_t n, uint32_t seed, double p, double factor) {
  q8r_rng r;
  q8r_rng_seed(&r, seed);
  for (int64_t i = 0; i < n; i++)
    if (q8r_rng_next(&r) < p) x[i] = (float)((double)x[i] * factor);
}

/* ------------------------------------------------------------------ */
/* scales                                                              */
/* ------------------------------------------------------------------ */

/* JS Math.max(a, b) for two doubles: NaN if either is NaN. */
static double js_max(double a, double b) {
  if (a != a || b != b) return NAN;
  if (a == b) return (signbit(a) && !signbit(b)) ? b : a;  /* max(-0, +0) = +0 */
  return a > b ? a : b;
}
static double js_min(double a, double b) {
  if (a != a || b != b) return NAN;
  if (a == b) return signbit(a) ? a : b;                    /* min(-0, +0) = -0 */
  return a < b ? a : b;
}
/* `v || 1e-10` for a number: 0, -0 and NaN are falsy. */
static double or_tiny(double v) { return (v == 0.0 || v != v) ? 1e-10 : v; }

/* fromRange(min, max, PER_TENSOR_SYMMETRIC) (quantization_types.ts:249-253) */
double q8r_scale_sym_from_range(double mn, double mx, int num_bits) {
  double absmax = js_max(fabs(mn), fabs(mx));
  double bound = ldexp(1.0, num_bits - 1) - 1.0;
  return or_tiny(absmax / bound);
}

/* fromRange(min, max, asymmetric) (quantization_types.ts:256-263) */
void q8r_params_asym_from_range(double mn, double mx, int is_ui8, int num_bits,
                                double* scale, double* zero_point) {
  double cmin = is_ui8 ? 0.0 : -ldexp(1.0, num_bits - 1);
  double cmax = is_ui8 ? ldexp(1.0, num_bits) - 1.0 : ldexp(1.0, num_bits - 1) - 1.0;
  double range = or_tiny(mx - mn);
  double s = range / (cmax - cmin);
  double zp = q8r_js_round(cmin - mn / s);
  *scale = s;
  *zero_point = js_max(cmin, js_min(cmax, zp));
}

/* ValueObserver.update (calibration.ts:24-34) */
void q8r_observe_minmax(const float* x, int64_t n, double* mn, double* mx) {
  double lo = INFINITY, hi = -INFINITY;
  for (int64_t i = 0; i < n; i++) {
    double v = x[i];
    if (v < lo) lo = v;
    if (v > hi) hi = v;
  }
  *mn = lo;
  *mx = hi;
}

/* fromConstantArray (quantization_types.ts:287-297), symmetric scheme */
double q8r_scale_const_array(const float* x, int64_t n, int num_bits) {
  double mn, mx;
  q8r_observe_minmax(x, n, &mn, &mx);
  if (!isfinite(mn)) mn = -1.0;
  if (!isfinite(mx)) mx = 1.0;
  if (mn == mx) { mn -= 0.5; mx += 0.5; }
  return q8r_scale_sym_from_range(mn, mx, num_bits);
}

/* fromConstantArrayPerChannel (:299-317) + fromRangePerChannel (:266-281) */
void q8r_scales_per_channel(const float* w, int64_t rows, int64_t cols, int axis,
                            int num_bits, double* scales) {
  int64_t nch = axis == 0 ? rows : cols;
  double bound = ldexp(1.0, num_bits - 1) - 1.0;
  for (int64_t c = 0; c < nch; c++) {
    double mn = INFINITY, mx = -INFINITY;
    int64_t cnt = axis == 0 ? cols : rows;
    for (int64_t j = 0; j < cnt; j++) {
      double v = axis == 0 ? w[c * cols + j] : w[j * cols + c];
      if (v < mn) mn = v;
      if (v > mx) mx = v;
    }
    if (!isfinite(mn)) mn = -1.0;
    if (!isfinite(mx)) mx = 1.0;
    if (mn == mx) { mn -= 0.5; mx += 0.5; }
    scales[c] = or_tiny(js_max(fabs(mn), fabs(mx)) / bound);
  }
}

/* fromConstantArrayPerGroup (:319-340) */
void q8r_scales_per_group(const float* x, int64_t n, int64_t group, int num_bits,
                          double* scales) {
  double bound = ldexp(1.0, num_bits - 1) - 1.0;
  int64_t ng = (n + group - 1) / group;
  for (int64_t g = 0; g < ng; g++) {
    int64_t start = g * group, end = start + group < n ? start + group : n;
    double absmax = 0.0;
    for (int64_t i = start; i < end; i++) {
      double a = fabs((double)x[i]);
      if (a > absmax) absmax = a;
    }
    scales[g] = or_tiny(absmax / bound);
  }
}

static double scale_observed(const float* x, int64_t n) {
  if (n == 0) return 6.0 / 127.0;          /* no data: defaultForActivation */
  double mn, mx;
  q8r_observe_minmax(x, n, &mn, &mx);
  return q8r_scale_sym_from_range(mn, mx, 8);
}

void q8r_scales_per_token(const float* x, int64_t M, int64_t K, double* scales) {
  for (int64_t m = 0; m < M; m++) scales[m] = scale_observed(x + m * K, K);
}

double q8r_scale_per_tensor_dynamic(const float* x, int64_t n) {
  return scale_observed(x, n);
}

/* ------------------------------------------------------------------ */
/* R1: compiled quantize                                               */
/* ------------------------------------------------------------------ */

/* (Math.min(Math.max(Math.round(Math.fround(x / s)), cMin), cMax) | 0)
 * with the zero-point form Math.round(Math.fround(Math.fround(x/s) + zp)). */
int q8r_quantize_value(float x, double s, double zp, int is_ui8) {
  double y = (double)q8r_fround((double)x / s);
  if (zp != 0.0) y = (double)q8r_fround(y + zp);
  double r = q8r_js_round(y);
  double lo = is_ui8 ? 0.0 : -128.0, hi = is_ui8 ? 255.0 : 127.0;
  r = js_min(js_max(r, lo), hi);
  if (r != r) return 0;                     /* NaN | 0 == 0 */
  return (int)r;
}

void q8r_quantize(const float* x, int64_t n, double s, double zp, int is_ui8, void* q) {
  if (is_ui8) {
    uint8_t* o = (uint8_t*)q;
    for (int64_t i = 0; i < n; i++) o[i] = (uint8_t)q8r_quantize_value(x[i], s, zp, 1);
  } else {
    int8_t* o = (int8_t*)q;
    for (int64_t i = 0; i < n; i++) o[i] = (int8_t)q8r_quantize_value(x[i], s, zp, 0);
  }
}

void q8r_quantize_rows(const float* x, int64_t M, int64_t K, const double* scales, int8_t* q) {
  for (int64_t m = 0; m < M; m++)
    for (int64_t k = 0; k < K; k++)
      q[m * K + k] = (int8_t)q8r_quantize_value(x[m * K + k], scales[m], 0.0, 0);
}

/* ------------------------------------------------------------------ */
/* R2: host weight quantize                                            */
/* ------------------------------------------------------------------ */

void q8r_clamp_range(int symmetric, int is_ui8, int num_bits, int* lo, int* hi) {
  if (symmetric) {
    int bound = (1 << (num_bits - 1)) - 1;
    *lo = -bound;
    *hi = bound;
  } else if (is_ui8) {
    *lo = 0;
    *hi = (1 << num_bits) - 1;
  } else {
    *lo = -(1 << (num_bits - 1));
    *hi = (1 << (num_bits - 1)) - 1;
  }
}

/* Math.max(cMin, Math.min(cMax, Math.round(w / s + zp))); a NaN result
 * becomes 0 when the constant is materialized into an Int8Array. */
int q8r_weight_quantize_value(double w, double s, double zp, int lo, int hi) {
  double r = js_max((double)lo, js_min((double)hi, q8r_js_round(w / s + zp)));
  if (r != r) return 0;
  return (int)r;
}

void q8r_weight_quantize_per_channel(const float* w, int64_t rows, int64_t cols, int axis,
                                     const double* scales, int8_t* q) {
  /* clampRange of a PER_CHANNEL params object: not symmetric -> [-128,127] */
  for (int64_t r = 0; r < rows; r++)
    for (int64_t c = 0; c < cols; c++) {
      double s = scales[axis == 0 ? r : c];
      q[r * cols + c] = (int8_t)q8r_weight_quantize_value(w[r * cols + c], s, 0.0, -128, 127);
    }
}

void q8r_weight_quantize_per_tensor(const float* w, int64_t n, double s, int lo, int hi,
                                    int8_t* q) {
  for (int64_t i = 0; i < n; i++) q[i] = (int8_t)q8r_weight_quantize_value(w[i], s, 0.0, lo, hi);
}

void q8r_weight_quantize_per_group(const float* w, int64_t n, int64_t group,
                                   const double* scales, int lo, int hi, int8_t* q) {
  for (int64_t i = 0; i < n; i++)
    q[i] = (int8_t)q8r_weight_quantize_value(w[i], scales[i / group], 0.0, lo, hi);
}

/* ------------------------------------------------------------------ */
/* D1: compiled dequantize                                             */
/* ------------------------------------------------------------------ */

/* Math.fround((+q) * s)  /  Math.fround(Math.fround((+q) - zp) * s) */
float q8r_dequantize_value(double q, double s, double zp) {
  if (zp != 0.0) q = (double)q8r_fround(q - zp);
  return q8r_fround(q * s);
}

void q8r_dequantize_i8(const int8_t* q, int64_t n, double s, double zp, float* y) {
  for (int64_t i = 0; i < n; i++) y[i] = q8r_dequantize_value((double)q[i], s, zp);
}
void q8r_dequantize_u8(const uint8_t* q, int64_t n, double s, double zp, float* y) {
  for (int64_t i = 0; i < n; i++) y[i] = q8r_dequantize_value((double)q[i], s, zp);
}
void q8r_dequantize_i32(const int32_t* q, int64_t n, double s, double zp, float* y) {
  for (int64_t i = 0; i < n; i++) y[i] = q8r_dequantize_value((double)q[i], s, zp);
}
void q8r_dequantize_rows_i8(const int8_t* q, int64_t M, int64_t K, const double* scales, float* y) {
  for (int64_t m = 0; m < M; m++)
    for (int64_t k = 0; k < K; k++)
      y[m * K + k] = q8r_dequantize_value((double)q[m * K + k], scales[m], 0.0);
}

/* ------------------------------------------------------------------ */
/* M1: quantized_dot                                                   */
/* ------------------------------------------------------------------ */

/* The JS kernel keeps `_acc` as a double; every partial sum is an integer
 * far below 2^53, so the double sum is exact, and the Int32Array store
 * wraps it modulo 2^32.  An int64 sum followed by the same wrap is equal. */
/* An operand element as the lowering's CastNode(load, dtype, 'i32') reads
 * it: an Int8Array (i8) or Uint8Array (ui8) element. */
static int64_t q8r_elem(const int8_t* p, int64_t i, int u8) {
  return u8 ? (int64_t)((const uint8_t*)p)[i] : (int64_t)p[i];
}

void q8r_quantized_dot_ex(const int8_t* A, int a_u8, const int8_t* B, int b_u8, int64_t M,
                          int64_t N, int64_t K, int b_layout, int32_t zpA, int32_t zpB,
                          int32_t* acc) {
  for (int64_t m = 0; m < M; m++)
    for (int64_t n = 0; n < N; n++) {
      int64_t s = 0;
      for (int64_t k = 0; k < K; k++) {
        int64_t a = q8r_elem(A, m * K + k, a_u8) - zpA;
        int64_t b = q8r_elem(B, b_layout == 0 ? k * N + n : n * K + k, b_u8) - zpB;
        s += a * b;
      }
      acc[m * N + n] = (int32_t)(uint32_t)(uint64_t)s;
    }
}

void q8r_quantized_dot(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                       int b_layout, int32_t zpA, int32_t zpB, int32_t* acc) {
  q8r_quantized_dot_ex(A, 0, B, 0, M, N, K, b_layout, zpA, zpB, acc);
}

/* quantized_conv: the loop nest buildConvNest emits
 * (lowering_registry.ts:335-449) -- zero-init the output, then for every
 * (n, oc, output position, ic, kernel position) add the guarded product
 * (x - zpx) * (w - zpw) (rules/quantization.ts:44-62), 0 for a tap in the
 * padding.  The JS accumulation is exact (|sum| < 2^53), the store is
 * ToInt32. */
void q8r_quantized_conv_ex(const int8_t* x, int x_u8, const int8_t* w, int w_u8, int d,
                           const int64_t* x_shape, const int64_t* w_shape, const int64_t* strides,
                           const int64_t* pad_lo, const int64_t* pad_hi, const int64_t* dilation,
                           int64_t groups, int32_t zpx, int32_t zpw, int32_t* out) {
  const int64_t N = x_shape[0], C = x_shape[1], O = w_shape[0], Cg = w_shape[1];
  const int64_t Og = O / groups;
  int64_t S[3] = {1, 1, 1}, K[3] = {1, 1, 1}, P[3] = {1, 1, 1};
  int64_t st[3] = {1, 1, 1}, lo[3] = {0, 0, 0}, dl[3] = {1, 1, 1};
  for (int i = 0; i < d; i++) {
    S[i] = x_shape[2 + i];
    K[i] = w_shape[2 + i];
    st[i] = strides[i];
    lo[i] = pad_lo[i];
    dl[i] = dilation[i];
    P[i] = (S[i] + pad_lo[i] + pad_hi[i] - ((K[i] - 1) * dilation[i] + 1)) / strides[i] + 1;
  }
  const int64_t Sn = S[0] * S[1] * S[2], Kn = K[0] * K[1] * K[2], Pn = P[0] * P[1] * P[2];
  for (int64_t n = 0; n < N; n++)
    for (int64_t o = 0; o < O; o++) {
      const int64_t g = o / Og;
      for (int64_t p0 = 0; p0 < P[0]; p0++)
        for (int64_t p1 = 0; p1 < P[1]; p1++)
          for (int64_t p2 = 0; p2 < P[2]; p2++) {
            int64_t acc = 0;
            for (int64_t ic = 0; ic < Cg; ic++) {
              const int8_t* xc = x + (n * C + g * Cg + ic) * Sn;
              const int8_t* wc = w + (o * Cg + ic) * Kn;
              for (int64_t k0 = 0; k0 < K[0]; k0++) {
                const int64_t s0 = p0 * st[0] + k0 * dl[0] - lo[0];
                if (s0 < 0 || s0 >= S[0]) continue;
                for (int64_t k1 = 0; k1 < K[1]; k1++) {
                  const int64_t s1 = p1 * st[1] + k1 * dl[1] - lo[1];
                  if (s1 < 0 || s1 >= S[1]) continue;
                  for (int64_t k2 = 0; k2 < K[2]; k2++) {
                    const int64_t s2 = p2 * st[2] + k2 * dl[2] - lo[2];
                    if (s2 < 0 || s2 >= S[2]) continue;
                    const int64_t a = q8r_elem(xc, (s0 * S[1] + s1) * S[2] + s2, x_u8) - zpx;
                    const int64_t b = q8r_elem(wc, (k0 * K[1] + k1) * K[2] + k2, w_u8) - zpw;
                    acc += a * b;
                  }
                }
              }
            }
            out[((n * O + o) * P[0] + p0) * P[1] * P[2] + p1 * P[2] + p2] =
                (int32_t)(uint32_t)(uint64_t)acc;
          }
    }
  (void)Pn;
}

void q8r_quantized_conv(const int8_t* x, const int8_t* w, int d, const int64_t* x_shape,
                        const int64_t* w_shape, const int64_t* strides, const int64_t* pad_lo,
                        const int64_t* pad_hi, const int64_t* dilation, int64_t groups,
                        int32_t zpx, int32_t zpw, int32_t* out) {
  q8r_quantized_conv_ex(x, 0, w, 0, d, x_shape, w_shape, strides, pad_lo, pad_hi, dilation, groups,
                        zpx, zpw, out);
}

/* W4A8 per-group GEMV as defined in q8ref.h: exact per-group integer
 * sums, then an f64 sum over groups in ascending order. */
void q8r_gemv_w4(const int8_t* xq, const double* sx, int64_t sx_stride, const uint8_t* wq4,
                 const double* sw, int64_t M, int64_t N, int64_t K, int64_t group,
                 const float* bias, int act, float* y) {
  const int64_t G = K / group, KB = (K + 1) / 2;
  for (int64_t m = 0; m < M; m++)
    for (int64_t n = 0; n < N; n++) {
      double S = 0.0;
      for (int64_t g = 0; g < G; g++) {
        int64_t acc = 0;
        for (int64_t k = g * group; k < (g + 1) * group; k++) {
          const int nib = (wq4[n * KB + k / 2] >> (4 * (k & 1))) & 0xF;
          const int q = nib >= 8 ? nib - 16 : nib;
          acc += (int64_t)xq[m * K + k] * q;
        }
        const double t = (double)acc * sw[n * G + g];
        S = g == 0 ? t : S + t;
      }
      float v = q8r_fround(S * sx[m * sx_stride]);
      if (bias) v = q8r_fround((double)v + (double)bias[n]);
      if (act == 1) v = q8r_relu(v);
      else if (act == 2) v = q8r_silu(v);
      y[m * N + n] = v;
    }
}

/* ------------------------------------------------------------------ */
/* epilogues and elementwise                                           */
/* ------------------------------------------------------------------ */

/* Math.max(v, 0) on a float: NaN stays NaN, -0 and negatives give +0. */
float q8r_relu(float v) {
  if (v != v) return v;
  return v > 0.0f ? v : 0.0f;
}

/* silu(x) = x * (1 / (1 + exp(-x))), each f32 op rounded:
 * Math.fround(x * Math.fround(1 / Math.fround(1 + Math.fround(Math.exp(-x))))) */
float q8r_silu(float x) {
  float e = q8r_fround(exp(-(double)x));
  float d = q8r_fround(1.0 + (double)e);
  float r = q8r_fround(1.0 / (double)d);
  return q8r_fround((double)x * (double)r);
}

float q8r_mul(float a, float b) { return q8r_fround((double)a * (double)b); }

void q8r_silu_mul(const float* g, const float* u, int64_t n, float* h) {
  for (int64_t i = 0; i < n; i++) h[i] = q8r_mul(q8r_silu(g[i]), u[i]);
}

void q8r_epilogue(const int32_t* acc, int64_t M, int64_t N, int mode,
                  const double* sA, int64_t sA_stride, const double* sB, int64_t sB_stride,
                  double s_out, const float* bias, int act, float* y) {
  for (int64_t m = 0; m < M; m++)
    for (int64_t n = 0; n < N; n++) {
      double a = (double)acc[m * N + n];
      float v;
      if (mode == 0) {
        v = q8r_fround(a * s_out);
      } else {
        float sv = q8r_fround(sA[m * sA_stride] * sB[n * sB_stride]);
        v = q8r_fround(a * (double)sv);
      }
      if (bias) v = q8r_fround((double)v + (double)bias[n]);
      if (act == 1) v = q8r_relu(v);
      else if (act == 2) v = q8r_silu(v);
      y[m * N + n] = v;
    }
}

/* ------------------------------------------------------------------ */
/* calibration observers (src/compiler/analysis/calibration.ts)        */
/* ------------------------------------------------------------------ */

void q8r_observer_init(q8r_observer* o, double* bins, int num_bins, int has_hist) {
  o->min = INFINITY;
  o->max = -INFINITY;
  o->count = 0.0;
  o->has_hist = has_hist;
  o->num_bins = num_bins;
  o->initialized = 0;
  o->range_min = 0.0;
  o->range_max = 0.0;
  o->total_count = 0.0;
  o->bins = bins;
  if (bins)
    for (int i = 0; i < num_bins; i++) bins[i] = 0.0;
}

/* Math.min(numBins - 1, Math.floor((v - lo) * scale)); NaN maps to -1 (a
 * typed-array store at a NaN index is dropped). */
static int64_t bin_of(double v, double lo, double scale, int num_bins) {
  double f = floor((v - lo) * scale);
  if (f != f) return -1;
  return f < (double)(num_bins - 1) ? (int64_t)f : num_bins - 1;
}

/* HistogramCollector.update (:58-80), _initRange (:82-92),
 * _expandAndRebucket (:94-126) */
static void hist_update(q8r_observer* o, const float* x, int64_t n) {
  if (!o->initialized) {
    double mn = INFINITY, mx = -INFINITY;
    for (int64_t i = 0; i < n; i++) {
      double v = x[i];
      if (v < mn) mn = v;
      if (v > mx) mx = v;
    }
    if (mn == mx) mx = mn + 1.0;
    o->range_min = mn;
    o->range_max = mx;
    o->initialized = 1;
  }
  double range = o->range_max - o->range_min;
  if (range <= 0.0) return;                       /* a NaN range continues, as in JS */
  int outside = 0;
  for (int64_t i = 0; i < n; i++) {
    double v = x[i];
    if (v < o->range_min || v > o->range_max) { outside = 1; break; }
  }
  if (outside) {
    double new_min = o->range_min, new_max = o->range_max;
    for (int64_t i = 0; i < n; i++) {
      double v = x[i];
      if (v < new_min) new_min = v;
      if (v > new_max) new_max = v;
    }
    double old_min = o->range_min, old_range = o->range_max - o->range_min;
    double* old = (double*)malloc(sizeof(double) * (size_t)o->num_bins);
    for (int i = 0; i < o->num_bins; i++) old[i] = o->bins[i];
    o->range_min = new_min;
    o->range_max = new_max;
    double new_scale = o->num_bins / (new_max - new_min);
    for (int i = 0; i < o->num_bins; i++) o->bins[i] = 0.0;
    if (old_range > 0.0) {
      double w = old_range / o->num_bins;
      for (int i = 0; i < o->num_bins; i++) {
        if (old[i] == 0.0) continue;
        double center = old_min + (i + 0.5) * w;
        int64_t b = bin_of(center, new_min, new_scale, o->num_bins);
        if (b >= 0) o->bins[b] += old[i];
      }
    }
    free(old);
    for (int64_t i = 0; i < n; i++) {
      int64_t b = bin_of(x[i], new_min, new_scale, o->num_bins);
      if (b >= 0) o->bins[b] += 1.0;
    }
    o->total_count += (double)n;
    return;
  }
  double scale = o->num_bins / range;
  for (int64_t i = 0; i < n; i++) {
    int64_t b = bin_of(x[i], o->range_min, scale, o->num_bins);
    if (b >= 0) o->bins[b] += 1.0;
  }
  o->total_count += (double)n;
}

/* ValueObserver.update (:24-34) */
void q8r_observer_update(q8r_observer* o, const float* x, int64_t n) {
  for (int64_t i = 0; i < n; i++) {
    double v = x[i];
    if (v < o->min) o->min = v;
    if (v > o->max) o->max = v;
  }
  o->count += (double)n;
  if (o->has_hist) hist_update(o, x, n);
}

/* computePercentileThreshold (:128-139) */
double q8r_hist_percentile(const q8r_observer* o, double percentile) {
  double target = o->total_count * percentile;
  double cum = 0.0;
  double w = (o->range_max - o->range_min) / o->num_bins;
  for (int i = 0; i < o->num_bins; i++) {
    cum += o->bins[i];
    if (cum >= target) return o->range_min + (i + 1) * w;
  }
  return o->range_max;
}

/* computeEntropyThreshold (:141-187) */
double q8r_hist_entropy(const q8r_observer* o, int nq) {
  if (o->total_count == 0.0) return o->range_max;
  int nb = o->num_bins;
  double* ref = (double*)malloc(sizeof(double) * (size_t)nb);
  double* q = (double*)malloc(sizeof(double) * (size_t)nb);
  for (int i = 0; i < nb; i++) ref[i] = o->bins[i] / o->total_count;
  int best_t = nb;
  double best_kl = INFINITY;
  for (int t = nq; t <= nb; t++) {
    double qw = (double)t / nq;
    for (int j = 0; j < t; j++) q[j] = 0.0;
    for (int i = 0; i < nq; i++) {
      int start = (int)floor(i * qw);
      double e = floor((i + 1) * qw);
      int end = e < t ? (int)e : t;
      double sum = 0.0;
      for (int j = start; j < end; j++) sum += ref[j];
      int cnt = end - start;
      if (cnt > 0) {
        double avg = sum / cnt;
        for (int j = start; j < end; j++) q[j] = avg;
      }
    }
    double kl = 0.0;
    for (int i = 0; i < t; i++)
      if (ref[i] > 0.0 && q[i] > 0.0) kl += ref[i] * log(ref[i] / q[i]);
    if (kl < best_kl) { best_kl = kl; best_t = t; }
  }
  free(ref);
  free(q);
  double w = (o->range_max - o->range_min) / nb;
  return o->range_min + best_t * w;
}

int q8r_calib_params(const q8r_observer* o, int mode, int scheme, int is_ui8,
                     double* scale, double* zero_point) {
  if (o->count == 0.0) return 0;                  /* getRange -> null */
  int asymmetric = scheme == 1;                   /* PER_TENSOR_ASYMMETRIC (:253) */
  double lo = o->min, hi = o->max;
  if (!asymmetric && o->has_hist && mode == 1) {
    double t = q8r_hist_percentile(o, 0.999);
    lo = -t; hi = t;
  } else if (!asymmetric && o->has_hist && mode == 2) {
    double t = q8r_hist_entropy(o, is_ui8 ? 256 : 255);
    lo = -t; hi = t;
  }
  if (scheme != 0) {                              /* fromRange, non-symmetric branch */
    q8r_params_asym_from_range(lo, hi, is_ui8, 8, scale, zero_point);
  } else {
    *scale = q8r_scale_sym_from_range(lo, hi, 8);
    *zero_point = 0.0;
  }
  return 1;
}
