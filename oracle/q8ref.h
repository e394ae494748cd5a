/*
 * q8ref.h -- CPU oracle for the int8 quantized-inference path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (mlfw_amd/, the HIP
 * library, the Node addon) may include, link or call this code.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * and only as the checker / the timed CPU baseline.
 *
 * Every function restates, in plain C, the arithmetic of one piece of the
 * reference (slexisvn/mlfw, TypeScript).  The reference evaluates all
 * float work as JavaScript doubles and rounds to binary32 only where its
 * generated code calls Math.fround (CPU backend, src/backend/cpu/codegen.ts:
 * 172-174 and 496) or stores into a Float32Array.  This file does the same:
 *   - "fround(v)"  is (float)v with round-to-nearest-even,
 *   - "JSround(y)" is ECMA-262 Math.round: nearest integer, ties toward +inf,
 *   - "ToInt32"    is JS `x | 0` (NaN -> 0, wrap mod 2^32).
 * Build flags must keep IEEE semantics: -ffp-contract=off, no fast-math.
 */
#ifndef Q8REF_H
#define Q8REF_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- seeded inputs: src/util/random.ts:5-14, src/nn/init.ts:31-52 ---- */
typedef struct { uint32_t a; } q8r_rng;
void     q8r_rng_seed(q8r_rng* r, uint32_t seed);
double   q8r_rng_next(q8r_rng* r);
void     q8r_fill_normal(q8r_rng* r, float* out, int64_t n, double mean, double std);
void     q8r_fill_uniform(q8r_rng* r, float* out, int64_t n, double a, double b);

/* C5 outliers: a second stream seeded `seed`; element i uses draw i and
 * becomes fround(x * factor) when that draw is below p. */
void     q8r_apply_outliers(float* x, int64_t n, uint32_t seed, double p, double factor);

/* ---- scale derivation: src/compiler/ir/graph/quantization_types.ts ---- */
/* fromRange(min,max,PER_TENSOR_SYMMETRIC) :248-254; numBits = 8 -> bound 127 */
double   q8r_scale_sym_from_range(double mn, double mx, int num_bits);
/* fromRange asymmetric :256-263 -> scale and clamped zero point */
void     q8r_params_asym_from_range(double mn, double mx, int is_ui8, int num_bits,
                                    double* scale, double* zero_point);
/* ValueObserver.update (src/compiler/analysis/calibration.ts:24-34):
 * running min/max that never takes a NaN (comparisons with NaN are false). */
void     q8r_observe_minmax(const float* x, int64_t n, double* mn, double* mx);
/* fromConstantArray :287-297 (per tensor, symmetric) */
double   q8r_scale_const_array(const float* x, int64_t n, int num_bits);
/* fromConstantArrayPerChannel :299-317 for a 2-D [rows, cols] array.
 * axis 0: channel = row, axis 1: channel = column. scales[numCh]. */
void     q8r_scales_per_channel(const float* w, int64_t rows, int64_t cols, int axis,
                                int num_bits, double* scales);
/* fromConstantArrayPerGroup :319-340 */
void     q8r_scales_per_group(const float* x, int64_t n, int64_t group, int num_bits,
                              double* scales);
/* Dynamic per-token scale (composed, no reference counterpart as an op):
 * each row goes through ValueObserver + fromRange(SYMMETRIC).  A row with
 * no element (K == 0) has no calibration data, so the pass falls back to
 * defaultForActivation (quantization_pass.ts:381-388, quantization_types.ts:283-285)
 * = 6/127. */
void     q8r_scales_per_token(const float* x, int64_t M, int64_t K, double* scales);
double   q8r_scale_per_tensor_dynamic(const float* x, int64_t n);

/* ---- rounding primitives ---- */
double   q8r_js_round(double y);
float    q8r_fround(double v);

/* ---- R1: compiled `quantize` op, src/compiler/passes/lowering/quant_math.ts:16-27 ----
 * q = ToInt32(min(max(JSround(fround(x/s)), cMin), cMax)), cMin/cMax from the
 * hard-coded 8-bit clamp (:7-14): i8 [-128,127], ui8 [0,255].
 * zero_point != 0: JSround(fround(fround(x/s) + zp)).  Output bytes are
 * int8 (is_ui8 = 0) or uint8 (is_ui8 = 1). */
int      q8r_quantize_value(float x, double s, double zp, int is_ui8);
void     q8r_quantize(const float* x, int64_t n, double s, double zp, int is_ui8, void* q);
/* R1 with one scale per row (per-token) */
void     q8r_quantize_rows(const float* x, int64_t M, int64_t K, const double* scales, int8_t* q);

/* ---- R2: host weight quantize, quantization_types.ts:75-79, :118-130 ----
 * q = max(cMin, min(cMax, JSround(w/s + zp))), all f64, no fround.
 * clampRange :62-73: [-(2^(b-1)-1), 2^(b-1)-1] for PER_TENSOR_SYMMETRIC
 * (symmetric=1), else [-2^(b-1), 2^(b-1)-1] (i8) / [0, 2^b-1] (ui8). */
int      q8r_weight_quantize_value(double w, double s, double zp, int lo, int hi);
void     q8r_clamp_range(int symmetric, int is_ui8, int num_bits, int* lo, int* hi);
/* per-channel over a 2-D [rows, cols] weight; output in the same layout */
void     q8r_weight_quantize_per_channel(const float* w, int64_t rows, int64_t cols, int axis,
                                         const double* scales, int8_t* q);
void     q8r_weight_quantize_per_tensor(const float* w, int64_t n, double s, int lo, int hi,
                                        int8_t* q);
/* quantizeArrayPerGroup (:143-153): element i uses the scale of group
 * floor(i / group); zero points are 0 (fromConstantArrayPerGroup). */
void     q8r_weight_quantize_per_group(const float* w, int64_t n, int64_t group,
                                       const double* scales, int lo, int hi, int8_t* q);

/* ---- D1: compiled `dequantize`, quant_math.ts:29-34 ----
 * y = fround(q * s); zp != 0: y = fround(fround(q - zp) * s). */
float    q8r_dequantize_value(double q, double s, double zp);
void     q8r_dequantize_i8(const int8_t* q, int64_t n, double s, double zp, float* y);
void     q8r_dequantize_u8(const uint8_t* q, int64_t n, double s, double zp, float* y);
void     q8r_dequantize_i32(const int32_t* q, int64_t n, double s, double zp, float* y);
void     q8r_dequantize_rows_i8(const int8_t* q, int64_t M, int64_t K, const double* scales, float* y);

/* ---- M1: quantized_dot, rules/quantization.ts:57-76 + lowering_registry emitMatmulInitAcc ----
 * acc[m,n] = sum_k (A[m,k]-zpA) * (B[k,n]-zpB), exact, stored ToInt32.
 * A is [M,K] row-major int8.  b_layout 0: B is [K,N] (rhs_contracting=[0]);
 * b_layout 1: B is [N,K] (rhs_contracting=[1], the nn.Linear weight). */
void     q8r_quantized_dot(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                           int b_layout, int32_t zpA, int32_t zpB, int32_t* acc);
/* The same with either operand read as ui8 (a Uint8Array: 0..255), the
 * verifier's other operand type (ops/quantization.ts:141-146). */
void     q8r_quantized_dot_ex(const int8_t* A, int a_u8, const int8_t* B, int b_u8, int64_t M,
                              int64_t N, int64_t K, int b_layout, int32_t zpA, int32_t zpB,
                              int32_t* acc);

/* ---- quantized_conv, src/compiler/ir/graph/ops/quantization.ts:156-190,
 * lowering rules/quantization.ts:44-62 through buildConvNest
 * (src/compiler/passes/lowering/lowering_registry.ts:335-449) ----
 * Layouts NC(spatial) / OI(spatial) (input_layout "NCHW", kernel_layout
 * "OIHW" and their 1-D / 3-D forms), spatial_dims d in 1..3:
 *   x [N, C, S_0..S_{d-1}], w [O, C/groups, K_0..K_{d-1}],
 *   out [N, O, P_0..P_{d-1}],
 *   P_i = floor((S_i + lo_i + hi_i - ((K_i - 1) * dil_i + 1)) / stride_i) + 1
 *   (inferConvResultTypes, src/compiler/ir/graph/ops/linalg.ts:222-248).
 * out[n,o,p] = sum over ic, k of (x[n, g*Cg + ic, p*stride + k*dil - lo] - zpx)
 *              * (w[o, ic, k] - zpw), g = o / (O / groups), where a tap whose
 * input coordinate falls outside [0, S_i) adds 0 (the guardFill of the
 * IfThenElse, not (0 - zpx) * (w - zpw)); exact, stored ToInt32. */
void     q8r_quantized_conv(const int8_t* x, const int8_t* w, int d, const int64_t* x_shape,
                            const int64_t* w_shape, const int64_t* strides, const int64_t* pad_lo,
                            const int64_t* pad_hi, const int64_t* dilation, int64_t groups,
                            int32_t zpx, int32_t zpw, int32_t* out);
/* The same with either operand read as ui8 (buildConvNest's CastNode of a
 * Uint8Array load). */
void     q8r_quantized_conv_ex(const int8_t* x, int x_u8, const int8_t* w, int w_u8, int d,
                               const int64_t* x_shape, const int64_t* w_shape,
                               const int64_t* strides, const int64_t* pad_lo,
                               const int64_t* pad_hi, const int64_t* dilation, int64_t groups,
                               int32_t zpx, int32_t zpw, int32_t* out);

/* ---- W4A8 per-group GEMV (no reference op; composed here) ----
 * Weights: 4-bit codes of fromConstantArrayPerGroup + quantizeArrayPerGroup
 * (quantization_types.ts:319-340, :143-153) over the flat [N, K] array with
 * K % group == 0, packed two per byte (element 2j in the low nibble, two's
 * complement); sw[n * G + g], G = K / group.  Activations: int8 codes xq
 * with scales sx[m * sx_stride].
 *   acc_g = sum_{k in group g} xq[m,k] * q[n,k]          (exact int)
 *   S     = (((acc_0 * sw_0) + acc_1 * sw_1) + ...)      (f64, g ascending)
 *   y     = fround(S * sx[m]), then bias fround(y + b[n]) and act as in
 *           q8r_epilogue. */
void     q8r_gemv_w4(const int8_t* xq, const double* sx, int64_t sx_stride, const uint8_t* wq4,
                     const double* sw, int64_t M, int64_t N, int64_t K, int64_t group,
                     const float* bias, int act, float* y);

/* ---- epilogues (quantization_pass.ts:335-355 E-pt, :431-456 E-pc) ----
 * mode 0 (E-pt):      y = fround(acc * s_out)            s_out = sA*sB in f64
 * mode 1 (E-pc/rowcol): y = fround(acc * fround(sA[m] * sB[n]))
 * sA / sB may be per-row / per-col arrays or broadcast scalars (stride 0).
 * Then bias (fround(y + b[n])) and act: 0 none, 1 ReLU (Math.max(v,0)),
 * 2 SiLU (decomposition_pass.ts:197-203,224-230). */
void     q8r_epilogue(const int32_t* acc, int64_t M, int64_t N, int mode,
                      const double* sA, int64_t sA_stride, const double* sB, int64_t sB_stride,
                      double s_out, const float* bias, int act, float* y);
float    q8r_relu(float v);
float    q8r_silu(float x);
float    q8r_mul(float a, float b);
/* h = fround(silu(g) * u) elementwise */
void     q8r_silu_mul(const float* g, const float* u, int64_t n, float* h);

/* ---- calibration observers: src/compiler/analysis/calibration.ts ----
 * ValueObserver (:11-39) with an optional HistogramCollector (:41-189).
 * bins are integer counts held in doubles, exactly as the reference's
 * Float64Array. */
typedef struct {
  double min, max, count;           /* ValueObserver */
  int has_hist, num_bins, initialized;
  double range_min, range_max, total_count;
  double* bins;                      /* num_bins entries, caller-owned */
} q8r_observer;
void     q8r_observer_init(q8r_observer* o, double* bins, int num_bins, int has_hist);
void     q8r_observer_update(q8r_observer* o, const float* x, int64_t n);
double   q8r_hist_percentile(const q8r_observer* o, double percentile);
double   q8r_hist_entropy(const q8r_observer* o, int num_quant_bins);
/* CalibrationResult.getQuantParams (:246-268).  mode 0 minmax, 1 percentile,
 * 2 entropy; scheme 0 per_tensor_symmetric, 1 per_tensor_asymmetric,
 * 2 per_channel (fromRange treats every scheme but the symmetric one with the
 * zero-point formula); returns 0 when the observer saw no data (the
 * reference returns null). */
int      q8r_calib_params(const q8r_observer* o, int mode, int scheme, int is_ui8,
                          double* scale, double* zero_point);

#ifdef __cplusplus
}
#endif
#endif
