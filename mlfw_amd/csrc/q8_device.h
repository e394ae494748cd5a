// q8_device.h -- device-side arithmetic shared by the gfx950 kernels.
//
// All helpers reproduce the reference CPU backend's JavaScript arithmetic
// (src/backend/cpu/codegen.ts): f64 evaluation, Math.fround = one RNE
// conversion to binary32, Math.round = nearest integer with ties toward +inf,
// `| 0` = NaN -> 0.  The library is compiled with -ffp-contract=off and no
// fast-math so that every f64 / f32 operation below is a single IEEE op.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace q8 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// ECMA-262 Math.round for an exact double.  y - floor(y) is exact.
__device__ __forceinline__ double js_round(double y) {
  double r = floor(y);
  return (y - r >= 0.5) ? r + 1.0 : r;
}

// (Math.min(Math.max(r, lo), hi) | 0) for an already-rounded r.
__device__ __forceinline__ int clamp_to_int(double r, int lo, int hi) {
  if (r != r) return 0;
  r = r < (double)lo ? (double)lo : r;
  r = r > (double)hi ? (double)hi : r;
  return (int)r;
}

// R1, exact form: quant_math.ts:16-27 evaluated as the CPU backend does.
__device__ __forceinline__ int quant_exact(float x, double s, double zp, int lo, int hi) {
  double y = (double)(float)((double)x / s);          // Math.fround(x / s)
  if (zp != 0.0) y = (double)(float)(y + zp);          // Math.fround(.. + zp)
  return clamp_to_int(js_round(y), lo, hi);
}

// R1 for the symmetric int8 case (zp = 0, clamp [-128,127]) with an f32
// fast path.  r32 = (float)(1/s).  t = x*r32 differs from y = x/s by at most
// 2^-22.9 relative, i.e. < 2^-15 for |y| < 256, and fround(y) differs from y
// by at most 2^-17 there; Math.round only changes value across a
// half-integer, so when t's fraction is more than 2^-13 away from 0.5 the
// integer is decided by t.  |t| >= 256 implies |y| > 128.5 (clamped).
// Callers guarantee s is a normal double in [2^-100, 2^100] (else they use
// quant_exact for every element).
// quant_sym_try is that decision without branches: floor(t) clamped to
// [-256, 256] (so |t| >= 256 saturates through the integer clamp), plus the
// rounding step; `bad` flags the inputs the fast path may not decide, which
// take the exact f64 path: every t whose fraction is within 2^-13 of 0.5,
// and NaN and infinite t (their fraction t - floor(t) is NaN).  Near-ties
// with |t| >= 256 are flagged too although the clamp decides them; the exact
// path gives the same code, and a single comparison is cheaper than
// excluding them (this test runs once per quantized value).
__device__ __forceinline__ int quant_sym_try(float x, float r32, bool& bad) {
  const float t = x * r32;
  const float fl = __builtin_floorf(t);
  const float fr = t - fl;
  int r = (int)__builtin_amdgcn_fmed3f(fl, -256.0f, 256.0f) + (fr > 0.5f ? 1 : 0);
  r = r < -128 ? -128 : (r > 127 ? 127 : r);
  bad = !(__builtin_fabsf(fr - 0.5f) > 0x1p-13f);
  return r;
}

__device__ __forceinline__ int quant_sym_fast(float x, float r32, double s) {
  bool bad;
  int r = quant_sym_try(x, r32, bad);
  if (bad) r = quant_exact(x, s, 0.0, -128, 127);
  return r;
}

// Order key of |x| for a NaN-ignoring absmax: the bit pattern of |x| (an
// integer order equal to the float order for non-negative floats), -1 for NaN.
__device__ __forceinline__ int absmax_key(float x) {
  unsigned u = __float_as_uint(x) & 0x7fffffffu;
  return u > 0x7f800000u ? -1 : (int)u;
}

// Scale from a reduced absmax key (fromRange symmetric, quantization_types.ts:
// 249-253): s = absmax/127 || 1e-10.  key -1 = only NaNs were seen: the
// observer's min/max stayed (+inf, -inf), so absmax = +inf.
__device__ __forceinline__ double scale_from_key(int key) {
  double amax = key < 0 ? __builtin_inf() : (double)__uint_as_float((unsigned)key);
  double s = amax / 127.0;
  return (s == 0.0 || s != s) ? 1e-10 : s;
}

// Four int8 codes packed little-endian into one dword.
__device__ __forceinline__ int pack4(int b0, int b1, int b2, int b3) {
  return (b0 & 0xff) | ((b1 & 0xff) << 8) | ((b2 & 0xff) << 16) | ((b3 & 0xff) << 24);
}

// absmax_key of four values.
__device__ __forceinline__ int key4(float4 v) {
  int a = absmax_key(v.x), b = absmax_key(v.y), c = absmax_key(v.z), d = absmax_key(v.w);
  a = a > b ? a : b;
  c = c > d ? c : d;
  return a > c ? a : c;
}

// Symmetric int8 codes of four values (R1 with zp = 0), packed; one branch
// to the exact path for the four.
__device__ __forceinline__ int quant4_sym(float4 v, bool fast, float r32, double s) {
  if (fast) {
    bool b0, b1, b2, b3;
    int c0 = quant_sym_try(v.x, r32, b0), c1 = quant_sym_try(v.y, r32, b1);
    int c2 = quant_sym_try(v.z, r32, b2), c3 = quant_sym_try(v.w, r32, b3);
    if (b0 | b1 | b2 | b3) {
      if (b0) c0 = quant_exact(v.x, s, 0.0, -128, 127);
      if (b1) c1 = quant_exact(v.y, s, 0.0, -128, 127);
      if (b2) c2 = quant_exact(v.z, s, 0.0, -128, 127);
      if (b3) c3 = quant_exact(v.w, s, 0.0, -128, 127);
    }
    return pack4(c0, c1, c2, c3);
  }
  return pack4(quant_exact(v.x, s, 0.0, -128, 127), quant_exact(v.y, s, 0.0, -128, 127),
               quant_exact(v.z, s, 0.0, -128, 127), quant_exact(v.w, s, 0.0, -128, 127));
}

// Whether the f32 fast path of quant_sym_fast is valid for scale s.
__device__ __forceinline__ bool fast_scale_ok(double s) {
  return s >= 0x1p-100 && s <= 0x1p100;
}

// D1: Math.fround((+q) * s), zero point form Math.fround(Math.fround(q - zp) * s).
__device__ __forceinline__ float dequant(double q, double s, double zp) {
  if (zp != 0.0) q = (double)(float)(q - zp);
  return (float)(q * s);
}

// Math.max(v, 0) on f32: NaN stays NaN, -0 and negatives give +0.
__device__ __forceinline__ float relu_js(float v) {
  return (v > 0.0f || v != v) ? v : 0.0f;
}

// SiLU decomposed (decomposition_pass.ts:197-203, 224-230), each op rounded:
// fround(x * fround(1 / fround(1 + fround(exp(-x))))), exp evaluated in f64.
// The add, divide and multiply are binary32 operations: for +, / and * of
// binary32 operands, rounding the binary64 result to binary32 gives the
// correctly rounded binary32 result (53 >= 2 * 24 + 2), which is what the
// IEEE binary32 instructions compute (no fast-math: the division is the
// correctly rounded sequence).
__device__ __forceinline__ float silu_js(float x) {
  const float e = (float)exp(-(double)x);
  const float d = 1.0f + e;
  const float r = 1.0f / d;
  return x * r;
}

// Wave64 reductions.
__device__ __forceinline__ int wave_max_i32(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    int w = __shfl_xor(v, o, 64);
    v = v > w ? v : w;
  }
  return v;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Key of a float for an order-preserving signed-int min/max (NaN excluded by
// the caller): non-negative floats keep their bits, negative ones flip the
// magnitude bits so that more negative is smaller.
__device__ __forceinline__ int order_key(float x) {
  int b = __float_as_int(x);
  return b >= 0 ? b : (int)(b ^ 0x7fffffff);
}
__device__ __forceinline__ float from_order_key(int k) {
  return __int_as_float(k >= 0 ? k : (int)(k ^ 0x7fffffff));
}

}  // namespace q8
