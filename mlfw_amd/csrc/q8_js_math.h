// q8_js_math.h -- the JS number semantics of the reference CPU backend's
// generated code (src/backend/cpu/codegen.ts:428-552) that q8_ewise needs,
// as device functions.  Included twice by q8_ewise.hip: once as code (the
// interpreter), once through Q8_JS_MATH_BODY's stringification as the
// source text that every run-time compiled elementwise kernel starts with,
// so both evaluate the same functions.  No preprocessor lines, include
// guards or comments inside the macro argument (stringification keeps the
// code only).
Q8_JS_MATH_BODY(
__device__ __forceinline__ int js_to_int32(double x) {
  if (!(x == x) || __builtin_isinf(x)) return 0;
  double t = trunc(x);
  if (t >= -2147483648.0 && t <= 2147483647.0) return (int)t;
  double m = fmod(t, 4294967296.0);
  if (m < 0.0) m += 4294967296.0;
  return (int)(unsigned int)m;
}
__device__ __forceinline__ double js_round_full(double y) {
  if (!(y == y) || __builtin_isinf(y)) return y;
  const double f = floor(y);
  double r = (y - f >= 0.5) ? f + 1.0 : f;
  if (r == 0.0 && (y < 0.0 || __builtin_signbit(y))) r = -0.0;
  return r;
}
__device__ __forceinline__ double js_max(double a, double b) {
  if (!(a == a) || !(b == b)) return __builtin_nan("");
  if (a == b) return __builtin_signbit(a) ? b : a;
  return a > b ? a : b;
}
__device__ __forceinline__ double js_min(double a, double b) {
  if (!(a == a) || !(b == b)) return __builtin_nan("");
  if (a == b) return __builtin_signbit(a) ? a : b;
  return a < b ? a : b;
}
__device__ __forceinline__ double js_rem(double a, double b) { return fmod(a, b); }
__device__ __forceinline__ double js_sign(double x) {
  if (!(x == x) || x == 0.0) return x;
  return x > 0.0 ? 1.0 : -1.0;
}
__device__ __forceinline__ bool truthy(double x) { return x == x && x != 0.0; }
)
