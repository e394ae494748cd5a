// q8_js_math.h -- the JS number semantics of the reference CPU backend's
// generated code (src/backend/cpu/codegen.ts:428-552) that q8_ewise needs,
// as device functions.  Included twice by q8_ewise.hip: once as code (the
// interpreter), once through Q8_JS_MATH_BODY's stringification as the
// source text that every run-time compiled elementwise kernel starts with,
// so both evaluate the same functions.  No preprocessor lines, include
// guards or comments inside the macro argument (stringification keeps the
// code only).
//
// The f32 forms (js_maxf ... js_to_int32f) are the same functions on values
// that are exactly binary32 (the compiled kernels hold such values as float):
// max, min, floor, round, sign and truncation of a binary32 value are
// binary32 values, and every step of them is exact in binary32 (y - floor(y)
// is exact, floor(y) + 1 is exact below 2^24, and from 2^23 on y is an
// integer), so they give the bits of the f64 forms.  They are written as
// selects, without early returns: a kernel's lanes see mixed values (zeros
// next to positive values after a ReLU), and every branch the lanes of a
// wave take apart is executed for the whole wave.  For equal operands
// js_maxf takes the AND of their bits and js_minf the OR: equal nonzero
// values have equal bits, and of +0 and -0 the AND is +0 (Math.max) and the
// OR -0 (Math.min).  js_roundf needs no NaN
// or infinity test: floor keeps them, y - floor(y) is then NaN and fails
// the comparison, so r = floor(y) = y.
//
// js_fround_div_const(a, c, rc) = Math.fround(a / c) for a constant c with
// rc = 1 / c rounded to nearest (c finite, 2^-1000 <= |c| <= 2^1000).
// q = a * rc differs from a / c by less than 2 * 2^-52 relative (two
// roundings of 2^-53 each), so q and the f64 quotient RN(a / c) are at most
// 2 units in the last place apart.  fround of two f64 values gives the same
// binary32 value unless a binary32 rounding midpoint lies between or on them;
// in the binary32 normal range a midpoint is an f64 whose low 29 fraction
// bits are 2^28.  So when q's low 29 bits are more than 4 from 2^28 and q
// lies in [2^-125, 2^127), fround(q) is the answer; q = 0 (a = 0, or a * rc
// below the f64 range, where a / c rounds to a binary32 zero of the same
// sign) is too.  Every other case divides.
//
// js_fround_div_const_f(a, |c|, rc, c < 0) is the same for a binary32 a,
// without the division near a midpoint (which is common when the quotient
// has few significant bits: x / 0.05 = x * 20 is a midpoint for about one
// binary32 x in 8).  It works on A = |a| (the sign is applied at the end;
// fround is odd).  When q = A * rc lies within 4 units of the midpoint m
// (low 29 bits of m = 2^28), RN(A / c) is within 6 units of m, so only its
// place against m decides: above m rounds up, below m rounds down, equal to
// m is the binary32 tie (to even).  RN(A / c) equals m exactly when
// |A / c - m| <= h = ulp(m) / 2 (m's last bit is 0, so f64 ties go to m),
// i.e. when |E| <= T with E = A - m * c and T = c * h.  E is exact: A is
// binary32 and m has 25 significant bits, so A and m * c are multiples of
// 2^(e_m + e_c - 76), and |E| <= 6 c ulp(m) < 2^(e_m + e_c - 48); with
// 2^-800 <= c <= 2^800 (the caller's range) and q in the binary32 normal
// range neither E nor T leaves the f64 normal range.  So one fma, one ldexp
// and two comparisons replace the division; outside [2^-125, 2^127) the
// division remains.  In both functions the empty asm statement on the
// dividend keeps the division inside its branch: without it the compiler
// evaluates the division for every element and selects the result.
//
// js_quant_i8(a, r32, c) is ToInt32(Math.min(Math.max(Math.round(
// Math.fround(a / c)), -128), 127)) for a binary32 a and a constant c in
// [2^-100, 2^100], r32 = (float)(1 / c): the symmetric int8 quantize
// (quant_math.ts:16-27) as QuantizationPass's expression writes it, NaN
// giving 0.  It is the library's int8 quantize fast path: t = a * r32 in
// binary32 is within 2^-15 of the quotient for every |quotient| < 256, and
// the fround within 2^-17, so Math.round can differ from the one of t only
// when t's fraction lies within 2^-13 of 1/2; those inputs (and NaN and
// infinite t, whose fraction is NaN) take js_quant_i8_exact, the
// expression's own steps in f64.  |t| >= 256 clamps: floor(t) saturates at
// +-256 before the integer clamp.
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
__device__ __forceinline__ float js_maxf(float a, float b) {
  const float e = __int_as_float(__float_as_int(a) & __float_as_int(b));
  const float r = a > b ? a : (a == b ? e : b);
  return (a == a && b == b) ? r : __builtin_nanf("");
}
__device__ __forceinline__ float js_minf(float a, float b) {
  const float e = __int_as_float(__float_as_int(a) | __float_as_int(b));
  const float r = a < b ? a : (a == b ? e : b);
  return (a == a && b == b) ? r : __builtin_nanf("");
}
__device__ __forceinline__ float js_roundf(float y) {
  const float f = __builtin_floorf(y);
  const float r = (y - f >= 0.5f) ? f + 1.0f : f;
  return r == 0.0f ? __builtin_copysignf(0.0f, y) : r;
}
__device__ __forceinline__ float js_signf(float x) {
  return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : x);
}
__device__ __forceinline__ bool truthyf(float x) { return x == x && x != 0.0f; }
__device__ __forceinline__ int js_to_int32f(float x) {
  if (x >= -2147483648.0f && x < 2147483648.0f) return (int)__builtin_truncf(x);
  return js_to_int32((double)x);
}
__device__ __forceinline__ float js_fround_div_const(double a, double c, double rc) {
  const double q = a * rc;
  const unsigned long long b = (unsigned long long)__double_as_longlong(q);
  const unsigned lo = (unsigned)b & 0x1FFFFFFFu;
  const unsigned ex = (unsigned)(b >> 52) & 0x7FFu;
  float r = (float)q;
  if (q != 0.0 && (lo - 0x0FFFFFFCu <= 8u || ex - 898u > 251u)) {
    double d = a;
    __asm__ volatile("" : "+v"(d));
    r = (float)(d / c);
  }
  return r;
}
__device__ __forceinline__ float js_fround_div_const_f(float a, double c, double rc, bool neg) {
  const double A = __builtin_fabs((double)a);
  const double q = A * rc;
  const long long b = __double_as_longlong(q);
  const unsigned lo = (unsigned)b & 0x1FFFFFFFu;
  const unsigned ex = (unsigned)(b >> 52);
  const long long mb = (b & ~0x1FFFFFFFLL) | 0x10000000LL;
  const double E = __builtin_fma(-__longlong_as_double(mb), c, A);
  const double T = __builtin_ldexp(c, (int)ex - 1076);
  const long long pick = mb + (long long)(E > T) - (long long)(E < -T);
  float r = (float)(lo - 0x0FFFFFFCu <= 8u ? __longlong_as_double(pick) : q);
  if (ex - 898u > 251u && q != 0.0) {
    double d = A;
    __asm__ volatile("" : "+v"(d));
    r = (float)(d / c);
  }
  return __builtin_signbit(a) != neg ? -r : r;
}
__device__ __noinline__ int js_quant_i8_exact(float a, double c) {
  const double r = js_round_full((double)(float)((double)a / c));
  return js_to_int32(js_min(js_max(r, -128.0), 127.0));
}
__device__ __forceinline__ int js_quant_i8(float a, float r32, double c) {
  const float t = a * r32;
  const float fl = __builtin_floorf(t);
  const float fr = t - fl;
  int r = (int)__builtin_amdgcn_fmed3f(fl, -256.0f, 256.0f) + (fr > 0.5f ? 1 : 0);
  r = r < -128 ? -128 : (r > 127 ? 127 : r);
  return __builtin_fabsf(fr - 0.5f) > 0x1p-13f ? r : js_quant_i8_exact(a, c);
}
)
