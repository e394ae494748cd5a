// q8_ewise.hip -- elementwise loop nests on the device with the reference CPU
// backend's arithmetic (src/backend/cpu/codegen.ts:428-552).
//
// The program (q8_ew_prog, include/q8hip.h) is straight-line code over
// Q8_EW_MAX_REGS f64 registers, passed by value in the kernel arguments, so a
// launch needs no device memory of its own.  Every lane evaluates one
// element of the loop nest at a time: it decodes the loop indices from the
// element's row-major position, runs the program, and stores the result
// register.  All lanes execute the same instruction stream (the opcode and
// register numbers come from the kernel arguments and stay in SGPRs), so the
// interpreter never diverges.
//
// Registers live in LDS, register r of lane t at R[r * NT + t]: a
// run-time register index into a private array would otherwise go to
// scratch memory, and this layout keeps a wave's 64 accesses to one
// register contiguous (no bank conflicts).
//
// Value semantics (all f64, like JS numbers):
//   * f32-typed arithmetic and non-exact externs round once to binary32
//     (Math.fround) when the instruction's `rnd` flag is set;
//   * exact externs (max, min, abs, floor, ceil, round, sign, sqrt, fmod)
//     are never rounded;
//   * comparisons give 1 / 0, a select takes its condition as JS truthiness;
//   * `| 0` is ECMA-262 ToInt32; typed-array stores convert as
//     Float32Array (RNE), Float64Array, Int32Array (ToInt32), Int8Array and
//     Uint8Array (low 8 bits of ToInt32).
// exp / log / tanh / pow come from the device's f64 libm, not V8's: their
// results can differ from the reference in the last bit of the f64, which
// one binary32 rounding almost always absorbs (the same unpinned boundary as
// SiLU's exp).
#include <hip/hip_runtime.h>

#include <cmath>

#include "../../include/q8hip.h"
#include "q8_internal.h"

namespace q8 {

namespace {

constexpr int EW_NT = 256;

struct EwPtrs {
  const void* in[Q8_EW_MAX_INPUTS];
  void* out;
};

// ECMA-262 ToInt32: NaN and infinities -> 0, otherwise trunc(x) mod 2^32.
__device__ __forceinline__ int32_t js_to_int32(double x) {
  if (!(x == x) || __builtin_isinf(x)) return 0;
  double t = trunc(x);
  if (t >= -2147483648.0 && t <= 2147483647.0) return (int32_t)t;
  double m = fmod(t, 4294967296.0);       // exact
  if (m < 0.0) m += 4294967296.0;          // exact: |m| < 2^32
  return (int32_t)(uint32_t)m;
}

// Math.round: nearest integer, ties toward +inf, -0 for y in [-0.5, -0].
__device__ __forceinline__ double js_round_full(double y) {
  if (!(y == y) || __builtin_isinf(y)) return y;
  const double f = floor(y);
  double r = (y - f >= 0.5) ? f + 1.0 : f;   // y - f is exact
  if (r == 0.0 && (y < 0.0 || __builtin_signbit(y))) r = -0.0;
  return r;
}

// Math.max / Math.min: NaN wins; +0 is larger than -0.
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

// JS `%` on numbers: the sign of the dividend, exact (C fmod).
__device__ __forceinline__ double js_rem(double a, double b) { return fmod(a, b); }

__device__ __forceinline__ double js_sign(double x) {
  if (!(x == x) || x == 0.0) return x;     // NaN, +0, -0
  return x > 0.0 ? 1.0 : -1.0;
}

__device__ __forceinline__ bool truthy(double x) { return x == x && x != 0.0; }

__device__ __forceinline__ double load_elem(const void* p, int dtype, int64_t off) {
  switch (dtype) {
    case Q8_I8: return (double)static_cast<const int8_t*>(p)[off];
    case Q8_U8: return (double)static_cast<const uint8_t*>(p)[off];
    case Q8_I32: return (double)static_cast<const int32_t*>(p)[off];
    case Q8_F32: return (double)static_cast<const float*>(p)[off];
    default: return static_cast<const double*>(p)[off];
  }
}

__device__ __forceinline__ void store_elem(void* p, int dtype, int64_t off, double v) {
  switch (dtype) {
    case Q8_F32: static_cast<float*>(p)[off] = (float)v; break;
    case Q8_F64: static_cast<double*>(p)[off] = v; break;
    case Q8_I32: static_cast<int32_t*>(p)[off] = js_to_int32(v); break;
    case Q8_I8: static_cast<int8_t*>(p)[off] = (int8_t)(uint8_t)(uint32_t)js_to_int32(v); break;
    default: static_cast<uint8_t*>(p)[off] = (uint8_t)(uint32_t)js_to_int32(v); break;
  }
}

__global__ __launch_bounds__(EW_NT) void k_ewise(q8_ew_prog p, EwPtrs ptr, int64_t n) {
  __shared__ double R[Q8_EW_MAX_REGS * EW_NT];
  const int t = threadIdx.x;
  auto reg = [&](int r) -> double& { return R[r * EW_NT + t]; };
  const int nd = p.ndims;
  for (int64_t e = blockIdx.x * (int64_t)EW_NT + t; e < n; e += (int64_t)gridDim.x * EW_NT) {
    // loop indices of element e (row-major, last fastest)
    int64_t idx[Q8_EW_MAX_DIMS];
    int64_t rem = e;
#pragma unroll
    for (int d = Q8_EW_MAX_DIMS - 1; d >= 0; --d) {
      if (d < nd) {
        const int64_t ext = p.extent[d];
        idx[d] = rem % ext;
        rem /= ext;
      } else {
        idx[d] = 0;
      }
    }
    for (int pc = 0; pc < p.ncode; ++pc) {
      const q8_ew_instr in = p.code[pc];
      double v = 0.0;
      if (in.op == Q8_EW_LOAD) {
        const int j = in.aux;
        int64_t off = p.in_coef[j][Q8_EW_MAX_DIMS];
#pragma unroll
        for (int d = 0; d < Q8_EW_MAX_DIMS; ++d) off += p.in_coef[j][d] * idx[d];
        v = load_elem(ptr.in[j], p.in_dtype[j], off);
      } else if (in.op == Q8_EW_CONST) {
        v = p.konst[in.aux];
      } else if (in.op == Q8_EW_INDEX) {
        v = (double)idx[in.aux < Q8_EW_MAX_DIMS ? in.aux : 0];
      } else {
        const double a = reg(in.a), b = reg(in.b);
        switch (in.op) {
          case Q8_EW_ADD: v = a + b; break;
          case Q8_EW_SUB: v = a - b; break;
          case Q8_EW_MUL: v = a * b; break;
          case Q8_EW_DIV: v = a / b; break;
          case Q8_EW_IDIV: v = trunc(a / b); break;
          case Q8_EW_MOD: v = js_rem(js_rem(a, b) + b, b); break;
          case Q8_EW_FLOORDIV: v = floor(a / b); break;
          case Q8_EW_TMOD: v = js_rem(a, b); break;
          case Q8_EW_TDIV: v = (double)js_to_int32(a / b); break;
          case Q8_EW_NEG: v = -a; break;
          case Q8_EW_CMP:
            switch (in.aux) {
              case 0: v = a == b; break;
              case 1: v = !(a == b); break;
              case 2: v = a < b; break;
              case 3: v = a <= b; break;
              case 4: v = a > b; break;
              default: v = a >= b; break;
            }
            break;
          case Q8_EW_SELECT: v = truthy(a) ? b : reg(in.c); break;
          case Q8_EW_TOINT32: v = (double)js_to_int32(a); break;
          case Q8_EW_TOBOOL: v = truthy(a) ? 1.0 : 0.0; break;
          case Q8_EW_MAX: v = js_max(a, b); break;
          case Q8_EW_MIN: v = js_min(a, b); break;
          case Q8_EW_ABS: v = fabs(a); break;
          case Q8_EW_FLOOR: v = floor(a); break;
          case Q8_EW_CEIL: v = ceil(a); break;
          case Q8_EW_ROUND: v = js_round_full(a); break;
          case Q8_EW_SIGN: v = js_sign(a); break;
          case Q8_EW_SQRT: v = sqrt(a); break;
          case Q8_EW_FMOD: v = js_rem(js_rem(a, b) + b, b); break;
          case Q8_EW_EXP: v = exp(a); break;
          case Q8_EW_LOG: v = log(a); break;
          case Q8_EW_TANH: v = tanh(a); break;
          case Q8_EW_RSQRT: v = 1.0 / sqrt(a); break;
          case Q8_EW_POW: v = pow(a, b); break;
          default: v = a; break;
        }
      }
      if (in.rnd) v = (double)(float)v;
      reg(in.dst) = v;
    }
    store_elem(ptr.out, p.out_dtype, e, reg(p.result));
  }
}

bool dtype_ok(int d) { return d == Q8_I8 || d == Q8_U8 || d == Q8_I32 || d == Q8_F32 || d == Q8_F64; }

}  // namespace

// Host-side checks of a program against its buffers; returns nullptr or a
// message.  Proves every load offset lies inside its input.
const char* ewise_check(const q8_ew_prog& p, const int64_t* in_numel, int64_t out_numel) {
  if (p.ndims < 0 || p.ndims > Q8_EW_MAX_DIMS) return "ndims out of range";
  if (p.ninputs < 0 || p.ninputs > Q8_EW_MAX_INPUTS) return "ninputs out of range";
  if (p.ncode < 1 || p.ncode > Q8_EW_MAX_CODE) return "ncode out of range";
  if (p.nconst < 0 || p.nconst > Q8_EW_MAX_CONST) return "nconst out of range";
  if (p.result < 0 || p.result >= Q8_EW_MAX_REGS) return "result register out of range";
  if (!dtype_ok(p.out_dtype)) return "bad output dtype";
  int64_t total = 1;
  for (int d = 0; d < p.ndims; ++d) {
    if (p.extent[d] < 0) return "negative extent";
    if (p.extent[d] > 0 && total > INT64_MAX / p.extent[d]) return "loop nest too large";
    total *= p.extent[d];
  }
  if (total != out_numel) return "out_numel differs from the product of the extents";
  for (int j = 0; j < p.ninputs; ++j) {
    if (!dtype_ok(p.in_dtype[j])) return "bad input dtype";
    if (total == 0) continue;
    // range of the affine offset over the box [0, extent)
    __int128 lo = p.in_coef[j][Q8_EW_MAX_DIMS], hi = lo;
    for (int d = 0; d < Q8_EW_MAX_DIMS; ++d) {
      if (d >= p.ndims) {
        if (p.in_coef[j][d] != 0) return "coefficient of an absent loop";
        continue;
      }
      const __int128 span = (__int128)p.in_coef[j][d] * (p.extent[d] - 1);
      if (span < 0) lo += span; else hi += span;
    }
    if (lo < 0 || hi >= in_numel[j]) return "an input offset falls outside its buffer";
  }
  bool loaded[Q8_EW_MAX_INPUTS] = {};
  for (int i = 0; i < p.ncode; ++i) {
    const q8_ew_instr& in = p.code[i];
    if (in.op >= Q8_EW_NOPS) return "unknown opcode";
    if (in.dst >= Q8_EW_MAX_REGS || in.a >= Q8_EW_MAX_REGS || in.b >= Q8_EW_MAX_REGS ||
        in.c >= Q8_EW_MAX_REGS)
      return "register out of range";
    if (in.op == Q8_EW_LOAD) {
      if (in.aux >= p.ninputs) return "load of an absent input";
      loaded[in.aux] = true;
    }
    if (in.op == Q8_EW_CONST && in.aux >= p.nconst) return "constant out of range";
    if (in.op == Q8_EW_INDEX && in.aux >= p.ndims) return "index of an absent loop";
    if (in.op == Q8_EW_CMP && in.aux > 5) return "bad comparison";
  }
  (void)loaded;
  return nullptr;
}

hipError_t launch_ewise(const q8_ew_prog& p, const void* const* inputs, void* out, int64_t n,
                        hipStream_t st) {
  if (n == 0) return hipSuccess;
  EwPtrs ptr{};
  for (int j = 0; j < p.ninputs; ++j) ptr.in[j] = inputs[j];
  ptr.out = out;
  const int64_t blocks = (n + EW_NT - 1) / EW_NT;
  const int grid = (int)(blocks < 16384 ? blocks : 16384);
  hipLaunchKernelGGL(k_ewise, dim3(grid), dim3(EW_NT), 0, st, p, ptr, n);
  return hipGetLastError();
}

}  // namespace q8
