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
// Registers live in LDS, register r of lane t at R[r * NT + t]: a wave's
// 64 accesses to one register are contiguous (no bank conflicts).  When
// every offset the nest forms fits in 31 bits (NARROW, checked on the host)
// the loop indices come from 32-bit multiply-high divisions by precomputed
// magic numbers and the offsets from 32-bit multiply-adds, else from int64
// division.  The externs with long f64 code paths are out of line.
//
// Measured on [4096, 4096] (bench.py's `ewise_*` lines: a per-channel
// dequant with bias, ReLU fused with quantize, a dequantize feeding an add):
// 187 / 272 / 181 us, 6-10% of HBM -- the interpreter is instruction-bound,
// not memory-bound.  Counters on the dequant-add program (5 instructions)
// show ~145 VALU and ~170 SALU instructions per element per lane: operand
// fetch and dispatch per program instruction, not the arithmetic.  Keeping
// the registers in VGPRs instead (uniform register numbers, GPR index mode,
// 2-4 elements per lane) measured slower (294 / 342 / 306 us): each indexed
// access costs a mode switch, and the register files cut occupancy.
// 32-bit indexing and the out-of-line externs gave 5-8% over int64
// indexing with every extern inlined (201 / 286 / 195 us).  These are the
// elementwise PrimFuncs the GEMM chain fusion does not absorb; a program
// that matters for speed belongs in a fused epilogue.
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
// exp / log / tanh come from the device's f64 libm; rounded to binary32 (the
// f32-typed externs) they equal V8's Math.fround(Math.exp / log / tanh(x))
// for every binary32 x (tests/test_gpu_ewise_exhaustive.py).  pow is not
// pinned: the f64 results of two libms can differ in the last bit.
#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

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

// x / d for 0 <= x < 2^31 by a multiply-high: m = ceil(2^(31+l) / d),
// l = ceil(log2 d), q = (x * m) >> (31 + l) (the round-up method: the error
// of m is below d / 2^(31+l), too small to change floor(x / d) for
// x < 2^31).  d = 1: m = 0, q = x.
struct EwDiv {
  uint32_t m[Q8_EW_MAX_DIMS];
  uint32_t sh[Q8_EW_MAX_DIMS];   // l - 1 (the multiply-high already shifts by 32)
};

__device__ __forceinline__ uint32_t ew_udiv(uint32_t x, uint32_t m, uint32_t sh) {
  return m == 0 ? x : (__umulhi(x, m) >> sh);
}

// The externs with long f64 code paths, out of line: inlined once per
// register file they would multiply the kernel's code and registers for
// instructions most programs never run.
__device__ __noinline__ double ew_slow(int op, double a, double b) {
  switch (op) {
    case Q8_EW_MOD: return js_rem(js_rem(a, b) + b, b);
    case Q8_EW_TMOD: return js_rem(a, b);
    case Q8_EW_FMOD: return js_rem(js_rem(a, b) + b, b);
    case Q8_EW_EXP: return exp(a);
    case Q8_EW_LOG: return log(a);
    case Q8_EW_TANH: return tanh(a);
    case Q8_EW_RSQRT: return 1.0 / sqrt(a);
    default: return pow(a, b);
  }
}

template <bool NARROW>
__global__ __launch_bounds__(EW_NT) void k_ewise(q8_ew_prog p, EwPtrs ptr, EwDiv dv, int64_t n) {
  using I = typename std::conditional<NARROW, uint32_t, int64_t>::type;
  __shared__ double R[Q8_EW_MAX_REGS * EW_NT];
  const int t = threadIdx.x;
  auto reg = [&](int r) -> double& { return R[r * EW_NT + t]; };
  const int nd = p.ndims;
  for (int64_t e = blockIdx.x * (int64_t)EW_NT + t; e < n; e += (int64_t)gridDim.x * EW_NT) {
    // loop indices of element e (row-major, last fastest)
    I idx[Q8_EW_MAX_DIMS];
    I rem = (I)e;
#pragma unroll
    for (int d = Q8_EW_MAX_DIMS - 1; d >= 0; --d) {
      if (d < nd) {
        I q;
        if constexpr (NARROW) q = ew_udiv(rem, dv.m[d], dv.sh[d]);
        else q = rem / p.extent[d];
        idx[d] = rem - q * (I)p.extent[d];
        rem = q;
      } else {
        idx[d] = 0;
      }
    }
    for (int pc = 0; pc < p.ncode; ++pc) {
      const q8_ew_instr in = p.code[pc];
      double v = 0.0;
      if (in.op == Q8_EW_LOAD) {
        const int j = in.aux;
        I off = (I)p.in_coef[j][Q8_EW_MAX_DIMS];
#pragma unroll
        for (int d = 0; d < Q8_EW_MAX_DIMS; ++d)
          if (d < nd) off += (I)p.in_coef[j][d] * idx[d];
        v = load_elem(ptr.in[j], p.in_dtype[j], (int64_t)off);
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
          case Q8_EW_MOD: v = ew_slow(Q8_EW_MOD, a, b); break;
          case Q8_EW_FLOORDIV: v = floor(a / b); break;
          case Q8_EW_TMOD: v = ew_slow(Q8_EW_TMOD, a, b); break;
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
          case Q8_EW_FMOD: v = ew_slow(Q8_EW_FMOD, a, b); break;
          case Q8_EW_EXP: v = ew_slow(Q8_EW_EXP, a, b); break;
          case Q8_EW_LOG: v = ew_slow(Q8_EW_LOG, a, b); break;
          case Q8_EW_TANH: v = ew_slow(Q8_EW_TANH, a, b); break;
          case Q8_EW_RSQRT: v = ew_slow(Q8_EW_RSQRT, a, b); break;
          case Q8_EW_POW: v = ew_slow(Q8_EW_POW, a, b); break;
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
  // 31-bit offsets: every extent, coefficient, offset and n
  bool narrow = n < ((int64_t)1 << 31);
  for (int d = 0; d < p.ndims; ++d) narrow = narrow && p.extent[d] < ((int64_t)1 << 31);
  for (int j = 0; j < p.ninputs; ++j) {
    int64_t hi = p.in_coef[j][Q8_EW_MAX_DIMS];
    narrow = narrow && hi >= 0 && hi < ((int64_t)1 << 31);
    for (int d = 0; d < p.ndims; ++d) {
      const int64_t c = p.in_coef[j][d];
      narrow = narrow && c > -((int64_t)1 << 31) && c < ((int64_t)1 << 31);
      if (c > 0) hi += c * (p.extent[d] - 1);   // ewise_check bounds it by in_numel
    }
    narrow = narrow && hi < ((int64_t)1 << 31);
  }
  EwDiv dv{};
  for (int d = 0; d < p.ndims; ++d) {
    const uint64_t x = (uint64_t)p.extent[d];
    if (!narrow || x <= 1) continue;     // extent 1 (or 0: no elements): q = x
    int l = 0;
    while (((uint64_t)1 << l) < x) ++l;
    dv.m[d] = (uint32_t)((((uint64_t)1 << (31 + l)) + x - 1) / x);
    dv.sh[d] = (uint32_t)(l - 1);
  }
  const int64_t blocks = (n + EW_NT - 1) / EW_NT;
  const int grid = (int)(blocks < 16384 ? blocks : 16384);
  if (narrow) hipLaunchKernelGGL((k_ewise<true>), dim3(grid), dim3(EW_NT), 0, st, p, ptr, dv, n);
  else hipLaunchKernelGGL((k_ewise<false>), dim3(grid), dim3(EW_NT), 0, st, p, ptr, dv, n);
  return hipGetLastError();
}

}  // namespace q8
