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
// The interpreter is instruction-bound, not memory-bound: counters on a
// 5-instruction program show ~145 VALU and ~170 SALU instructions per
// element per lane, operand fetch and dispatch per program instruction, not
// the arithmetic; on bench.py's [4096, 4096] programs (a per-channel
// dequant with bias, ReLU fused with quantize, a dequantize feeding an add)
// it takes 187 / 272 / 182 us, 6-10% of HBM.  Keeping its registers in
// VGPRs instead (uniform register numbers, GPR index mode, 2-4 elements per
// lane) measured slower (294 / 342 / 306 us).  So a call over 2^20 elements
// or more runs the program compiled instead (hiprtc, once per program and
// device, below): 21 / 17.5 / 27 us on the same programs, the first at 78%
// of HBM and the last at 69% (their 64 MiB outputs stored non-temporally),
// the quantize at 60% (the same bytes stream in 16 us).  The compiled form
// runs a symmetric int8 quantize chain as the library's quantize fast path
// (js_quant_i8): with the division, round and clamps as separate steps the
// ReLU + quantize program took 23 us.
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
#include <hip/hiprtc.h>

#include <atomic>
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <mutex>
#include <string>
#include <type_traits>
#include <unordered_map>
#include <vector>

#include "../../include/q8hip.h"
#include "q8_internal.h"

namespace q8 {

namespace {

constexpr int EW_NT = 256;

struct EwPtrs {
  const void* in[Q8_EW_MAX_INPUTS];
  void* out;
};

// The JS helpers (q8_js_math.h): ECMA-262 ToInt32 (NaN and infinities ->
// 0, else trunc(x) mod 2^32); Math.round (nearest, ties toward +inf, -0 for
// y in [-0.5, -0]); Math.max / Math.min (NaN wins, +0 above -0); JS `%`
// (C fmod: the sign of the dividend, exact); Math.sign; JS truthiness.
#define Q8_JS_MATH_BODY(...) __VA_ARGS__
#include "q8_js_math.h"
#undef Q8_JS_MATH_BODY

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

// ---------------------------------------------------------------- compiled programs
// A program run over many elements is compiled instead: its HIP source (the
// loop nest with its extents, offsets and dtypes as constants, one statement
// per instruction over the same JS helpers, q8_js_math.h) goes through
// hiprtc once per program and device, and later calls launch the cached
// kernel.  The interpreter stays for small calls, where a compile (a few
// hundred ms) would not pay, and as the fallback when hiprtc fails.
std::atomic<int> g_ewise_jit_mode{0};              // 0 auto, 1 never, 2 always
std::atomic<long long> g_ewise_jit_compiled{0}, g_ewise_jit_launches{0};

namespace {

const char kJsMathSrc[] =
#define Q8_JS_MATH_BODY(...) #__VA_ARGS__
#include "q8_js_math.h"
#undef Q8_JS_MATH_BODY
    ;

constexpr int64_t EW_JIT_MIN_ELEMS = (int64_t)1 << 20;   // auto mode: compile from 2^20 elements
constexpr size_t EW_JIT_MAX_PROGRAMS = 256;               // then every further program is interpreted

// An exact C literal of v (hexadecimal significand).
std::string ew_lit(double v) {
  if (v != v) return "__builtin_nan(\"\")";
  if (__builtin_isinf(v)) return v > 0 ? "__builtin_inf()" : "(-__builtin_inf())";
  char buf[64];
  snprintf(buf, sizeof buf, "(%a)", v);
  return buf;
}

const char* ew_ctype(int dt) {
  switch (dt) {
    case Q8_I8: return "signed char";
    case Q8_U8: return "unsigned char";
    case Q8_I32: return "int";
    case Q8_F32: return "float";
    default: return "double";
  }
}

const char* ew_ctype4(int dt) {
  switch (dt) {
    case Q8_I8: return "char4";
    case Q8_U8: return "uchar4";
    case Q8_I32: return "int4";
    default: return "float4";
  }
}

int ew_size(int dt) {
  switch (dt) {
    case Q8_I8: case Q8_U8: return 1;
    case Q8_I32: case Q8_F32: return 4;
    default: return 8;
  }
}

// Load kinds of an input in the 4-element form
enum { EW_LD_EACH = 0, EW_LD_VEC = 1, EW_LD_BCAST = 2 };

// An exact C literal of a binary32 value v.
std::string ew_litf(double v) {
  if (v != v) return "__builtin_nanf(\"\")";
  if (__builtin_isinf(v)) return v > 0 ? "__builtin_inff()" : "(-__builtin_inff())";
  char buf[64];
  snprintf(buf, sizeof buf, "(%af)", v);
  return buf;
}

bool ew_is_f32(double v) { return v != v || (double)(float)v == v; }

// Static types of the compiled kernels' values: TF a binary32 value held as
// float, TI an int32 value (ToInt32's result, an i32 load) held as int, TD
// any other number, held as double.
enum { EW_TF = 0, EW_TI = 1, EW_TD = 2 };

// The kernel source of program p over V = 1 or 4 consecutive elements per
// lane (V = 4: the last loop's extent a multiple of 4, so the four share
// every other index; input j is read as one 4-vector (kind EW_LD_VEC:
// contiguous along the last loop and 4-element aligned), as one value for
// all four (EW_LD_BCAST: broadcast along it) or element by element, and the
// output is stored as one 4-vector, non-temporally when nts).  Each lane takes U such groups a
// grid stride apart and issues the loads of all U groups (every input the
// program reads) before any arithmetic, so that a lane has U loads in
// flight per input; a group past the end loads the last group again
// (clamped, so the loads stay unconditional) and is not stored.
//
// The program is straight-line code, so every instruction's value becomes a
// constant of its own (operands are read before the destination register
// names the new value, as in the interpreter), with a static type.  A value
// is float when it is exactly binary32: f32, i8 and u8 loads, binary32
// constants, loop indices below 2^24, comparisons, and every rounded
// (`rnd`) value.  Operations on float operands run in binary32 where that
// gives the f64 evaluation's bits: max, min, abs, neg, floor, ceil, round,
// sign, comparisons and ToInt32 are exact; fround(a + b), fround(a - b),
// fround(a * b) and fround(a / b) of binary32 a and b are the binary32
// operations themselves (53 >= 2 * 24 + 2: rounding the f64 result to
// binary32 gives the correctly rounded binary32 result).  fround(a / c) by a
// constant c that is not binary32 goes through js_fround_div_const (through
// js_fround_div_const_f, without a division, when a is binary32).  Every
// other operation runs in f64 on the operands converted exactly.
std::string ewise_jit_source(const q8_ew_prog& p, bool narrow, int V, int U, const int* kind, bool nts) {
  const std::string I = narrow ? "unsigned int" : "long long";
  auto icon = [&](int64_t v) {
    char buf[48];
    snprintf(buf, sizeof buf, "((%s)(%" PRId64 "LL))", I.c_str(), v);
    return std::string(buf);
  };
  const int last = p.ndims - 1;
  // No #include: hiprtc declares the HIP built-ins, vector types and math
  // functions itself, and an included header is found only where comgr
  // locates the ROCm tree (not under every launcher, e.g. a profiler's).
  std::string s = kJsMathSrc;
  if (nts)   // native vectors: the non-temporal store builtin takes no HIP vector structs
    s += "\ntypedef float ew_f4 __attribute__((ext_vector_type(4)));\n"
         "typedef int ew_i4 __attribute__((ext_vector_type(4)));\n"
         "typedef double ew_d2 __attribute__((ext_vector_type(2)));\n";
  s += "\nstruct EwJitPtrs { const void* in[" + std::to_string(Q8_EW_MAX_INPUTS) + "]; void* out; };\n";
  s += "extern \"C\" __global__ __launch_bounds__(" + std::to_string(EW_NT) +
       ") void q8_ew_jit(EwJitPtrs ptr, long long n) {\n";
  const std::string Vs = std::to_string(V);
  s += "  const long long G = (long long)gridDim.x * " + std::to_string(EW_NT) + ", nv = n / " + Vs + ";\n";
  s += "  for (long long t = (long long)blockIdx.x * " + std::to_string(EW_NT) + " + threadIdx.x; t < nv; t += G * " +
       std::to_string(U) + ") {\n";
  for (int u = 0; u < U; ++u) {
    const std::string us = std::to_string(u);
    if (u == 0) s += "    const long long t0 = t;\n";
    else s += "    const long long t" + us + " = t + " + us + " * G < nv ? t + " + us + " * G : nv - 1;\n";
    s += "    const long long e" + us + " = t" + us + " * " + Vs + ";\n";
    s += "    " + I + " rem" + us + " = (" + I + ")e" + us + ";\n";
    for (int d = last; d >= 0; --d) {
      const std::string x = icon(p.extent[d]);
      s += "    const " + I + " i" + std::to_string(d) + "_" + us + " = rem" + us + " % " + x + "; rem" + us +
           " /= " + x + ";\n";
    }
    s += "    (void)rem" + us + ";\n";
  }

  // register state: the type of the value it names, the value's variable
  // (per lane: name + "_" + lane) or a literal, and the constant if known
  struct Reg { int t = EW_TF; std::string name = "0.0f"; bool lit = true; bool known = true; double k = 0.0; };
  Reg reg[Q8_EW_MAX_REGS];
  const int NL = U * V;   // lane L: group L / V, element L % V of it
  auto X = [&](int r, int k) { return reg[r].lit ? reg[r].name : reg[r].name + "_" + std::to_string(k); };
  auto D = [&](int r, int k) { return reg[r].t == EW_TD ? X(r, k) : "(double)" + X(r, k); };
  static const char* ctype[] = {"float", "int", "double"};
  static const char* cmp_ops[] = {"==", "!=", "<", "<=", ">", ">="};
  static const char* lanes[] = {"x", "y", "z", "w"};
  // defines instruction pc's value from per-lane expressions of type t,
  // rounded to binary32 when rnd is set
  auto define = [&](int pc, const q8_ew_instr& in, int t, const std::vector<std::string>& ex) {
    const bool rnd = in.rnd && t != EW_TF;
    const int tt = rnd ? EW_TF : t;
    const std::string name = "v" + std::to_string(pc);
    for (int L = 0; L < NL; ++L)
      s += std::string("    const ") + ctype[tt] + " " + name + "_" + std::to_string(L) + " = " +
           (rnd ? "(float)(" + ex[L] + ")" : ex[L]) + ";\n";
    Reg& r = reg[in.dst];
    r.t = tt;
    r.name = name;
    r.lit = false;
    r.known = false;
  };
  // every load first: per LOAD instruction, its values per lane
  std::vector<std::vector<std::string>> ld(p.ncode);
  for (int pc = 0; pc < p.ncode; ++pc) {
    const q8_ew_instr& in = p.code[pc];
    if (in.op != Q8_EW_LOAD) continue;
    const int j = in.aux;
    const int dt = p.in_dtype[j];
    const int t = dt == Q8_F64 ? EW_TD : dt == Q8_I32 ? EW_TI : EW_TF;
    const std::string base = std::string("((const ") + ew_ctype(dt) + "*)ptr.in[" + std::to_string(j) + "])";
    const std::string cv = std::string("(") + ctype[t] + ")";
    const int kd = V == 1 ? EW_LD_EACH : kind[j];
    ld[pc].resize(NL);
    for (int u = 0; u < U; ++u) {
      const std::string us = std::to_string(u);
      std::string off = icon(p.in_coef[j][Q8_EW_MAX_DIMS]);
      for (int d = 0; d < p.ndims; ++d)
        if (p.in_coef[j][d] != 0) off += " + " + icon(p.in_coef[j][d]) + " * i" + std::to_string(d) + "_" + us;
      const std::string q = "q" + std::to_string(pc) + "_" + us;
      for (int k = 0; k < V; ++k) {
        std::string& e = ld[pc][u * V + k];
        if (kd == EW_LD_VEC && dt == Q8_F64) e = q + (k < 2 ? "a." : "b.") + lanes[k & 1];
        else if (kd == EW_LD_VEC) e = cv + q + "." + lanes[k];
        else if (kd == EW_LD_BCAST) e = q;
        else e = q + "_" + std::to_string(k);
      }
      if (kd == EW_LD_VEC && dt == Q8_F64) {
        s += "    const double2 " + q + "a = *(const double2*)(" + base + " + " + off + "), " + q +
             "b = *(const double2*)(" + base + " + " + off + " + 2);\n";
      } else if (kd == EW_LD_VEC) {
        s += std::string("    const ") + ew_ctype4(dt) + " " + q + " = *(const " + ew_ctype4(dt) + "*)(" + base +
             " + " + off + ");\n";
      } else if (kd == EW_LD_BCAST) {
        s += std::string("    const ") + ctype[t] + " " + q + " = " + cv + base + "[" + off + "];\n";
      } else {
        for (int k = 0; k < V; ++k)
          s += std::string("    const ") + ctype[t] + " " + q + "_" + std::to_string(k) + " = " + cv + base + "[" +
               off + (k ? " + " + icon(p.in_coef[j][last] * k) : "") + "];\n";
      }
    }
  }
  // The symmetric int8 quantize chain, as QuantizationPass's expression
  // leaves it: DIV(a, c) rounded to binary32, ROUND, MAX with -128, MIN
  // with 127, TOINT32 (constants may sit between them), with a binary32 a
  // and a constant c in [2^-100, 2^100], and every intermediate register
  // read by the next step only.  It is emitted at the DIV as one
  // js_quant_i8 per element (the library's quantize fast path) and bound to
  // the TOINT32's register when that instruction is reached.
  auto reads_later = [&](int r, int from) {   // r read at or after `from` before it is redefined
    for (int q = from; q < p.ncode; ++q) {
      const q8_ew_instr& x = p.code[q];
      const bool src = x.op != Q8_EW_LOAD && x.op != Q8_EW_CONST && x.op != Q8_EW_INDEX;
      if (src && (x.a == r || x.b == r || x.c == r)) return true;
      if (x.dst == r) return false;
    }
    return r == p.result;
  };
  std::vector<int> qchain(p.ncode, -1);        // at the DIV: pc of its TOINT32; at the rest: -2
  std::string qname;                          // the fused value awaiting its TOINT32
  auto match_quant = [&](int pc) {
    const q8_ew_instr& dv = p.code[pc];
    if (dv.op != Q8_EW_DIV || !dv.rnd || reg[dv.a].t != EW_TF || !reg[dv.b].known) return -1;
    const double c = reg[dv.b].k;
    if (!(c >= 0x1p-100 && c <= 0x1p100)) return -1;
    // constants as they will stand at each step
    bool kn[Q8_EW_MAX_REGS];
    double kv[Q8_EW_MAX_REGS];
    for (int r = 0; r < Q8_EW_MAX_REGS; ++r) { kn[r] = reg[r].known; kv[r] = reg[r].k; }
    const int want[4] = {Q8_EW_ROUND, Q8_EW_MAX, Q8_EW_MIN, Q8_EW_TOINT32};
    int cur = dv.dst, q = pc + 1;
    std::vector<int> steps;
    for (int k = 0; k < 4; ++k) {
      while (q < p.ncode && p.code[q].op == Q8_EW_CONST) {
        const q8_ew_instr& x = p.code[q];
        if (x.dst == cur) return -1;
        kn[x.dst] = true;
        kv[x.dst] = x.rnd ? (double)(float)p.konst[x.aux] : p.konst[x.aux];
        ++q;
      }
      if (q >= p.ncode || p.code[q].op != want[k]) return -1;
      const q8_ew_instr& x = p.code[q];
      if (k == 0 || k == 3) {
        if (x.a != cur) return -1;
      } else {
        const double bound = k == 1 ? -128.0 : 127.0;
        const int other = x.a == cur ? x.b : x.b == cur ? x.a : -1;
        if (other < 0 || other == cur || !kn[other] || kv[other] != bound) return -1;
      }
      if (reads_later(cur, q + 1)) return -1;
      steps.push_back(q);
      cur = x.dst;
      ++q;
    }
    for (int st : steps) qchain[st] = -2;
    return steps.back();
  };
  for (int pc = 0; pc < p.ncode; ++pc) {
    const q8_ew_instr& in = p.code[pc];
    std::vector<std::string> ex(NL);
    if (qchain[pc] == -2) {                     // a step of a fused quantize chain
      if (in.op == Q8_EW_TOINT32) {
        Reg& r = reg[in.dst];
        r.t = EW_TI;
        r.name = qname;
        r.lit = false;
        r.known = false;
      }
      continue;
    }
    if (in.op == Q8_EW_DIV) {
      const int end = match_quant(pc);
      if (end >= 0) {
        const double c = reg[in.b].k;
        qname = "v" + std::to_string(pc);
        for (int L = 0; L < NL; ++L)
          s += "    const int " + qname + "_" + std::to_string(L) + " = js_quant_i8(" + X(in.a, L) + ", " +
               ew_litf((double)(float)(1.0 / c)) + ", " + ew_lit(c) + ");\n";
        continue;
      }
    }
    if (in.op == Q8_EW_LOAD) {
      const int dt = p.in_dtype[in.aux];
      define(pc, in, dt == Q8_F64 ? EW_TD : dt == Q8_I32 ? EW_TI : EW_TF, ld[pc]);
      continue;
    }
    if (in.op == Q8_EW_CONST) {
      double v = p.konst[in.aux];
      if (in.rnd) v = (double)(float)v;
      Reg& r = reg[in.dst];
      r.t = ew_is_f32(v) ? EW_TF : EW_TD;
      r.name = r.t == EW_TF ? ew_litf(v) : ew_lit(v);
      r.lit = true;
      r.known = true;
      r.k = v;
      continue;
    }
    const int ta = reg[in.a].t, tb = reg[in.b].t, tc = reg[in.c].t;
    const bool ff = ta == EW_TF && tb == EW_TF, ii = ta == EW_TI && tb == EW_TI;
    int t = EW_TD;
    for (int L = 0; L < NL; ++L) {
      const int k = L % V;
      const std::string us = std::to_string(L / V);
      const std::string a = X(in.a, L), b = X(in.b, L), c = X(in.c, L);
      const std::string da = D(in.a, L), db = D(in.b, L), dc = D(in.c, L);
      std::string v;
      switch (in.op) {
        case Q8_EW_INDEX:
          t = p.extent[in.aux] <= ((int64_t)1 << 24) ? EW_TF : EW_TD;
          v = std::string("(") + ctype[t] + ")(i" + std::to_string(in.aux) + "_" + us +
              (in.aux == last && k ? " + " + icon(k) : "") + ")";
          break;
        case Q8_EW_ADD: case Q8_EW_SUB: case Q8_EW_MUL: case Q8_EW_DIV: {
          const char* o = in.op == Q8_EW_ADD ? " + " : in.op == Q8_EW_SUB ? " - " : in.op == Q8_EW_MUL ? " * " : " / ";
          const Reg& rb = reg[in.b];
          const double cb = rb.k;
          if (in.rnd && ff) {
            t = EW_TF;
            v = a + o + b;
          } else if (in.rnd && in.op == Q8_EW_DIV && rb.known && cb == cb && !__builtin_isinf(cb) &&
                     __builtin_fabs(cb) >= 0x1p-1000 && __builtin_fabs(cb) <= 0x1p1000) {
            t = EW_TF;
            const double ac = __builtin_fabs(cb);
            if (ta == EW_TF && ac >= 0x1p-800 && ac <= 0x1p800)
              v = "js_fround_div_const_f(" + a + ", " + ew_lit(ac) + ", " + ew_lit(1.0 / ac) + ", " +
                  (cb < 0 ? "true" : "false") + ")";
            else
              v = "js_fround_div_const(" + da + ", " + ew_lit(cb) + ", " + ew_lit(1.0 / cb) + ")";
          } else {
            v = da + o + db;
          }
          break;
        }
        case Q8_EW_IDIV: v = "trunc(" + da + " / " + db + ")"; break;
        case Q8_EW_MOD: case Q8_EW_FMOD: v = "js_rem(js_rem(" + da + ", " + db + ") + " + db + ", " + db + ")"; break;
        case Q8_EW_FLOORDIV: v = "floor(" + da + " / " + db + ")"; break;
        case Q8_EW_TMOD: v = "js_rem(" + da + ", " + db + ")"; break;
        case Q8_EW_TDIV: t = EW_TI; v = "js_to_int32(" + da + " / " + db + ")"; break;
        case Q8_EW_NEG:
          if (ta == EW_TF) { t = EW_TF; v = "-" + a; } else { v = "-" + da; }
          break;
        case Q8_EW_CMP: {
          const char* o = cmp_ops[in.aux <= 5 ? in.aux : 5];
          t = EW_TF;
          v = (ff || ii ? "((" + a + " " + o + " " + b + ")" : "((" + da + " " + o + " " + db + ")") + " ? 1.0f : 0.0f)";
          break;
        }
        case Q8_EW_SELECT: {
          const std::string cond = ta == EW_TF ? "truthyf(" + a + ")" : ta == EW_TI ? "(" + a + " != 0)"
                                                                                    : "truthy(" + a + ")";
          if (tb == tc) { t = tb; v = "(" + cond + " ? " + b + " : " + c + ")"; }
          else { v = "(" + cond + " ? " + db + " : " + dc + ")"; }
          break;
        }
        case Q8_EW_TOINT32:
          t = EW_TI;
          v = ta == EW_TF ? "js_to_int32f(" + a + ")" : ta == EW_TI ? a : "js_to_int32(" + a + ")";
          break;
        case Q8_EW_TOBOOL:
          t = EW_TF;
          v = (ta == EW_TF ? "(truthyf(" + a + ")" : ta == EW_TI ? "((" + a + " != 0)" : "(truthy(" + a + ")") +
              " ? 1.0f : 0.0f)";
          break;
        case Q8_EW_MAX: case Q8_EW_MIN: {
          const bool mx = in.op == Q8_EW_MAX;
          if (ff) { t = EW_TF; v = std::string(mx ? "js_maxf(" : "js_minf(") + a + ", " + b + ")"; }
          else if (ii) { t = EW_TI; v = "(" + a + (mx ? " > " : " < ") + b + " ? " + a + " : " + b + ")"; }
          else { v = std::string(mx ? "js_max(" : "js_min(") + da + ", " + db + ")"; }
          break;
        }
        case Q8_EW_ABS:
          if (ta == EW_TF) { t = EW_TF; v = "__builtin_fabsf(" + a + ")"; } else { v = "fabs(" + da + ")"; }
          break;
        case Q8_EW_FLOOR: case Q8_EW_CEIL: case Q8_EW_ROUND: {
          const char* ff32 = in.op == Q8_EW_FLOOR ? "__builtin_floorf(" : in.op == Q8_EW_CEIL ? "__builtin_ceilf(" : "js_roundf(";
          const char* ff64 = in.op == Q8_EW_FLOOR ? "floor(" : in.op == Q8_EW_CEIL ? "ceil(" : "js_round_full(";
          if (ta == EW_TF) { t = EW_TF; v = ff32 + a + ")"; }
          else if (ta == EW_TI) { t = EW_TI; v = a; }
          else { v = ff64 + a + ")"; }
          break;
        }
        case Q8_EW_SIGN:
          if (ta == EW_TF) { t = EW_TF; v = "js_signf(" + a + ")"; } else { v = "js_sign(" + da + ")"; }
          break;
        case Q8_EW_SQRT: v = "sqrt(" + da + ")"; break;
        case Q8_EW_EXP: v = "exp(" + da + ")"; break;
        case Q8_EW_LOG: v = "log(" + da + ")"; break;
        case Q8_EW_TANH: v = "tanh(" + da + ")"; break;
        case Q8_EW_RSQRT: v = "1.0 / sqrt(" + da + ")"; break;
        case Q8_EW_POW: v = "pow(" + da + ", " + db + ")"; break;
        default: t = ta; v = a; break;
      }
      ex[L] = v;
    }
    define(pc, in, t, ex);
  }
  // the store: Float32Array / Float64Array conversion, ToInt32 and its low bits
  const int rt = reg[p.result].t;
  auto conv = [&](int k) {
    const std::string r = X(p.result, k);
    const std::string i32 = rt == EW_TI ? r : rt == EW_TF ? "js_to_int32f(" + r + ")" : "js_to_int32(" + r + ")";
    switch (p.out_dtype) {
      case Q8_F32: return rt == EW_TF ? r : "(float)" + r;
      case Q8_F64: return rt == EW_TD ? r : "(double)" + r;
      case Q8_I32: return i32;
      case Q8_I8: return "(signed char)(unsigned char)(unsigned int)" + i32;
      default: return "(unsigned char)(unsigned int)" + i32;
    }
  };
  for (int u = 0; u < U; ++u) {
    const std::string us = std::to_string(u), e = "e" + us;
    const int L0 = u * V;
    std::string st;
    if (V == 4 && p.out_dtype == Q8_F64) {
      if (nts)
        st = "__builtin_nontemporal_store((ew_d2){" + conv(L0) + ", " + conv(L0 + 1) + "}, (ew_d2*)ptr.out + " + e +
             " / 2); __builtin_nontemporal_store((ew_d2){" + conv(L0 + 2) + ", " + conv(L0 + 3) +
             "}, (ew_d2*)ptr.out + " + e + " / 2 + 1);";
      else
        st = "((double2*)ptr.out)[" + e + " / 2] = make_double2(" + conv(L0) + ", " + conv(L0 + 1) + "); " +
             "((double2*)ptr.out)[" + e + " / 2 + 1] = make_double2(" + conv(L0 + 2) + ", " + conv(L0 + 3) + ");";
    } else if (V == 4) {
      const char* t4 = p.out_dtype == Q8_F32 ? "float4" : p.out_dtype == Q8_I32 ? "int4"
                       : p.out_dtype == Q8_I8 ? "char4" : "uchar4";
      const char* mk = p.out_dtype == Q8_F32 ? "make_float4" : p.out_dtype == Q8_I32 ? "make_int4"
                       : p.out_dtype == Q8_I8 ? "make_char4" : "make_uchar4";
      const std::string val = std::string(mk) + "(" + conv(L0) + ", " + conv(L0 + 1) + ", " + conv(L0 + 2) + ", " +
                              conv(L0 + 3) + ")";
      if (nts) {
        // the four values as one native vector (f32, i32) or one 32-bit word (i8, u8)
        const char* nt = p.out_dtype == Q8_F32 ? "ew_f4" : p.out_dtype == Q8_I32 ? "ew_i4" : "int";
        st = std::string("{ const ") + t4 + " t_ = " + val + "; __builtin_nontemporal_store(*(const " + nt +
             "*)&t_, (" + nt + "*)((" + t4 + "*)ptr.out + " + e + " / 4)); }";
      } else {
        st = std::string("((") + t4 + "*)ptr.out)[" + e + " / 4] = " + val + ";";
      }
    } else if (nts) {
      st = std::string("__builtin_nontemporal_store((") + ew_ctype(p.out_dtype) + ")(" + conv(L0) + "), (" +
           ew_ctype(p.out_dtype) + "*)ptr.out + " + e + ");";
    } else {
      st = std::string("((") + ew_ctype(p.out_dtype) + "*)ptr.out)[" + e + "] = " + conv(L0) + ";";
    }
    s += u == 0 ? "    " + st + "\n" : "    if (t + " + us + " * G < nv) { " + st + " }\n";
  }
  s += "  }\n}\n";
  return s;
}

// Guards the compile cache and g_jit_error: why the last failed compile
// failed (the failing step, its error string, the hiprtc log), "" if none has.
std::mutex g_jit_mu;
std::string g_jit_error;

// The compiled kernel of a program source on the current device (nullptr
// if hiprtc or the module load failed; the failure is cached too).  With
// may_compile false only a kernel already compiled is returned, and a miss
// is not cached.
hipFunction_t ewise_jit_kernel(const std::string& src, bool may_compile) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  static std::unordered_map<std::string, hipFunction_t> cache;
  const std::string key = std::to_string(dev) + "\n" + src;
  std::lock_guard<std::mutex> lock(g_jit_mu);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  if (!may_compile || cache.size() >= EW_JIT_MAX_PROGRAMS) return nullptr;
  hipFunction_t fn = nullptr;
  std::string why;
  hiprtcProgram prog;
  hiprtcResult rc = hiprtcCreateProgram(&prog, src.c_str(), "q8_ew_jit.hip", 0, nullptr, nullptr);
  if (rc != HIPRTC_SUCCESS) {
    why = std::string("hiprtcCreateProgram: ") + hiprtcGetErrorString(rc);
  } else {
    // the library's own arithmetic flags: IEEE, no contraction, no packed FP32
    const char* opts[] = {"--offload-arch=gfx950", "-O3", "-ffp-contract=off", "-fno-fast-math",
                          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
    rc = hiprtcCompileProgram(prog, (int)(sizeof opts / sizeof opts[0]), opts);
    size_t sz = 0;
    if (rc != HIPRTC_SUCCESS) {
      why = std::string("hiprtcCompileProgram: ") + hiprtcGetErrorString(rc);
      size_t ln = 0;
      if (hiprtcGetProgramLogSize(prog, &ln) == HIPRTC_SUCCESS && ln > 1) {
        std::string log(ln, '\0');
        if (hiprtcGetProgramLog(prog, &log[0]) == HIPRTC_SUCCESS) why += "\n" + log;
      }
    } else if ((rc = hiprtcGetCodeSize(prog, &sz)) != HIPRTC_SUCCESS || sz == 0) {
      why = std::string("hiprtcGetCodeSize: ") + hiprtcGetErrorString(rc);
    } else {
      std::vector<char> code(sz);
      hipModule_t mod;
      hipError_t he;
      if ((rc = hiprtcGetCode(prog, code.data())) != HIPRTC_SUCCESS)
        why = std::string("hiprtcGetCode: ") + hiprtcGetErrorString(rc);
      else if ((he = hipModuleLoadData(&mod, code.data())) != hipSuccess)
        why = std::string("hipModuleLoadData: ") + hipGetErrorString(he);
      else if ((he = hipModuleGetFunction(&fn, mod, "q8_ew_jit")) != hipSuccess) {
        why = std::string("hipModuleGetFunction: ") + hipGetErrorString(he);
        fn = nullptr;
      }
    }
    hiprtcDestroyProgram(&prog);
  }
  if (!fn) g_jit_error = why;
  (void)hipGetLastError();   // a failed load must not surface at the next launch
  cache.emplace(key, fn);
  if (fn) g_ewise_jit_compiled.fetch_add(1, std::memory_order_relaxed);
  return fn;
}

}  // namespace

size_t ewise_jit_error(char* buf, size_t cap) {
  std::lock_guard<std::mutex> lock(g_jit_mu);
  if (buf && cap > 0) snprintf(buf, cap, "%s", g_jit_error.c_str());
  return g_jit_error.size();
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
  const int mode = g_ewise_jit_mode.load(std::memory_order_relaxed);
  if (mode == 2 || (mode == 0 && n >= EW_JIT_MIN_ELEMS)) {
    // four elements per lane when the last loop's extent allows it and the
    // output is 16-byte aligned (as torch and the addon allocate)
    int kind[Q8_EW_MAX_INPUTS] = {};
    const int last = p.ndims - 1;
    const bool v4 = p.ndims >= 1 && p.extent[last] % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(out) % (4 * (uintptr_t)ew_size(p.out_dtype) < 16
                                                            ? 4 * (uintptr_t)ew_size(p.out_dtype) : 16) == 0;
    for (int j = 0; v4 && j < p.ninputs; ++j) {
      const int64_t cl = p.in_coef[j][last];
      bool aligned = cl == 1 && p.in_coef[j][Q8_EW_MAX_DIMS] % 4 == 0 &&
                     reinterpret_cast<uintptr_t>(inputs[j]) % (uintptr_t)(4 * ew_size(p.in_dtype[j]) < 16
                                                                         ? 4 * ew_size(p.in_dtype[j]) : 16) == 0;
      for (int d = 0; d < last; ++d) aligned = aligned && p.in_coef[j][d] % 4 == 0;
      kind[j] = cl == 0 ? EW_LD_BCAST : aligned ? EW_LD_VEC : EW_LD_EACH;
    }
    // groups per lane: 2 when the program has arithmetic enough for the
    // second group's loads to overlap the first group's work (measured on
    // [4096, 4096]: a 7-operation ReLU + quantize 22.6 -> 21.5 us), else 1
    // (a 2-operation dequant + add, bound by HBM, 28.3 -> 29.3 us with 2);
    // 1 as well for the externs with long f64 code paths, whose copies
    // would grow the kernel's code
    bool slow = false;
    int arith = 0;
    for (int i = 0; i < p.ncode; ++i) {
      const int op = p.code[i].op;
      slow = slow || op == Q8_EW_EXP || op == Q8_EW_LOG || op == Q8_EW_TANH || op == Q8_EW_POW ||
             op == Q8_EW_MOD || op == Q8_EW_FMOD || op == Q8_EW_TMOD || op == Q8_EW_RSQRT;
      arith += op != Q8_EW_LOAD && op != Q8_EW_CONST;
    }
    const int U = !slow && arith >= 6 ? 2 : 1;
    // no compile while the stream is captured into a graph: a module load
    // there may be refused, and a refusal must not stick to the program;
    // a program compiled before launches the same way captured or not
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const bool may_compile = hipStreamIsCapturing(st, &cap) != hipSuccess || cap == hipStreamCaptureStatusNone;
    (void)hipGetLastError();
    // non-temporal stores above 32 MiB of output: smaller outputs stay in
    // the MALL for the kernel that reads them next (the rule the quantize
    // kernels follow); measured on [4096, 4096] dequant + add, 64 MiB of
    // f32 out: 28.3 -> 26.6 us
    const bool nts = n * (int64_t)ew_size(p.out_dtype) > ((int64_t)32 << 20);
    if (hipFunction_t fn = ewise_jit_kernel(ewise_jit_source(p, narrow, v4 ? 4 : 1, U, kind, nts), may_compile)) {
      long long nn = (long long)n;
      void* args[] = {&ptr, &nn};
      const int64_t vblocks = (n / (v4 ? 4 : 1) + (int64_t)EW_NT * U - 1) / ((int64_t)EW_NT * U);
      const unsigned vgrid = (unsigned)(vblocks < 16384 ? vblocks : 16384);
      const hipError_t err = hipModuleLaunchKernel(fn, vgrid, 1, 1, EW_NT, 1, 1, 0, st, args, nullptr);
      if (err == hipSuccess) g_ewise_jit_launches.fetch_add(1, std::memory_order_relaxed);
      return err;
    }
  }
  if (narrow) hipLaunchKernelGGL((k_ewise<true>), dim3(grid), dim3(EW_NT), 0, st, p, ptr, dv, n);
  else hipLaunchKernelGGL((k_ewise<false>), dim3(grid), dim3(EW_NT), 0, st, p, ptr, dv, n);
  return hipGetLastError();
}

}  // namespace q8
