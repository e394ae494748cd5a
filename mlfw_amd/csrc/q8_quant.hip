// q8_quant.hip -- HBM-bound kernels of the int8 path for gfx950:
// seeded input fill, static / per-token / per-tensor quantize, dequantize,
// per-channel weight packing and the fused SiLU*up + per-token quantize.
//
// Layout: every fp32 / int8 tensor is row-major in HBM.  Rows are read with
// 128-bit coalesced loads (float4 = 16 B per lane, 1 KiB per wave64
// instruction) when the row length is a multiple of 4 elements and the base
// is 16-byte aligned; a scalar grid-stride form handles everything else.
// Per-row absmax reductions run in registers: a row of up to 12 KiB floats
// stays in VGPRs (VPT float4 per thread) so the row is read from HBM once.
#include <atomic>

#include "q8_device.h"
#include "q8_internal.h"

namespace q8 {

static constexpr int NT = 256;   // threads per block for the streaming kernels

// ------------------------------------------------------------------ inputs
// mulberry32 (src/util/random.ts:5-14) in counter form: the generator state
// after draw i is seed + (i+1) * 0x6D2B79F5 (mod 2^32), so every draw is
// independent of the others.
__device__ __forceinline__ double mb32(uint32_t seed, uint64_t i) {
  uint32_t a = seed + (uint32_t)(i + 1) * 0x6D2B79F5u;
  uint32_t t = (a ^ (a >> 15)) * (1u | a);
  t = (t + ((t ^ (t >> 7)) * (61u | t))) ^ t;
  return (double)(t ^ (t >> 14)) / 4294967296.0;
}

// normal_ (src/nn/init.ts:40-52): element pair p uses draws 2p, 2p+1.
__global__ __launch_bounds__(NT) void k_fill_normal(float* __restrict__ out, int64_t n,
                                                    uint32_t seed, uint64_t offset,
                                                    double mean, double std) {
  int64_t pairs = (n + 1) >> 1;
  for (int64_t p = blockIdx.x * (int64_t)NT + threadIdx.x; p < pairs;
       p += (int64_t)gridDim.x * NT) {
    double u1 = mb32(seed, offset + 2 * p);
    if (u1 == 0.0) u1 = 1e-10;
    double u2 = mb32(seed, offset + 2 * p + 1);
    double r = sqrt(-2.0 * log(u1));
    double theta = 6.283185307179586 * u2;
    out[2 * p] = (float)(mean + std * r * cos(theta));
    if (2 * p + 1 < n) out[2 * p + 1] = (float)(mean + std * r * sin(theta));
  }
}

// uniform_ (src/nn/init.ts:31-37)
__global__ __launch_bounds__(NT) void k_fill_uniform(float* __restrict__ out, int64_t n,
                                                     uint32_t seed, uint64_t offset,
                                                     double a, double b) {
  double range = b - a;
  for (int64_t i = blockIdx.x * (int64_t)NT + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * NT)
    out[i] = (float)(a + mb32(seed, offset + i) * range);
}

// Compute units of the current device, cached per device (the first call
// is made by device set-up, so launches inside a graph capture only read).
int cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

static int grid_for(int64_t work, int64_t per_block, int cap) {
  int64_t g = (work + per_block - 1) / per_block;
  if (g < 1) g = 1;
  return (int)(g > cap ? cap : g);
}

hipError_t launch_fill_normal(float* out, int64_t n, uint32_t seed, uint64_t offset,
                              double mean, double std, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_normal, dim3(grid_for((n + 1) / 2, NT, 65536)), dim3(NT), 0, st,
                     out, n, seed, offset, mean, std);
  return hipGetLastError();
}

hipError_t launch_fill_uniform(float* out, int64_t n, uint32_t seed, uint64_t offset,
                               double a, double b, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_uniform, dim3(grid_for(n, NT, 65536)), dim3(NT), 0, st,
                     out, n, seed, offset, a, b);
  return hipGetLastError();
}

__global__ __launch_bounds__(NT) void k_apply_outliers(float* __restrict__ x, int64_t n,
                                                       uint32_t seed, double p, double factor) {
  for (int64_t i = blockIdx.x * (int64_t)NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * NT)
    if (mb32(seed, (uint64_t)i) < p) x[i] = (float)((double)x[i] * factor);
}

hipError_t launch_apply_outliers(float* x, int64_t n, uint32_t seed, double p, double factor,
                                 hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_apply_outliers, dim3(grid_for(n, NT, 65536)), dim3(NT), 0, st,
                     x, n, seed, p, factor);
  return hipGetLastError();
}

// ------------------------------------------------------------------ helpers
// Block-wide max of an int key over TPB threads (TPB / 64 waves).  `red`
// is LDS of TPB / 64 ints.
template <int TPB>
__device__ __forceinline__ int block_max_i32_n(int key, int* red) {
  key = wave_max_i32(key);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = key;
  __syncthreads();
  int k = red[0];
#pragma unroll
  for (int w = 1; w < TPB / 64; ++w) k = k > red[w] ? k : red[w];
  __syncthreads();   // red is reused by the next row
  return k;
}

// Block-wide max of an int key (256 threads = 4 waves).  `red` is LDS.
__device__ __forceinline__ int block_max_i32(int key, int* red) {
  key = wave_max_i32(key);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) red[wid] = key;
  __syncthreads();
  int k = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) k = k > red[w] ? k : red[w];
  __syncthreads();   // red is reused by the next row
  return k;
}

// ------------------------------------------------------------------ static quantize
// R1 with a compile-time scale (quant_math.ts:16-27), any n, any alignment.
__global__ __launch_bounds__(NT) void k_quant_static(const float* __restrict__ x, int64_t n,
                                                     double s, double zp, int is_u8,
                                                     uint8_t* __restrict__ q) {
  const int lo = is_u8 ? 0 : -128, hi = is_u8 ? 255 : 127;
  const bool fast = (zp == 0.0) && !is_u8 && fast_scale_ok(s);
  const float r32 = (float)(1.0 / s);
  const int64_t stride = (int64_t)gridDim.x * NT;
  const int64_t i0 = blockIdx.x * (int64_t)NT + threadIdx.x;
  const bool vec = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(q) & 3) == 0);
  if (vec) {
    const int64_t n4 = n >> 2;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    int* q4 = reinterpret_cast<int*>(q);
    for (int64_t i = i0; i < n4; i += stride) {
      float4 v = x4[i];
      int p;
      if (fast) {
        p = quant4_sym(v, true, r32, s);
      } else {
        p = pack4(quant_exact(v.x, s, zp, lo, hi), quant_exact(v.y, s, zp, lo, hi),
                  quant_exact(v.z, s, zp, lo, hi), quant_exact(v.w, s, zp, lo, hi));
      }
      q4[i] = p;
    }
    for (int64_t i = (n4 << 2) + i0; i < n; i += stride)
      q[i] = (uint8_t)(fast ? quant_sym_fast(x[i], r32, s) : quant_exact(x[i], s, zp, lo, hi));
  } else {
    for (int64_t i = i0; i < n; i += stride)
      q[i] = (uint8_t)(fast ? quant_sym_fast(x[i], r32, s) : quant_exact(x[i], s, zp, lo, hi));
  }
}

hipError_t launch_quant_static(const float* x, int64_t n, double s, double zp, int is_u8,
                               void* q, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_quant_static, dim3(grid_for((n + 3) / 4, NT, 8192)), dim3(NT), 0, st,
                     x, n, s, zp, is_u8, static_cast<uint8_t*>(q));
  return hipGetLastError();
}

// ------------------------------------------------------------------ per-token quantize
// One block per row (grid-stride over rows).  The first VPT*1024 elements
// of the row stay in registers between the absmax reduction and the
// quantize, so such rows are read once; longer rows re-read the tail.
// Loads are non-temporal: the input is touched once, and keeping it out of
// the caches measured ~5-10% faster than plain loads.  Stores are
// non-temporal too (NTS) unless the codes are small enough to stay in the
// MALL for the GEMM that reads them next (see launch_quant_rows).
// A block with several rows loads the next row while it reduces and
// quantizes the current one (two register sets, used alternately).  Every
// row is loaded through its own buffer resource whose size is 0 past the
// last row, so the loads are issued unconditionally and a missing row
// reads zeros without touching memory; the loads in flight are then the
// same on every path and the wait before a row's reduction leaves the
// next row's loads outstanding.
// TPB threads per block; ONE: the grid has a block per row (no prefetch of
// a next row, half the registers).
template <int VPT, bool FULL, bool NTS, int TPB = NT, bool ONE = false>
__global__ __launch_bounds__(TPB) void k_quant_rows(const float* __restrict__ x, int64_t ldx,
                                                   int64_t M,
                                                   int64_t K, int8_t* __restrict__ q,
                                                   double* __restrict__ scales) {
  constexpr int NT = TPB;
  __shared__ int red[NT / 64];
  const int tid = threadIdx.x;
  const int64_t K4 = K >> 2;       // FULL: K4 == VPT * NT, no bounds to test
  const int last = (int)K4 - 1;
  const int64_t G = gridDim.x;
  // The resource spans only the part of the row the VPT register loads
  // cover (at most VPT * NT float4, 48 KiB), so num_records never wraps
  // however long the row is; the rest of a long row is read directly.
  constexpr int64_t SPAN = (int64_t)VPT * NT * 16;
  const int rec = (int)(K * 4 < SPAN ? K * 4 : SPAN);
  auto load_row = [&](int64_t row, float4* v) {
    const bool in = row < M;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(x + (in ? row : 0) * ldx), (short)0, in ? rec : 0, 0x00020000);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int i = tid + j * NT;
      const uint32_t off = (FULL || i <= last) ? 16u * (uint32_t)i : 0x80000000u;
      const v4f t = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
      v[j] = make_float4(t.x, t.y, t.z, t.w);
    }
  };
  auto process_row = [&](int64_t row, const float4* v) {
    const v4f* xr = reinterpret_cast<const v4f*>(x + row * ldx);
    int* qr = reinterpret_cast<int*>(q + row * K);
    int key = -1;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int k = key4(v[j]);
      key = (FULL || tid + j * NT <= last) && k > key ? k : key;
    }
    if constexpr (!FULL) {
      for (int64_t i = tid + (int64_t)VPT * NT; i < K4; i += NT) {
        const v4f t = xr[i];
        int k = key4(make_float4(t.x, t.y, t.z, t.w));
        key = key > k ? key : k;
      }
    }
    key = block_max_i32_n<NT>(key, red);
    const double s = scale_from_key(key);
    if (tid == 0) scales[row] = s;
    const bool fast = fast_scale_ok(s);
    const float r32 = (float)(1.0 / s);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int i = tid + j * NT;
      if (FULL || i < K4) {
        const int c = quant4_sym(v[j], fast, r32, s);
        if constexpr (NTS) __builtin_nontemporal_store(c, qr + i);
        else qr[i] = c;
      }
    }
    if constexpr (!FULL) {
      for (int64_t i = tid + (int64_t)VPT * NT; i < K4; i += NT) {
        const v4f t = xr[i];
        const int c = quant4_sym(make_float4(t.x, t.y, t.z, t.w), fast, r32, s);
        if constexpr (NTS) __builtin_nontemporal_store(c, qr + i);
        else qr[i] = c;
      }
    }
  };
  if constexpr (ONE) {
    float4 v[VPT];
    load_row(blockIdx.x, v);
    __builtin_amdgcn_sched_barrier(0);
    process_row(blockIdx.x, v);
    return;
  }
  float4 va[VPT], vb[VPT];
  int64_t row = blockIdx.x;
  load_row(row, va);
  for (; row < M; row += 2 * G) {
    load_row(row + G, vb);
    // no arithmetic above this point of the iteration (the scheduler would
    // otherwise start on the first loaded group and issue the rest after it)
    __builtin_amdgcn_sched_barrier(0);
    process_row(row, va);
    load_row(row + 2 * G, va);
    if (row + G >= M) break;                       // uniform
    __builtin_amdgcn_sched_barrier(0);
    process_row(row + G, vb);
  }
}

// Any K / row stride / alignment: two passes over the row with scalar loads.
__global__ __launch_bounds__(NT) void k_quant_rows_scalar(const float* __restrict__ x, int64_t ldx,
                                                          int64_t M,
                                                          int64_t K, int8_t* __restrict__ q,
                                                          double* __restrict__ scales) {
  __shared__ int red[NT / 64];
  for (int64_t row = blockIdx.x; row < M; row += gridDim.x) {
    const float* xr = x + row * ldx;
    int key = -1;
    for (int64_t i = threadIdx.x; i < K; i += NT) {
      int k = absmax_key(xr[i]);
      key = key > k ? key : k;
    }
    key = block_max_i32(key, red);
    const double s = K == 0 ? 6.0 / 127.0 : scale_from_key(key);
    if (threadIdx.x == 0) scales[row] = s;
    const bool fast = fast_scale_ok(s);
    const float r32 = (float)(1.0 / s);
    for (int64_t i = threadIdx.x; i < K; i += NT)
      q[row * K + i] = (int8_t)(fast ? quant_sym_fast(xr[i], r32, s)
                                     : quant_exact(xr[i], s, 0.0, -128, 127));
  }
}

hipError_t launch_quant_rows(const float* x, int64_t ldx, int64_t M, int64_t K, int8_t* q,
                             double* scales, hipStream_t st) {
  if (M == 0) return hipSuccess;
  const int grid = (int)(M < 1048576 ? M : 1048576);
  const bool vec = (K % 4 == 0) && (ldx % 4 == 0) && ((reinterpret_cast<uintptr_t>(x) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(q) & 3) == 0);
  if (!vec) {
    hipLaunchKernelGGL(k_quant_rows_scalar, dim3(grid), dim3(NT), 0, st, x, ldx, M, K, q, scales);
    return hipGetLastError();
  }
  const int64_t K4 = K / 4;
  if (K4 == 0) {        // rows of zero length: only the scales are written
    hipLaunchKernelGGL(k_quant_rows_scalar, dim3(grid), dim3(NT), 0, st, x, ldx, M, K, q, scales);
    return hipGetLastError();
  }
  // Row workers: one workgroup per row (measured against resident grids of
  // 0.5x to 4x the 8 workgroups per CU, which pipeline several rows per
  // workgroup: equal for 2048-4096 rows, 10-20% slower for 16384); a grid
  // capped at 2^20 workgroups walks the rest with the pipelined loop.
  const int workers = (int)(M < 1048576 ? M : 1048576);
  // The codes are read next by the GEMM.  Up to 32 MiB (an eighth of the
  // 256 MB MALL) they are stored normally and stay in the cache for it (C3
  // step, 16 MiB of codes: 86.5 -> 85.1 us); larger outputs gain nothing
  // there and use non-temporal stores, faster for this kernel (64 MiB:
  // 53.9 us instead of 57.2 us).
  const bool nts = M * K > ((int64_t)32 << 20);
#define Q8_QROWS_S(V, FULLK, S)                                                             \
  hipLaunchKernelGGL((k_quant_rows<V, FULLK, S>), dim3(workers), dim3(NT), 0, st, x, ldx, M, K, q, \
                     scales)
#define Q8_QROWS_W(FULLK, S)                                                                \
  hipLaunchKernelGGL((k_quant_rows<6, FULLK, S, 512, true>), dim3(workers), dim3(512), 0, st, x, ldx, M, \
                     K, q, scales)
#define Q8_QROWS(V)                                                                          \
  do {                                                                                       \
    if (K4 == (V) * NT) {                                                                    \
      if (nts) Q8_QROWS_S(V, true, true); else Q8_QROWS_S(V, true, false);                   \
    } else {                                                                                 \
      if (nts) Q8_QROWS_S(V, false, true); else Q8_QROWS_S(V, false, false);                 \
    }                                                                                        \
  } while (0)
  if (K4 <= 1 * NT) Q8_QROWS(1);
  else if (K4 <= 2 * NT) Q8_QROWS(2);
  else if (K4 <= 4 * NT) Q8_QROWS(4);
  else if (K4 <= 8 * NT) Q8_QROWS(8);
  else if (K4 <= 6 * 512 && M <= workers) {
    // rows of up to 12288 elements, one block per row: 512 threads with 6
    // float4 each and no second register set (no next row to prefetch) --
    // 2048 x 11008: 22.2 us against 27.3 us for 256 threads x 12 with the
    // prefetch set (165 VGPRs, 3 waves per SIMD)
    if (K4 == 6 * 512) {
      if (nts) Q8_QROWS_W(true, true); else Q8_QROWS_W(true, false);
    } else {
      if (nts) Q8_QROWS_W(false, true); else Q8_QROWS_W(false, false);
    }
  } else Q8_QROWS(12);
#undef Q8_QROWS_W
#undef Q8_QROWS
#undef Q8_QROWS_S
  return hipGetLastError();
}

// ------------------------------------------------------------------ per-tensor quantize
// The reduction key lives in the caller's own scales[0] (8 bytes), so calls
// with distinct outputs share no memory and may run concurrently on any
// streams.  The key is the binary64 bit pattern of a candidate scale,
// amax_b / 127 for a block's NaN-ignoring absmax amax_b, combined with a
// 64-bit atomic max: non-negative doubles order like their bit patterns,
// and x -> x / 127 (one rounding) is non-decreasing, so the max of the
// candidates is exactly max(amax) / 127.  It starts at -1 ("no non-NaN
// value seen").  Phase 1 raises it; phase 2 turns it into the final scale
//   s = key < 0 ? Infinity : (key == 0 ? 1e-10 : key)
// (S-abs with fromRange's `|| 1e-10`, and the (+inf, -inf) range of an
// observer that saw only NaNs), quantizes its share with s, and block 0
// stores s back into scales[0].  That mapping is idempotent (s maps to s),
// so a block that reads scales[0] after block 0's store derives the same s;
// every access to the key is atomic.
__global__ void k_set_i64(long long* p, long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ double scale_from_dkey(long long key) {
  if (key < 0) return __builtin_inf();
  const double s = __longlong_as_double(key);
  return s == 0.0 ? 1e-10 : s;
}

__global__ __launch_bounds__(NT) void k_absmax_tensor(const float* __restrict__ x, int64_t n,
                                                      long long* __restrict__ dkey) {
  __shared__ int red[NT / 64];
  int key = -1;
  const int64_t stride = (int64_t)gridDim.x * NT;
  const int64_t i0 = blockIdx.x * (int64_t)NT + threadIdx.x;
  if ((reinterpret_cast<uintptr_t>(x) & 15) == 0) {
    const int64_t n4 = n >> 2;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    for (int64_t i = i0; i < n4; i += stride) {
      int k = key4(x4[i]);
      key = key > k ? key : k;
    }
    for (int64_t i = (n4 << 2) + i0; i < n; i += stride) {
      int k = absmax_key(x[i]);
      key = key > k ? key : k;
    }
  } else {
    for (int64_t i = i0; i < n; i += stride) {
      int k = absmax_key(x[i]);
      key = key > k ? key : k;
    }
  }
  key = block_max_i32(key, red);
  if (threadIdx.x == 0 && key >= 0) {
    const double s = (double)__uint_as_float((unsigned)key) / 127.0;
    __hip_atomic_fetch_max(dkey, __double_as_longlong(s), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
}

__global__ __launch_bounds__(NT) void k_quant_tensor(const float* __restrict__ x, int64_t n,
                                                     long long* dkey, int8_t* __restrict__ q) {
  const double s = n == 0 ? 6.0 / 127.0
                          : scale_from_dkey(__hip_atomic_load(dkey, __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT));
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(dkey, __double_as_longlong(s), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool fast = fast_scale_ok(s);
  const float r32 = (float)(1.0 / s);
  const int64_t stride = (int64_t)gridDim.x * NT;
  const int64_t i0 = blockIdx.x * (int64_t)NT + threadIdx.x;
  if ((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(q) & 3) == 0) {
    const int64_t n4 = n >> 2;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    int* q4 = reinterpret_cast<int*>(q);
    for (int64_t i = i0; i < n4; i += stride) q4[i] = quant4_sym(x4[i], fast, r32, s);
    for (int64_t i = (n4 << 2) + i0; i < n; i += stride)
      q[i] = (int8_t)(fast ? quant_sym_fast(x[i], r32, s) : quant_exact(x[i], s, 0.0, -128, 127));
  } else {
    for (int64_t i = i0; i < n; i += stride)
      q[i] = (int8_t)(fast ? quant_sym_fast(x[i], r32, s) : quant_exact(x[i], s, 0.0, -128, 127));
  }
}

hipError_t launch_quant_tensor(const float* x, int64_t n, int8_t* q, double* scales,
                               hipStream_t st) {
  // A fill kernel (not a memset) starts the key, so the sequence can be
  // captured in a HIP graph.
  long long* dkey = reinterpret_cast<long long*>(scales);
  hipLaunchKernelGGL(k_set_i64, dim3(1), dim3(1), 0, st, dkey, -1LL);
  const int grid = grid_for((n + 3) / 4, NT * 4, 2048);
  if (n > 0) hipLaunchKernelGGL(k_absmax_tensor, dim3(grid), dim3(NT), 0, st, x, n, dkey);
  hipLaunchKernelGGL(k_quant_tensor, dim3(grid), dim3(NT), 0, st, x, n, dkey, q);
  return hipGetLastError();
}

// ------------------------------------------------------------------ dequantize
// D1 (quant_math.ts:29-34).  grid.y walks rows, grid.x 4-element groups of
// a row: every lane loads one 32-bit word of codes (4 int8/uint8, or one
// int32 per element for SRC 2 as a 16-byte load) and stores one float4, so
// each wave-wide store writes 1 KiB contiguous.  GPT groups per thread are
// loaded before any is converted; one f64 multiply and one RNE conversion
// per element.  TPB x GPT groups per workgroup pass: 512 x 2 for rows of
// 4096 elements and more (16384 x 4096 i8: 54.5 us, 77% of HBM, against
// 56.5 us for 256 x 4, 59 us for 128 x 8 and 65 us for 1024 x 1), 256 x 4
// below.
template <int SRC, int TPB, int GPT>  // SRC 0 i8, 1 u8, 2 i32
__global__ __launch_bounds__(TPB) void k_dequant_vec(const void* __restrict__ qv, int64_t M,
                                                     int64_t K, const double* __restrict__ scales,
                                                     int per_row, double zp,
                                                     float* __restrict__ y) {
  constexpr int NT = TPB;
  const int64_t groups = K >> 2;
  for (int64_t row = blockIdx.y; row < M; row += gridDim.y) {
    const double s = scales[per_row ? row : 0];
    for (int64_t g0 = blockIdx.x * (int64_t)(NT * GPT) + threadIdx.x; g0 < groups;
         g0 += (int64_t)gridDim.x * NT * GPT) {
      // every load is issued, unconditionally (a lane past the row end
      // reloads the last group and stores nothing), before any arithmetic
      v4i c32[SRC == 2 ? GPT : 1];
      int c8[GPT];
#pragma unroll
      for (int t = 0; t < GPT; ++t) {
        const int64_t g = min(g0 + (int64_t)t * NT, groups - 1);
        if constexpr (SRC == 2)
          c32[t] = __builtin_nontemporal_load(
              reinterpret_cast<const v4i*>(static_cast<const int32_t*>(qv) + row * K) + g);
        else
          c8[t] = __builtin_nontemporal_load(
              reinterpret_cast<const int*>(static_cast<const int8_t*>(qv) + row * K) + g);
      }
      // an unconditional use of each value here, after all the loads: the
      // compiler may not sink a load into the branch that stores its group
#pragma unroll
      for (int t = 0; t < GPT; ++t) {
        if constexpr (SRC == 2) asm volatile("" ::"v"(c32[t]));
        else asm volatile("" ::"v"(c8[t]));
      }
      int w[GPT][4];
#pragma unroll
      for (int t = 0; t < GPT; ++t) {
        if constexpr (SRC == 2) {
          w[t][0] = c32[t].x; w[t][1] = c32[t].y; w[t][2] = c32[t].z; w[t][3] = c32[t].w;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int b = (c8[t] >> (8 * e)) & 0xff;
            w[t][e] = SRC == 0 ? (int)(int8_t)b : b;
          }
        }
      }
#pragma unroll
      for (int t = 0; t < GPT; ++t) {
        const int64_t g = g0 + (int64_t)t * NT;
        if (g < groups) {
          v4f o = {dequant((double)w[t][0], s, zp), dequant((double)w[t][1], s, zp),
                   dequant((double)w[t][2], s, zp), dequant((double)w[t][3], s, zp)};
          __builtin_nontemporal_store(o, reinterpret_cast<v4f*>(y + row * K) + g);
        }
      }
    }
  }
}

__global__ __launch_bounds__(NT) void k_dequant_scalar(const void* __restrict__ qv, int src,
                                                       int64_t M, int64_t K,
                                                       const double* __restrict__ scales,
                                                       int per_row, double zp,
                                                       float* __restrict__ y) {
  const int64_t n = M * K;
  for (int64_t i = blockIdx.x * (int64_t)NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * NT) {
    const double s = scales[per_row ? i / K : 0];
    double v;
    if (src == 0) v = (double)static_cast<const int8_t*>(qv)[i];
    else if (src == 1) v = (double)static_cast<const uint8_t*>(qv)[i];
    else v = (double)static_cast<const int32_t*>(qv)[i];
    y[i] = dequant(v, s, zp);
  }
}

hipError_t launch_dequant(const void* q, int src, int64_t M, int64_t K, const double* scales,
                          int per_row, double zp, float* y, hipStream_t st) {
  if (M == 0 || K == 0) return hipSuccess;
  const bool vec = (K % 4 == 0) && ((reinterpret_cast<uintptr_t>(q) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(y) & 15) == 0);
  if (!vec) {
    hipLaunchKernelGGL(k_dequant_scalar, dim3(grid_for(M * K, NT, 65536)), dim3(NT), 0, st,
                       q, src, M, K, scales, per_row, zp, y);
    return hipGetLastError();
  }
  const unsigned gy = (unsigned)(M < 65535 ? M : 65535);
#define Q8_DQ(SRC, T, G)                                                                        \
  hipLaunchKernelGGL((k_dequant_vec<SRC, T, G>), dim3(grid_for(K / 4, (T) * (G), 1024), gy), dim3(T), \
                     0, st, q, M, K, scales, per_row, zp, y)
  if (K / 4 >= 1024) {
    if (src == 0) Q8_DQ(0, 512, 2);
    else if (src == 1) Q8_DQ(1, 512, 2);
    else Q8_DQ(2, 512, 2);
  } else {
    if (src == 0) Q8_DQ(0, 256, 4);
    else if (src == 1) Q8_DQ(1, 256, 4);
    else Q8_DQ(2, 256, 4);
  }
#undef Q8_DQ
  return hipGetLastError();
}

// ------------------------------------------------------------------ weight packing
// fromConstantArrayPerChannel's per-channel fix-ups on a (min, max) pair,
// then fromRangePerChannel's scale (quantization_types.ts:266-281, 311-316).
__device__ __forceinline__ double channel_scale(double mn, double mx) {
  if (!isfinite(mn)) mn = -1.0;
  if (!isfinite(mx)) mx = 1.0;
  if (mn == mx) { mn -= 0.5; mx += 0.5; }
  double a = fabs(mn) > fabs(mx) ? fabs(mn) : fabs(mx);
  double s = a / 127.0;
  return (s == 0.0 || s != s) ? 1e-10 : s;
}

// axis 0: one block per row (channel).  fminf / fmaxf ignore NaN exactly
// like the reference's `v < min` / `v > max` updates.
__global__ __launch_bounds__(NT) void k_wscale_rows(const float* __restrict__ W, int64_t rows,
                                                    int64_t cols, double* __restrict__ scales) {
  __shared__ float rmn[NT / 64], rmx[NT / 64];
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    float mn = __builtin_inff(), mx = -__builtin_inff();
    for (int64_t c = threadIdx.x; c < cols; c += NT) {
      float v = W[r * cols + c];
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      mn = fminf(mn, __shfl_xor(mn, o, 64));
      mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    }
    if ((threadIdx.x & 63) == 0) { rmn[threadIdx.x >> 6] = mn; rmx[threadIdx.x >> 6] = mx; }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < NT / 64; ++w) { mn = fminf(mn, rmn[w]); mx = fmaxf(mx, rmx[w]); }
      mn = fminf(rmn[0], mn);
      mx = fmaxf(rmx[0], mx);
      scales[r] = channel_scale((double)mn, (double)mx);
    }
    __syncthreads();
  }
}

// axis 1: a block owns 64 columns; 4 row phases stride the rows.
__global__ __launch_bounds__(NT) void k_wscale_cols(const float* __restrict__ W, int64_t rows,
                                                    int64_t cols, double* __restrict__ scales) {
  __shared__ float smn[NT], smx[NT];
  const int col_in = threadIdx.x & 63, phase = threadIdx.x >> 6;
  const int64_t c = blockIdx.x * 64LL + col_in;
  float mn = __builtin_inff(), mx = -__builtin_inff();
  if (c < cols)
    for (int64_t r = phase; r < rows; r += NT / 64) {
      float v = W[r * cols + c];
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
  smn[threadIdx.x] = mn;
  smx[threadIdx.x] = mx;
  __syncthreads();
  if (phase == 0 && c < cols) {
    for (int p = 1; p < NT / 64; ++p) {
      mn = fminf(mn, smn[p * 64 + col_in]);
      mx = fmaxf(mx, smx[p * 64 + col_in]);
    }
    scales[c] = channel_scale((double)mn, (double)mx);
  }
}

// per tensor: order-key min / max of the whole array into work[0], work[1],
// the two 32-bit halves of the caller's scales[0]; k_wscale_tensor (one
// thread) reads both keys and then overwrites them with the f64 scale.
__global__ void k_set_minmax_init(int* work) {
  work[0] = 0x7fffffff;             // key of +NaN-free max -> min starts high
  work[1] = (int)0x80000000;        // max starts low
}

__global__ __launch_bounds__(NT) void k_wminmax_tensor(const float* __restrict__ W, int64_t n,
                                                       int* __restrict__ work) {
  __shared__ int rmn[NT / 64], rmx[NT / 64];
  int mn = 0x7fffffff, mx = (int)0x80000000;
  for (int64_t i = blockIdx.x * (int64_t)NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * NT) {
    float v = W[i];
    if (v == v) {
      int k = order_key(v);
      mn = mn < k ? mn : k;
      mx = mx > k ? mx : k;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    int a = __shfl_xor(mn, o, 64), b = __shfl_xor(mx, o, 64);
    mn = mn < a ? mn : a;
    mx = mx > b ? mx : b;
  }
  if ((threadIdx.x & 63) == 0) { rmn[threadIdx.x >> 6] = mn; rmx[threadIdx.x >> 6] = mx; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < NT / 64; ++w) { mn = mn < rmn[w] ? mn : rmn[w]; mx = mx > rmx[w] ? mx : rmx[w]; }
    atomicMin(&work[0], mn);
    atomicMax(&work[1], mx);
  }
}

// fromConstantArray (quantization_types.ts:287-297) on the reduced keys.
// The keys are read before the scale overwrites them (one thread).
__global__ void k_wscale_tensor(double* scales) {
  const int* work = reinterpret_cast<const int*>(scales);
  const int kmn = work[0], kmx = work[1];
  const bool none = kmn == 0x7fffffff && kmx == (int)0x80000000;
  double mn = none ? __builtin_inf() : (double)from_order_key(kmn);
  double mx = none ? -__builtin_inf() : (double)from_order_key(kmx);
  scales[0] = channel_scale(mn, mx);
}

// R2 (quantization_types.ts:75-79, 118-130): q = clamp(JSround(w/s + 0)), f64.
__device__ __forceinline__ int wquant(float w, double s, int lo, int hi) {
  return clamp_to_int(js_round((double)w / s + 0.0), lo, hi);
}

// axis 0 / per tensor: same layout in and out.
__global__ __launch_bounds__(NT) void k_wquant_rows(const float* __restrict__ W, int64_t rows,
                                                    int64_t cols, const double* __restrict__ scales,
                                                    int per_tensor, int8_t* __restrict__ Wq) {
  const int lo = per_tensor ? -127 : -128, hi = 127;
  const int64_t n = rows * cols;
  for (int64_t i = blockIdx.x * (int64_t)NT + threadIdx.x; i < n; i += (int64_t)gridDim.x * NT) {
    const double s = scales[per_tensor ? 0 : i / cols];
    Wq[i] = (int8_t)wquant(W[i], s, lo, hi);
  }
}

// axis 1: W is [K=rows, N=cols]; Wq is [N, K].  64x64 tiles transposed
// through LDS so both the fp32 reads and the int8 writes are coalesced.
__global__ __launch_bounds__(NT) void k_wquant_cols_t(const float* __restrict__ W, int64_t rows,
                                                      int64_t cols, const double* __restrict__ scales,
                                                      int per_tensor, int8_t* __restrict__ Wq) {
  __shared__ int8_t tile[64][65];
  const int lo = per_tensor ? -127 : -128, hi = 127;
  const int64_t k0 = blockIdx.y * 64LL, n0 = blockIdx.x * 64LL;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t n = n0 + tx;
  const double s = n < cols ? scales[per_tensor ? 0 : n] : 1.0;
  for (int r = ty; r < 64; r += NT / 64) {
    const int64_t k = k0 + r;
    int8_t v = 0;
    if (k < rows && n < cols) v = (int8_t)wquant(W[k * cols + n], s, lo, hi);
    tile[tx][r] = v;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += NT / 64) {
    const int64_t nn = n0 + r, kk = k0 + tx;
    if (nn < cols && kk < rows) Wq[nn * rows + kk] = tile[r][tx];
  }
}

hipError_t launch_pack_weight(const float* W, int64_t rows, int64_t cols, int axis, int per_tensor,
                              int8_t* Wq, double* scales, hipStream_t st) {
  // An empty channel keeps the (inf, -inf) start values, which the fix-ups
  // turn into (-1, 1) -> 1/127; the scale kernels below produce that too.
  const int64_t nch = per_tensor ? 1 : (axis == 0 ? rows : cols);
  if (nch == 0) return hipSuccess;
  if (per_tensor) {
    int* work = reinterpret_cast<int*>(scales);
    hipLaunchKernelGGL(k_set_minmax_init, dim3(1), dim3(1), 0, st, work);
    hipLaunchKernelGGL(k_wminmax_tensor, dim3(grid_for(rows * cols, NT * 8, 2048)), dim3(NT), 0, st,
                       W, rows * cols, work);
    hipLaunchKernelGGL(k_wscale_tensor, dim3(1), dim3(1), 0, st, scales);
  } else if (axis == 0) {
    hipLaunchKernelGGL(k_wscale_rows, dim3((unsigned)(rows < 1048576 ? rows : 1048576)), dim3(NT),
                       0, st, W, rows, cols, scales);
  } else {
    hipLaunchKernelGGL(k_wscale_cols, dim3((unsigned)((cols + 63) / 64)), dim3(NT), 0, st,
                       W, rows, cols, scales);
  }
  if (rows == 0 || cols == 0) return hipGetLastError();
  if (axis == 0) {
    hipLaunchKernelGGL(k_wquant_rows, dim3(grid_for(rows * cols, NT, 65536)), dim3(NT), 0, st,
                       W, rows, cols, scales, per_tensor, Wq);
  } else {
    dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
    hipLaunchKernelGGL(k_wquant_cols_t, grid, dim3(NT), 0, st, W, rows, cols, scales, per_tensor, Wq);
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------ SiLU(g)*u + per-token quantize
// TPB threads per row: 256, or 512 for long rows, where a 256-thread
// block would hold 8-12 float4 of g and of u per lane and run 2 waves per
// SIMD; at 512 threads a lane holds 4-6 and the SIMD keeps more waves to
// hide the f64 exp behind the loads of other rows.
template <int VPT, int TPB>
__global__ __launch_bounds__(TPB) void k_silu_mul_quant_rows(const float* __restrict__ g,
                                                             const float* __restrict__ u,
                                                             int64_t ldg, int64_t ldu,
                                                             int64_t M, int64_t K,
                                                             float* __restrict__ h,
                                                             int8_t* __restrict__ q,
                                                             double* __restrict__ scales) {
  constexpr int NT = TPB;
  __shared__ int red[NT / 64];
  const int tid = threadIdx.x;
  const int64_t K4 = K >> 2;
  for (int64_t row = blockIdx.x; row < M; row += gridDim.x) {
    const float4* gr = reinterpret_cast<const float4*>(g + row * ldg);
    const float4* ur = reinterpret_cast<const float4*>(u + row * ldu);
    float4 v[VPT];
    int key = -1;
    // loads issued unconditionally (a lane past the row end reloads the
    // last group), so they are all in flight together
    float4 a[VPT], b[VPT];
    const int last = (int)K4 - 1;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int i = min(tid + j * NT, last);
      a[j] = gr[i];
      b[j] = ur[i];
    }
    // keep the SiLU arithmetic below every load (it would otherwise be
    // scheduled between them and hold later loads behind the first waits)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int64_t i = tid + (int64_t)j * NT;
      // fround(silu * up): a binary32 multiply (the exact product, rounded once)
      v[j] = make_float4(silu_js(a[j].x) * b[j].x, silu_js(a[j].y) * b[j].y,
                         silu_js(a[j].z) * b[j].z, silu_js(a[j].w) * b[j].w);
      if (i < K4) {
        if (h) reinterpret_cast<float4*>(h + row * K)[i] = v[j];
        const int k = key4(v[j]);
        key = key > k ? key : k;
      }
    }
    key = block_max_i32_n<TPB>(key, red);
    const double s = scale_from_key(key);
    if (tid == 0) scales[row] = s;
    const bool fast = fast_scale_ok(s);
    const float r32 = (float)(1.0 / s);
    int* qr = reinterpret_cast<int*>(q + row * K);
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int64_t i = tid + (int64_t)j * NT;
      if (i < K4) qr[i] = quant4_sym(v[j], fast, r32, s);
    }
  }
}

// Fallback for K % 4 != 0, a row stride that is not a multiple of 4,
// misaligned pointers or rows above 12 Ki elements: h is formed twice (scan,
// then quantize) from g and u.
__global__ __launch_bounds__(NT) void k_silu_mul_quant_rows_scalar(
    const float* __restrict__ g, const float* __restrict__ u, int64_t ldg, int64_t ldu, int64_t M,
    int64_t K,
    float* __restrict__ h, int8_t* __restrict__ q, double* __restrict__ scales) {
  __shared__ int red[NT / 64];
  for (int64_t row = blockIdx.x; row < M; row += gridDim.x) {
    int key = -1;
    for (int64_t i = threadIdx.x; i < K; i += NT) {
      float v = silu_js(g[row * ldg + i]) * u[row * ldu + i];
      if (h) h[row * K + i] = v;
      int k = absmax_key(v);
      key = key > k ? key : k;
    }
    key = block_max_i32(key, red);
    const double s = K == 0 ? 6.0 / 127.0 : scale_from_key(key);
    if (threadIdx.x == 0) scales[row] = s;
    const bool fast = fast_scale_ok(s);
    const float r32 = (float)(1.0 / s);
    for (int64_t i = threadIdx.x; i < K; i += NT) {
      float v = silu_js(g[row * ldg + i]) * u[row * ldu + i];
      q[row * K + i] = (int8_t)(fast ? quant_sym_fast(v, r32, s) : quant_exact(v, s, 0.0, -128, 127));
    }
  }
}

hipError_t launch_silu_mul_quant_rows(const float* g, int64_t ldg, const float* u, int64_t ldu,
                                      int64_t M, int64_t K,
                                      float* h, int8_t* q, double* scales, hipStream_t st) {
  if (M == 0) return hipSuccess;
  const int grid = (int)(M < 1048576 ? M : 1048576);
  const bool vec = (K % 4 == 0) && (ldg % 4 == 0) && (ldu % 4 == 0) && (K / 4 <= 6 * 512) &&
                   ((reinterpret_cast<uintptr_t>(g) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(u) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(h) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(q) & 3) == 0);
  if (!vec) {
    hipLaunchKernelGGL(k_silu_mul_quant_rows_scalar, dim3(grid), dim3(NT), 0, st, g, u, ldg, ldu, M,
                       K, h, q, scales);
    return hipGetLastError();
  }
  const int64_t K4 = K / 4;
  if (K4 == 0) {
    hipLaunchKernelGGL(k_silu_mul_quant_rows_scalar, dim3(grid), dim3(NT), 0, st, g, u, ldg, ldu, M,
                       K, h, q, scales);
    return hipGetLastError();
  }
  const int workers = (int)(M < 8 * cu_count() ? M : 8 * cu_count());
  // 256 threads per row up to 4 float4 per lane, then 512 (measured at
  // [2048, 8192] and [2048, 11008] against 256 threads x 8-12 and 1024
  // threads x 2-3 per lane, with and without occupancy limits)
  if (K4 <= 4 * 256)
    hipLaunchKernelGGL((k_silu_mul_quant_rows<4, 256>), dim3(workers), dim3(256), 0, st, g, u, ldg, ldu, M, K,
                       h, q, scales);
  else if (K4 <= 4 * 512)
    hipLaunchKernelGGL((k_silu_mul_quant_rows<4, 512>), dim3(workers), dim3(512), 0, st, g, u, ldg, ldu, M, K,
                       h, q, scales);
  else
    hipLaunchKernelGGL((k_silu_mul_quant_rows<6, 512>), dim3(workers), dim3(512), 0, st, g, u, ldg, ldu, M, K,
                       h, q, scales);
  return hipGetLastError();
}

}  // namespace q8
