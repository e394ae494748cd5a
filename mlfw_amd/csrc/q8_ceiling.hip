// q8_ceiling.hip -- measurement kernels for bench.py (libq8ceiling.so).
//
// Not part of the int8 path or its C ABI: these two kernels measure, on the
// box the benchmark runs on, the practical ceilings the path's kernels are
// held against next to the datasheet peaks.
//   * q8c_mfma: the C3 GEMM's MFMA work without its data movement -- 256
//     workgroups x 4 waves, each wave 2048 v_mfma_i32_32x32x32_i8 on a 4x4
//     grid of accumulators (the GEMM's per-wave count at 4096^3) with
//     random int8 operands (operand entropy sets the power draw, and so the
//     clock MI355X holds), cycled through 16 fragments held in registers:
//     nothing but MFMAs issues in the loop.  Reports the kernel time and the shader clock
//     read in the kernel (s_memtime against the 100 MHz s_memrealtime).
//   * q8c_stream: a streaming read or write of `bytes` (16-byte
//     non-temporal accesses, 1 KiB per wave instruction), the HBM floor of a
//     single kernel of that size including launch and ramp, timed as a graph
//     of `buffers` launches over distinct buffers (rotation defeats the
//     256 MB MALL).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t mix(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

__global__ __launch_bounds__(256, 1) void k_mfma(int iters, uint32_t seed, int* out,
                                                 long long* clk) {
  // 16 random fragments, generated once; the loop cycles through them with
  // compile-time indices, so no VGPR that feeds an in-flight MFMA is ever
  // rewritten (such a write stalls issue until the MFMA has read it) and
  // the only instructions in the loop are the MFMAs and the loop count.
  const uint32_t base = seed + (blockIdx.x * 256u + threadIdx.x) * 64u;
  v4i f[16];
#pragma unroll
  for (int i = 0; i < 16; ++i)
    f[i] = v4i{(int)mix(base + 4 * i), (int)mix(base + 4 * i + 1), (int)mix(base + 4 * i + 2),
               (int)mix(base + 4 * i + 3)};
  v16i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  long long t0 = 0, r0 = 0;
  if (threadIdx.x == 0) {
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  // each pass: 4 phases x 16 MFMAs; phase p pairs A fragment (i + 4p) % 16
  // with B fragment (8 + j + 4p) % 16
  for (int it = 0; it < iters; it += 4) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f[(i + 4 * p) & 15], f[(8 + j + 4 * p) & 15],
                                                            acc[i][j], 0, 0, 0);
  }
  int s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) s ^= acc[i][j][r];
  out[blockIdx.x * 256 + threadIdx.x] = s;
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    clk[0] = __builtin_amdgcn_s_memtime() - t0;
    clk[1] = __builtin_amdgcn_s_memrealtime() - r0;
  }
}

__global__ __launch_bounds__(256) void k_read(const v4i* __restrict__ p, int64_t nchunks, int* out) {
  constexpr int U = 4;
  const int64_t base = (int64_t)blockIdx.x * 256 * U;
  v4i w[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + (int64_t)u * 256 + threadIdx.x;
    w[u] = i < nchunks ? __builtin_nontemporal_load(p + i) : v4i{0, 0, 0, 0};
  }
  v4i acc = w[0] ^ w[1] ^ w[2] ^ w[3];
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x5eed1234) out[blockIdx.x] = acc.x;
}

__global__ __launch_bounds__(256) void k_write(v4i* __restrict__ p, int64_t nchunks, int seed) {
  constexpr int U = 4;
  const int64_t base = (int64_t)blockIdx.x * 256 * U;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + (int64_t)u * 256 + threadIdx.x;
    if (i < nchunks) __builtin_nontemporal_store(v4i{seed, (int)i, u, seed}, p + i);
  }
}

}  // namespace

extern "C" {

// MFMA ceiling: `reps` launches back to back; *us = average launch time,
// *mhz = shader clock over block 0's run of the last launch, *loop_cycles =
// that run's shader cycles (2048 MFMAs x 32 cycles = 65,536 when the MFMA
// pipe never idles).
__attribute__((visibility("default")))
int q8c_mfma(int iters_per_wave, int reps, double* us, double* mhz, double* loop_cycles) {
  const int blocks = 256;
  if (iters_per_wave < 1 || reps < 1 || !us || !mhz) return 1;
  int* out = nullptr;
  long long* clk = nullptr;
  hipEvent_t a = nullptr, b = nullptr;
  int rc = 2;
  if (hipMalloc(&out, blocks * 256 * sizeof(int)) != hipSuccess) return 2;
  if (hipMalloc(&clk, 2 * sizeof(long long)) == hipSuccess && hipEventCreate(&a) == hipSuccess &&
      hipEventCreate(&b) == hipSuccess) {
    // iters counts 16-MFMA steps: 2048 MFMAs per wave = 128 steps
    const int steps = iters_per_wave / 16 > 0 ? iters_per_wave / 16 : 1;
    hipLaunchKernelGGL(k_mfma, dim3(blocks), dim3(256), 0, 0, steps, 1u, out, clk);
    bool ok = hipEventRecord(a, 0) == hipSuccess;
    for (int i = 0; ok && i < reps; ++i)
      hipLaunchKernelGGL(k_mfma, dim3(blocks), dim3(256), 0, 0, steps, 7u * i + 3u, out, clk);
    ok = ok && hipGetLastError() == hipSuccess && hipEventRecord(b, 0) == hipSuccess;
    if (ok && hipEventSynchronize(b) == hipSuccess) {
      float ms = 0.f;
      long long h[2] = {0, 0};
      if (hipEventElapsedTime(&ms, a, b) == hipSuccess &&
          hipMemcpy(h, clk, sizeof(h), hipMemcpyDeviceToHost) == hipSuccess) {
        *us = 1e3 * ms / reps;
        *mhz = h[1] > 0 ? 100.0 * (double)h[0] / (double)h[1] : 0.0;
        if (loop_cycles) *loop_cycles = (double)h[0];
        rc = 0;
      }
    }
  }
  if (a) (void)hipEventDestroy(a);
  if (b) (void)hipEventDestroy(b);
  if (clk) (void)hipFree(clk);
  (void)hipFree(out);
  return rc;
}

// Streaming-read (write = 0) or streaming-write (write = 1) floor: a graph
// of `buffers` launches, each on its own buffer of `bytes`, replayed `reps`
// times; *us = average per launch.
__attribute__((visibility("default")))
int q8c_stream(size_t bytes, int buffers, int reps, int write, double* us) {
  if (bytes < 16 || buffers < 1 || reps < 1 || !us) return 1;
  std::vector<v4i*> bufs(buffers, nullptr);
  int* out = nullptr;
  hipStream_t s = nullptr;
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  hipEvent_t a = nullptr, b = nullptr;
  int rc = 2;
  bool ok = hipMalloc(&out, 1 << 20) == hipSuccess;
  for (int i = 0; ok && i < buffers; ++i)
    ok = hipMalloc(&bufs[i], bytes) == hipSuccess && hipMemset(bufs[i], i, bytes) == hipSuccess;
  ok = ok && hipStreamCreate(&s) == hipSuccess && hipEventCreate(&a) == hipSuccess &&
       hipEventCreate(&b) == hipSuccess;
  const int64_t nch = (int64_t)(bytes / 16);
  const int grid = (int)((nch + 1023) / 1024);
  if (ok && hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) == hipSuccess) {
    for (int i = 0; i < buffers; ++i) {
      if (write)
        hipLaunchKernelGGL(k_write, dim3(grid), dim3(256), 0, s, bufs[i], nch, i);
      else
        hipLaunchKernelGGL(k_read, dim3(grid), dim3(256), 0, s, bufs[i], nch, out);
    }
    ok = hipStreamEndCapture(s, &g) == hipSuccess &&
         hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) == hipSuccess;
    if (ok) ok = hipGraphLaunch(ge, s) == hipSuccess && hipStreamSynchronize(s) == hipSuccess;
    if (ok) {
      ok = hipEventRecord(a, s) == hipSuccess;
      for (int i = 0; ok && i < reps; ++i) ok = hipGraphLaunch(ge, s) == hipSuccess;
      ok = ok && hipEventRecord(b, s) == hipSuccess;
      float ms = 0.f;
      if (ok && hipEventSynchronize(b) == hipSuccess && hipEventElapsedTime(&ms, a, b) == hipSuccess) {
        *us = 1e3 * ms / ((double)reps * buffers);
        rc = 0;
      }
    }
  }
  if (ge) (void)hipGraphExecDestroy(ge);
  if (g) (void)hipGraphDestroy(g);
  if (a) (void)hipEventDestroy(a);
  if (b) (void)hipEventDestroy(b);
  if (s) (void)hipStreamDestroy(s);
  for (auto p : bufs)
    if (p) (void)hipFree(p);
  if (out) (void)hipFree(out);
  return rc;
}

}  // extern "C"
