// q8_zp.hip -- quantized_dot with zero points and ui8 operands, on top of
// the signed int8 GEMM / GEMV.
//
// The reference's quantized_dot (rules/quantization.ts:23-42) adds
// ((a|0) - zpA) * ((b|0) - zpB), with a and b read from Int8Array (i8) or
// Uint8Array (ui8) operands, and stores the exact sum ToInt32.  With
//   a' = a (i8) or (int8)(a ^ 0x80) = a - 128 (ui8),   cA = 128*[ui8] - zpA,
// (and b', cB likewise) every term is (a' + cA)(b' + cB), so
//   acc = sum a'b' + cB * sum_k a'[m,k] + cA * sum_k b'[n,k] + K * cA * cB
// where sum a'b' is the int8 GEMM of the flipped operands and the rest is a
// rank-1 correction from row sums -- all exact modulo 2^32, which is the
// ToInt32 of the exact sum.
#include "q8_device.h"
#include "q8_internal.h"

namespace q8 {

static int zp_grid(int64_t items, int cap) {
  const int64_t g = (items + 255) / 256;
  return (int)(g < 1 ? 1 : (g < cap ? g : cap));
}

// dst = src ^ 0x80 bytewise (a ui8 code u becomes the int8 u - 128).
__global__ __launch_bounds__(256) void k_flip_u8(const uint8_t* __restrict__ src,
                                                 int8_t* __restrict__ dst, int64_t n, int vec) {
  const int64_t t0 = blockIdx.x * 256LL + threadIdx.x, stride = (int64_t)gridDim.x * 256;
  int64_t done = 0;
  if (vec) {
    const int64_t n16 = n >> 4;
    for (int64_t j = t0; j < n16; j += stride) {
      v4i v = reinterpret_cast<const v4i*>(src)[j];
      v ^= 0x80808080;
      reinterpret_cast<v4i*>(dst)[j] = v;
    }
    done = n16 << 4;
  }
  for (int64_t j = done + t0; j < n; j += stride) dst[j] = (int8_t)(src[j] ^ 0x80u);
}

// out[r] = sum_k X[r,k] (int8 values, int32 wrap), one workgroup per row.
__global__ __launch_bounds__(256) void k_row_sums_i8(const int8_t* __restrict__ X, int64_t rows,
                                                     int64_t K, int vec, int32_t* __restrict__ out) {
  __shared__ int red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const int8_t* x = X + r * K;
    uint32_t s = 0;
    int64_t done = 0;
    if (vec) {                                          // K % 4 == 0, 4-byte aligned rows
      const int* x4 = reinterpret_cast<const int*>(x);
      for (int64_t j = tid; j < (K >> 2); j += 256)
        s = (uint32_t)__builtin_amdgcn_sdot4(x4[j], 0x01010101, (int)s, false);
      done = K;
    }
    for (int64_t j = done + tid; j < K; j += 256) s += (uint32_t)(int)x[j];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += (uint32_t)__shfl_xor((int)s, o, 64);
    if (lane == 0) red[wave] = (int)s;
    __syncthreads();
    if (tid == 0)
      out[r] = (int32_t)((uint32_t)red[0] + (uint32_t)red[1] + (uint32_t)red[2] + (uint32_t)red[3]);
    __syncthreads();
  }
}

// acc[m,n] += cB * rsA[m] + cA * csB[n] + K * cA * cB   (mod 2^32)
__global__ __launch_bounds__(256) void k_zp_correct(int32_t* __restrict__ acc, int64_t M, int64_t N,
                                                    const int32_t* __restrict__ rsA,
                                                    const int32_t* __restrict__ csB, int32_t cA,
                                                    int32_t cB, uint32_t kcc) {
  const int64_t total = M * N, stride = (int64_t)gridDim.x * 256;
  for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < total; i += stride) {
    const int64_t m = i / N, n = i - m * N;
    uint32_t v = (uint32_t)acc[i] + kcc;
    if (rsA) v += (uint32_t)cB * (uint32_t)rsA[m];
    if (csB) v += (uint32_t)cA * (uint32_t)csB[n];
    acc[i] = (int32_t)v;
  }
}

// dst[0..n) = value (a byte): 16-byte stores over the aligned middle, byte
// stores at the ends.  A kernel rather than hipMemsetAsync, so that a
// caller may capture q8_memset in a HIP graph.
__global__ __launch_bounds__(256) void k_fill_u8(uint8_t* __restrict__ dst, int64_t head,
                                                 int64_t n16, int64_t n, uint32_t v4) {
  const int64_t t0 = blockIdx.x * 256LL + threadIdx.x, stride = (int64_t)gridDim.x * 256;
  v4i* mid = reinterpret_cast<v4i*>(dst + head);
  const v4i v = {(int)v4, (int)v4, (int)v4, (int)v4};
  for (int64_t j = t0; j < n16; j += stride) mid[j] = v;
  const int64_t tail0 = head + 16 * n16;
  for (int64_t j = t0; j < head + (n - tail0); j += stride) {
    const int64_t i = j < head ? j : tail0 + (j - head);
    dst[i] = (uint8_t)(v4 & 0xffu);
  }
}

hipError_t launch_fill_u8(void* dst, int value, int64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  uint8_t* d = static_cast<uint8_t*>(dst);
  int64_t head = (int64_t)((16 - (reinterpret_cast<uintptr_t>(d) & 15)) & 15);
  if (head > n) head = n;
  const int64_t n16 = (n - head) / 16;
  const uint32_t b = (uint32_t)value & 0xffu;
  const int64_t items = n16 > 0 ? n16 : n;
  hipLaunchKernelGGL(k_fill_u8, dim3((unsigned)zp_grid(items, 8 * cu_count())), dim3(256), 0, st, d,
                     head, n16, n, b * 0x01010101u);
  return hipGetLastError();
}

hipError_t launch_flip_u8(const uint8_t* src, int8_t* dst, int64_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  const int vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
  const int64_t items = vec ? (n + 15) / 16 : n;
  hipLaunchKernelGGL(k_flip_u8, dim3((unsigned)zp_grid(items, 8 * cu_count())), dim3(256), 0, st,
                     src, dst, n, vec);
  return hipGetLastError();
}

hipError_t launch_row_sums_i8(const int8_t* X, int64_t rows, int64_t K, int32_t* out,
                              hipStream_t st) {
  if (rows == 0) return hipSuccess;
  const int vec = (K % 4 == 0) && (reinterpret_cast<uintptr_t>(X) & 3) == 0;
  const int64_t grid = rows < 65536 ? rows : 65536;
  hipLaunchKernelGGL(k_row_sums_i8, dim3((unsigned)grid), dim3(256), 0, st, X, rows, K, vec, out);
  return hipGetLastError();
}

hipError_t launch_zp_correct(int32_t* acc, int64_t M, int64_t N, const int32_t* rsA,
                             const int32_t* csB, int32_t cA, int32_t cB, int64_t K,
                             hipStream_t st) {
  if (M * N == 0) return hipSuccess;
  const uint32_t kcc = (uint32_t)(uint64_t)K * (uint32_t)cA * (uint32_t)cB;
  hipLaunchKernelGGL(k_zp_correct, dim3((unsigned)zp_grid(M * N, 8 * cu_count())), dim3(256), 0,
                     st, acc, M, N, rsA, csB, cA, cB, kcc);
  return hipGetLastError();
}

}  // namespace q8
