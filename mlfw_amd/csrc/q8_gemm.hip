// q8_gemm.hip -- int8 x int8 -> int32 matmul with the dequant epilogue fused,
// for gfx950 (CDNA4).
//
// GEMM (M > 16): C[M,N] = A[M,K] . B[N,K]^T, both operands K-contiguous.
//   * v_mfma_i32_32x32x32_i8: a wave64 multiplies a 32x32 int8 A block by a
//     32x32 int8 B block into 16 int32 accumulators per lane.  Each lane
//     feeds 16 consecutive K bytes of one row of A and of one row of B
//     (row = lane % 32, K half = lane / 32), so A and B fragments are plain
//     128-bit LDS reads.
//   * A workgroup owns a BM x BN output tile and walks K in BK = 128 byte
//     steps.  Each step's A and B tiles are staged in LDS (row-major, 128 B
//     per row) with the 16-byte chunk index XOR-swizzled by (row & 7): the
//     32 lanes that read one column of chunks hit 8 different 16-byte bank
//     groups, so the ds_read_b128 fragment loads are conflict-free.
//   * Global -> LDS is double-buffered: step t+1 is loaded into registers
//     while the MFMAs of step t run out of the other LDS buffer; one
//     barrier per K step.
//   * The epilogue converts the int32 accumulators with the reference's
//     f64 arithmetic (fround(acc * fround(sA[m] * sB[n])) or
//     fround(acc * s_out)), adds the bias and applies ReLU / SiLU before the
//     only store of the output.
// GEMV (M <= 16): HBM-bound on B.  A workgroup of 4 waves owns 4*R rows of
//   B; the int8 activations are staged once per workgroup in LDS; each lane
//   streams 16-byte slices of R weight rows and accumulates with
//   v_dot4_i32_i8; a wave reduction finishes every (token, row) pair.
#include "q8_device.h"
#include "q8_internal.h"

namespace q8 {

// ------------------------------------------------------------------ epilogue
__device__ __forceinline__ float epi_value(int acc, int64_t m, int64_t n, const GemmEpi& e) {
  float y;
  if (e.mode == 0) {
    y = (float)((double)acc * e.s_out);
  } else {
    const float sv = (float)(e.sA[m * e.sA_stride] * e.sB[n * e.sB_stride]);
    y = (float)((double)acc * (double)sv);
  }
  if (e.bias) y = (float)((double)y + (double)e.bias[n]);
  if (e.act == 1) y = relu_js(y);
  else if (e.act == 2) y = silu_js(y);
  return y;
}

// Stores one 32x32 accumulator block of this lane: element r is row
// row0 + (r / 4) * 8 + (r % 4) of column `col`.  Kept out of line so the
// caller's loops over blocks unroll and index the accumulators statically.
__device__ __noinline__ void store_acc_block(v16i a, int64_t row0, int64_t col, int M, int N,
                                             const GemmEpi& e, void* out) {
  if (col >= N) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = row0 + (r >> 2) * 8 + (r & 3);
    if (row < M) {
      if (e.out_i32) static_cast<int32_t*>(out)[row * N + col] = a[r];
      else static_cast<float*>(out)[row * N + col] = epi_value(a[r], row, col, e);
    }
  }
}

// ------------------------------------------------------------------ MFMA GEMM
constexpr int BK = 128;

template <int BM, int BN, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N, 1)
void k_gemm_i8(const int8_t* __restrict__ A, const int8_t* __restrict__ B, int M, int N, int K,
               GemmEpi e, void* __restrict__ out) {
  constexpr int NT = 64 * WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_CH = BM * (BK / 16) / NT;   // 16-byte chunks per thread per step
  constexpr int B_CH = BN * (BK / 16) / NT;
  static_assert(A_CH * NT == BM * (BK / 16) && B_CH * NT == BN * (BK / 16), "tile / threads");
  constexpr int TILE_BYTES = (BM + BN) * BK;
  extern __shared__ __attribute__((aligned(16))) int8_t lds[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int wm = (wave / WAVES_N) * WM, wn = (wave % WAVES_N) * WN;

  v16i acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;

  v4i ra[A_CH], rb[B_CH];
  const int KT = (K + BK - 1) / BK;

  auto gload = [&](int kt) {
    const int kb = kt * BK;
#pragma unroll
    for (int c = 0; c < A_CH; ++c) {
      const int ch = tid + c * NT, row = ch >> 3, col = ch & 7;
      const int gm = m0 + row, gk = kb + col * 16;
      v4i v = {0, 0, 0, 0};
      if (gm < M && gk < K) v = *reinterpret_cast<const v4i*>(A + (int64_t)gm * K + gk);
      ra[c] = v;
    }
#pragma unroll
    for (int c = 0; c < B_CH; ++c) {
      const int ch = tid + c * NT, row = ch >> 3, col = ch & 7;
      const int gn = n0 + row, gk = kb + col * 16;
      v4i v = {0, 0, 0, 0};
      if (gn < N && gk < K) v = *reinterpret_cast<const v4i*>(B + (int64_t)gn * K + gk);
      rb[c] = v;
    }
  };
  auto lstore = [&](int buf) {
    int8_t* la = lds + buf * TILE_BYTES;
    int8_t* lb = la + BM * BK;
#pragma unroll
    for (int c = 0; c < A_CH; ++c) {
      const int ch = tid + c * NT, row = ch >> 3, col = ch & 7;
      *reinterpret_cast<v4i*>(la + row * BK + ((col ^ (row & 7)) << 4)) = ra[c];
    }
#pragma unroll
    for (int c = 0; c < B_CH; ++c) {
      const int ch = tid + c * NT, row = ch >> 3, col = ch & 7;
      *reinterpret_cast<v4i*>(lb + row * BK + ((col ^ (row & 7)) << 4)) = rb[c];
    }
  };

  gload(0);
  lstore(0);
  __syncthreads();

  const int r32 = lane & 31, khalf = lane >> 5;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) gload(kt + 1);
    const int8_t* la = lds + cur * TILE_BYTES;
    const int8_t* lb = la + BM * BK;
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      const int chunk = kk * 2 + khalf;
      const int sw = ((chunk ^ (r32 & 7)) << 4);
      v4i af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const v4i*>(la + (wm + i * 32 + r32) * BK + sw);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bf[j] = *reinterpret_cast<const v4i*>(lb + (wn + j * 32 + r32) * BK + sw);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) lstore(cur ^ 1);
    __syncthreads();
  }

  // 32x32 accumulator layout: lane l, element r holds
  //   row = (r / 4) * 8 + (l / 32) * 4 + (r % 4), col = l % 32.
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      store_acc_block(acc[i][j], m0 + wm + i * 32 + khalf * 4, n0 + wn + j * 32 + r32, M, N, e, out);
}

constexpr int gemm_lds_bytes(int bm, int bn) { return 2 * (bm + bn) * BK; }

// Generic fallback for K % 16 != 0 or unaligned operands: one thread per
// output, byte loads, exact int32 (wrapping) accumulation.
__global__ __launch_bounds__(256) void k_gemm_i8_generic(const int8_t* __restrict__ A,
                                                         const int8_t* __restrict__ B, int M, int N,
                                                         int K, GemmEpi e, void* __restrict__ out) {
  const int64_t idx = blockIdx.x * 256LL + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int64_t m = idx / N, n = idx % N;
  uint32_t s = 0;
  for (int k = 0; k < K; ++k) s += (uint32_t)((int)A[m * K + k] * (int)B[n * K + k]);
  const int acc = (int)s;
  if (e.out_i32) static_cast<int32_t*>(out)[idx] = acc;
  else static_cast<float*>(out)[idx] = epi_value(acc, m, n, e);
}

hipError_t setup_kernel_attributes();

hipError_t launch_gemm(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                       const GemmEpi& e, void* out, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  const bool vec = (K % 16 == 0) && ((reinterpret_cast<uintptr_t>(A) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(B) & 15) == 0);
  if (!vec) {
    const int64_t n = M * N;
    hipLaunchKernelGGL(k_gemm_i8_generic, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       A, B, (int)M, (int)N, (int)K, e, out);
    return hipGetLastError();
  }
  const int64_t tiles256 = ((M + 255) / 256) * ((N + 255) / 256);
  const int64_t tiles128 = ((M + 127) / 128) * ((N + 127) / 128);
  if (tiles256 >= 192) {
    dim3 grid((unsigned)((N + 255) / 256), (unsigned)((M + 255) / 256));
    k_gemm_i8<256, 256, 2, 2><<<grid, dim3(256), gemm_lds_bytes(256, 256), st>>>(
        A, B, (int)M, (int)N, (int)K, e, out);
  } else if (tiles128 >= 192) {
    dim3 grid((unsigned)((N + 127) / 128), (unsigned)((M + 127) / 128));
    k_gemm_i8<128, 128, 2, 2><<<grid, dim3(256), gemm_lds_bytes(128, 128), st>>>(
        A, B, (int)M, (int)N, (int)K, e, out);
  } else {
    dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    k_gemm_i8<64, 64, 2, 2><<<grid, dim3(256), gemm_lds_bytes(64, 64), st>>>(
        A, B, (int)M, (int)N, (int)K, e, out);
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------ GEMV (M <= 16)
constexpr int GEMV_KC = 4096;    // K bytes staged per pass
constexpr int GEMV_R = 4;        // weight rows per wave

template <int MT>
__global__ __launch_bounds__(256)
void k_gemv_i8(const int8_t* __restrict__ A, const int8_t* __restrict__ B, int M, int N, int K,
               GemmEpi e, void* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) int8_t xs[];   // [MT][GEMV_KC]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t nb = (int64_t)blockIdx.x * (4 * GEMV_R) + wave * GEMV_R;

  int acc[MT][GEMV_R];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < GEMV_R; ++r) acc[m][r] = 0;

  for (int k0 = 0; k0 < K; k0 += GEMV_KC) {
    const int kc = (K - k0) < GEMV_KC ? (K - k0) : GEMV_KC;
    const int cpr = kc >> 4;                       // 16-byte chunks per token row
    __syncthreads();                               // previous pass done with xs
    for (int c = tid; c < MT * cpr; c += 256) {
      const int m = c / cpr, off = (c - m * cpr) << 4;
      v4i v = {0, 0, 0, 0};
      if (m < M) v = *reinterpret_cast<const v4i*>(A + (int64_t)m * K + k0 + off);
      *reinterpret_cast<v4i*>(xs + m * GEMV_KC + off) = v;
    }
    __syncthreads();
    for (int j = 0; j * 1024 < kc; ++j) {
      const int kb = j * 1024 + lane * 16;
      if (kb < kc) {
        v4i w[GEMV_R];
#pragma unroll
        for (int r = 0; r < GEMV_R; ++r) {
          v4i v = {0, 0, 0, 0};
          if (nb + r < N) v = *reinterpret_cast<const v4i*>(B + (nb + r) * (int64_t)K + k0 + kb);
          w[r] = v;
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const v4i xv = *reinterpret_cast<const v4i*>(xs + m * GEMV_KC + kb);
#pragma unroll
          for (int r = 0; r < GEMV_R; ++r) {
            int a = acc[m][r];
            a = __builtin_amdgcn_sdot4(xv.x, w[r].x, a, false);
            a = __builtin_amdgcn_sdot4(xv.y, w[r].y, a, false);
            a = __builtin_amdgcn_sdot4(xv.z, w[r].z, a, false);
            a = __builtin_amdgcn_sdot4(xv.w, w[r].w, a, false);
            acc[m][r] = a;
          }
        }
      }
    }
  }

#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int r = 0; r < GEMV_R; ++r) {
      const int s = wave_sum_i32(acc[m][r]);
      const int64_t n = nb + r;
      if (lane == ((m * GEMV_R + r) & 63) && m < M && n < N) {
        if (e.out_i32) static_cast<int32_t*>(out)[(int64_t)m * N + n] = s;
        else static_cast<float*>(out)[(int64_t)m * N + n] = epi_value(s, m, n, e);
      }
    }
}

hipError_t launch_gemv(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                       const GemmEpi& e, void* out, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  const bool vec = (K % 16 == 0) && ((reinterpret_cast<uintptr_t>(A) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(B) & 15) == 0);
  if (!vec) return launch_gemm(A, B, M, N, K, e, out, st);   // generic path handles it
  const dim3 grid((unsigned)((N + 4 * GEMV_R - 1) / (4 * GEMV_R)));
  const dim3 block(256);
  if (M <= 1)
    hipLaunchKernelGGL(k_gemv_i8<1>, grid, block, 1 * GEMV_KC, st, A, B, (int)M, (int)N, (int)K, e, out);
  else if (M <= 2)
    hipLaunchKernelGGL(k_gemv_i8<2>, grid, block, 2 * GEMV_KC, st, A, B, (int)M, (int)N, (int)K, e, out);
  else if (M <= 4)
    hipLaunchKernelGGL(k_gemv_i8<4>, grid, block, 4 * GEMV_KC, st, A, B, (int)M, (int)N, (int)K, e, out);
  else if (M <= 8)
    hipLaunchKernelGGL(k_gemv_i8<8>, grid, block, 8 * GEMV_KC, st, A, B, (int)M, (int)N, (int)K, e, out);
  else
    hipLaunchKernelGGL(k_gemv_i8<16>, grid, block, 16 * GEMV_KC, st, A, B, (int)M, (int)N, (int)K, e, out);
  return hipGetLastError();
}

hipError_t setup_kernel_attributes() {
  hipError_t err;
#define Q8_SET_LDS(kern, bytes)                                                              \
  err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),                             \
                            hipFuncAttributeMaxDynamicSharedMemorySize, (bytes));            \
  if (err != hipSuccess) return err;
  Q8_SET_LDS((k_gemm_i8<256, 256, 2, 2>), gemm_lds_bytes(256, 256));
  Q8_SET_LDS((k_gemm_i8<128, 128, 2, 2>), gemm_lds_bytes(128, 128));
  Q8_SET_LDS((k_gemm_i8<64, 64, 2, 2>), gemm_lds_bytes(64, 64));
  Q8_SET_LDS(k_gemv_i8<1>, 1 * GEMV_KC);
  Q8_SET_LDS(k_gemv_i8<2>, 2 * GEMV_KC);
  Q8_SET_LDS(k_gemv_i8<4>, 4 * GEMV_KC);
  Q8_SET_LDS(k_gemv_i8<8>, 8 * GEMV_KC);
  Q8_SET_LDS(k_gemv_i8<16>, 16 * GEMV_KC);
#undef Q8_SET_LDS
  return hipSuccess;
}

}  // namespace q8
