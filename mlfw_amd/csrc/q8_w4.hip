// q8_w4.hip -- 4-bit per-group weights for gfx950: packing and the W4A8 GEMV.
//
// Weights: fromConstantArrayPerGroup + quantizeArrayPerGroup
// (src/compiler/ir/graph/quantization_types.ts:319-340, :143-153) over the
// flat [N, K] array with K % group == 0, so every group is a run of `group`
// elements of one row: scale s = absmax / 7 || 1e-10 (f64), code
// q = max(-8, min(7, Math.round(w / s))) (f64, no fround), two codes per
// byte (element 2j in the low nibble, two's complement); scales [N * G],
// G = K / group.
//
// W4A8 GEMV (the reference has no such op; this composition keeps it exact):
//   acc_g = sum over the group of xq[m,k] * q[n,k]             exact int32
//   S     = acc_0*sw_0 + acc_1*sw_1 + ...                       f64, ascending g
//   y     = fround(S * sx[m]), bias fround(y + b[n]), ReLU / SiLU
// Fast kernel (M <= 4, power-of-two group 32..2048, K <= 8192): a row's
// 16-byte chunks of packed codes (32 elements each) sit on consecutive
// lanes, and every lane keeps one chunk's activations for all the rows its
// workgroup visits.  Nibbles become dot4 operands without sign extension: the
// byte (nibble ^ 8) is q + 8 in [0, 15], so
//   dot4(x, q + 8) = dot4(x, q) + 8 * sum(x)
// and the 8 * sum(x) of each chunk is subtracted once; the activation bytes
// are regrouped into even / odd elements once per workgroup (v_perm).  The
// lanes of one group are reduced by shuffles; the group's leader lane,
// which loaded that group's scale together with the weights, writes
// acc_g * sw_g (f64) to LDS, and one lane per (row, token) adds the groups
// in order from LDS.  HBM-bound on the K / 2 bytes per row: half the int8
// weight traffic.
// Generic kernel (any M, any group dividing K): one thread per output.
#include <algorithm>

#include "q8_device.h"
#include "q8_internal.h"

namespace q8 {

__device__ __forceinline__ __amdgpu_buffer_rsrc_t w4_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Math.max(-8, Math.min(7, Math.round(w / s))) stored to an Int8Array
// (NaN -> 0; Math.round ties toward +inf).
__device__ __forceinline__ int w4_code(float w, double s) {
  const double y = (double)w / s;
  if (y != y) return 0;
  const double f = floor(y);
  double r = (y - f >= 0.5) ? f + 1.0 : f;
  r = r < -8.0 ? -8.0 : (r > 7.0 ? 7.0 : r);
  return (int)r;
}

// One thread per group: absmax, scale, then codes (two per byte).
__global__ __launch_bounds__(256) void k_pack_w4(const float* __restrict__ W, int64_t total,
                                                 int64_t group, uint8_t* __restrict__ wq,
                                                 double* __restrict__ scales) {
  const int64_t g = blockIdx.x * 256LL + threadIdx.x;
  const int64_t ngroups = total / group;
  if (g >= ngroups) return;
  const float* w = W + g * group;
  double amax = 0.0;
  for (int64_t i = 0; i < group; ++i) {
    const double a = fabs((double)w[i]);
    if (a > amax) amax = a;                      // NaN never compares greater
  }
  double s = amax / 7.0;
  if (s == 0.0 || s != s) s = 1e-10;
  scales[g] = s;
  uint8_t* out = wq + (g * group) / 2;
  for (int64_t i = 0; i < group; i += 2)
    out[i / 2] = (uint8_t)((w4_code(w[i], s) & 0xF) | ((w4_code(w[i + 1], s) & 0xF) << 4));
}

// Activation chunk (32 bytes) -> even / odd element dwords and 8 * sum.
struct XChunk {
  int e[4], o[4];
  int corr;
};

// Lane i += lane i + SH of its row of 16 (0 past the row's end).
template <int SH>
__device__ __forceinline__ int w4_row_shl(int v) {
  return __builtin_amdgcn_update_dpp(0, v, 0x100 + SH, 0xF, 0xF, true);
}

// Workgroup barrier that waits for this wave's LDS operations only: the
// prefetched weights stay in flight (__syncthreads would also wait for
// every outstanding global load).
__device__ __forceinline__ void w4_lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A block of rows is P passes of RPP rows: a row's K / 32 chunks (NCP =
// that count rounded up to a power of two, <= 256) map to consecutive
// lanes, and every lane keeps the same chunk -- one load of its activations
// serves every row the workgroup visits.  A workgroup does blocks
// blockIdx.x and blockIdx.x + gridDim.x (when it exists): every load of
// both is issued before any arithmetic, and the f64 products of the two go
// to two LDS buffers, so one barrier per block suffices.  A buffer is
// [G][pitch] (pitch = ROWS * MT + 1 doubles): the lane summing output o
// reads column o, so a wave's reads are consecutive.
template <int MT, int P>
__global__ __launch_bounds__(256) void k_gemv_w4(const int8_t* __restrict__ xq,
                                                 const double* __restrict__ sx, int sx_stride,
                                                 const uint8_t* __restrict__ wq4,
                                                 const double* __restrict__ sw, int M, int N, int K,
                                                 int ncp_log2, int rpp_log2, int lpg_log2,
                                                 const float* __restrict__ bias, int act,
                                                 float* __restrict__ y) {
  extern __shared__ double tg[];
  const int tid = threadIdx.x;
  const uint32_t KB = (uint32_t)K >> 1;           // packed bytes per row
  const int nch = K >> 5;                         // 32-element chunks per row
  const int G = K >> (lpg_log2 + 5);              // groups per row
  const int RPP = 1 << rpp_log2;                  // rows per pass
  const int ROWS = P * RPP;                       // rows per block
  const int NO = ROWS * MT;                       // outputs per block (<= 256)
  const int pitch = NO + 1;
  const int nblk = (N + ROWS - 1) / ROWS;
  const int c = tid & ((1 << ncp_log2) - 1);      // this lane's chunk
  const int rsub = tid >> ncp_log2;               // row within a pass
  const bool live_c = c < nch && rsub < RPP;
  const bool leader = (c & ((1 << lpg_log2) - 1)) == 0;
  const uint32_t cg = (uint32_t)c >> lpg_log2;    // this lane's group

  const __amdgpu_buffer_rsrc_t rw = w4_rsrc(wq4, (uint32_t)N * KB);
  const __amdgpu_buffer_rsrc_t rs = w4_rsrc(sw, (uint32_t)N * (uint32_t)G * 8u);
  // weight chunks and (leader lanes) group scales of block b.  A dead lane
  // reads row N, past the end of both buffers, which loads zero (selecting
  // the row, not the offset, keeps the select a v_cndmask).
  auto load_block = [&](int b, v4i* wo, double* so) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int row = b * ROWS + p * RPP + rsub;
      const bool live = row < N && live_c;
      const uint32_t rw_row = live ? (uint32_t)row : (uint32_t)N;
      const uint32_t rs_row = (live && leader) ? (uint32_t)row : (uint32_t)N;
      wo[p] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                          rw, rw_row * KB + 16u * (uint32_t)c, 0, 0));
      so[p] = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(
                                             rs, (rs_row * (uint32_t)G + cg) * 8u, 0, 0));
    }
  };
  // bias of the output this lane finishes in block b (no bias: an empty
  // buffer, every load reads zero)
  const __amdgpu_buffer_rsrc_t rb = w4_rsrc(bias, bias ? (uint32_t)N * 4u : 0u);
  auto load_bias = [&](int b) -> float {
    const int n = b * ROWS + tid / MT;
    const uint32_t nb = (tid < NO && n < N) ? (uint32_t)n : (uint32_t)N;
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, nb * 4u, 0, 0));
  };

  // this lane's activation chunk for every token, loaded once and first
  // (vector loads complete in order: waiting for these does not wait for
  // the weights)
  const __amdgpu_buffer_rsrc_t rx = w4_rsrc(xq, (uint32_t)M * (uint32_t)K);
  v4i xa[MT][2];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const uint32_t xm = (m < M && live_c) ? (uint32_t)m : (uint32_t)M;   // token M: past the end
    const uint32_t off = xm * (uint32_t)K + 32u * (uint32_t)c;
    xa[m][0] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
    xa[m][1] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, off + 16u, 0, 0));
  }
  // the token scale of the output this lane finishes (the same token in
  // both blocks), before the weights so that waiting for it does not wait
  // for them; one value per lane, not an array indexed by token, which the
  // compiler would keep in scratch memory
  const int om = tid % MT;
  const double sxm = (tid < NO && om < M) ? sx[(int64_t)om * sx_stride] : 0.0;
  // the first two blocks of weights.  Every load is issued on every path
  // (a block past the end reads zero without touching memory), so the
  // loads in flight are the same at every wait.  The bias, needed last,
  // follows each block's weights.
  const int gs = gridDim.x;
  v4i wa[P], wb[P];
  double sa[P], sb[P];
  load_block(blockIdx.x, wa, sa);
  const float ba = load_bias(blockIdx.x);
  load_block(blockIdx.x + gs, wb, sb);
  const float bb = load_bias(blockIdx.x + gs);
  // nothing below may be scheduled above the loads
  __builtin_amdgcn_sched_barrier(0);
  XChunk xc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    const v4i a0 = xa[m][0], a1 = xa[m][1];
    const int a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    int sum = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      xc[m].e[d] = (int)__builtin_amdgcn_perm((unsigned)a[2 * d + 1], (unsigned)a[2 * d], 0x06040200u);
      xc[m].o[d] = (int)__builtin_amdgcn_perm((unsigned)a[2 * d + 1], (unsigned)a[2 * d], 0x07050301u);
      sum = __builtin_amdgcn_sdot4(a[2 * d], 0x01010101, sum, false);
      sum = __builtin_amdgcn_sdot4(a[2 * d + 1], 0x01010101, sum, false);
    }
    xc[m].corr = 8 * sum;
  }

  // products of block b into t0, barrier, then the ordered sums
  auto run_block = [&](int b, const v4i* w, const double* swv, float bv, double* t0) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      int acc[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[m] = -xc[m].corr;
      const int wd[4] = {w[p].x, w[p].y, w[p].z, w[p].w};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int lo = (wd[d] & 0x0F0F0F0F) ^ 0x08080808;          // even elements, q + 8
        const int hi = ((wd[d] >> 4) & 0x0F0F0F0F) ^ 0x08080808;   // odd elements, q + 8
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          acc[m] = __builtin_amdgcn_sdot4(xc[m].e[d], lo, acc[m], false);
          acc[m] = __builtin_amdgcn_sdot4(xc[m].o[d], hi, acc[m], false);
        }
      }
      // the group's sum lands on its first lane (groups are aligned runs
      // of 2^lpg_log2 lanes of one row)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        int v = acc[m];
        if (lpg_log2 >= 1) v += w4_row_shl<1>(v);
        if (lpg_log2 >= 2) v += w4_row_shl<2>(v);
        if (lpg_log2 >= 3) v += w4_row_shl<4>(v);
        if (lpg_log2 >= 4) v += w4_row_shl<8>(v);
        if (lpg_log2 >= 5) v += __shfl_down(v, 16, 64);
        if (lpg_log2 >= 6) v += __shfl_down(v, 32, 64);
        acc[m] = v;
      }
      // products on every lane (the wait for the scales stays outside the
      // branch), stored by the leaders
      double prod[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) prod[m] = (double)acc[m] * swv[p];
      if (leader && live_c) {
        const int o = (p * RPP + rsub) * MT;
#pragma unroll
        for (int m = 0; m < MT; ++m) t0[(int)cg * pitch + o + m] = prod[m];
      }
    }
    w4_lds_barrier();
    // one lane per (row, token): the f64 sum over groups in ascending order
    if (tid < NO) {
      const int m = tid % MT, n = b * ROWS + tid / MT;
      if (m < M && n < N) {
        // -0.0 is the exact identity of IEEE addition: S starts as t[0]
        const double* t = t0 + tid;
        double S = -0.0;
        int g = 0;
        for (; g + 8 <= G; g += 8) {
          double v[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = t[(g + j) * pitch];
#pragma unroll
          for (int j = 0; j < 8; ++j) S = S + v[j];
        }
        for (; g < G; ++g) S = S + t[g * pitch];
        float v = (float)(S * sxm);
        if (bias) v = v + bv;
        if (act == 1) v = relu_js(v);
        else if (act == 2) v = silu_js(v);
        y[(int64_t)m * N + n] = v;
      }
    }
  };

  run_block(blockIdx.x, wa, sa, ba, tg);
  if (blockIdx.x + gs < nblk)                     // uniform
    run_block(blockIdx.x + gs, wb, sb, bb, tg + G * pitch);
}

// ---- MFMA W4A8 GEMV, 2 <= M <= 16 tokens.  One v_mfma_i32_16x16x32_i8 per
// 16 weight rows x 32 K elements x all 16 token columns: lane l holds row
// (resp. token) l % 16 and 8 of the 32 elements, in A and B alike (the
// order of K inside an instruction is free as long as both operands use
// the same one).  The 4 packed weight bytes of a lane become two dot
// operands without sign extension -- the low nibbles (elements 0, 2, 4, 6)
// and the high ones (1, 3, 5, 7), each `(n ^ 8)` = q + 8 -- and the
// activations are regrouped into the same even / odd order (v_perm); a
// second MFMA with the constant -8 as A adds -8 * sum(x) to the same
// accumulator, so it holds sum x * q exactly.
//
// A step of a wave covers SPAN = 32 (narrow) or 128 (WIDE, groups of a
// multiple of 128) elements: in the wide form lane (r, q) loads 16 packed
// bytes (32 elements) of row r and the 32 matching activation bytes of
// token r, and runs four MFMA pairs on them.  The workgroup's 4 waves take
// quarters of K (whole groups); at the end of each group a wave writes its
// int32 accumulators to LDS [group][output], then one lane per output adds
// acc_g * sw_g (f64) over the groups in order.  All of a wave's weight and
// activation loads are issued before its first MFMA.
__device__ __forceinline__ v4i w4_mma8(int w, int x0, int x1, v4i acc) {
  const long minus8 = (long)0xF8F8F8F8F8F8F8F8ull;
  const int lo = (w & 0x0F0F0F0F) ^ 0x08080808;         // elements 0,2,4,6 of 8: q + 8
  const int hi = ((w >> 4) & 0x0F0F0F0F) ^ 0x08080808;  // elements 1,3,5,7
  const long a = (long)(uint32_t)lo | ((long)(uint32_t)hi << 32);
  const int xe = (int)__builtin_amdgcn_perm((unsigned)x1, (unsigned)x0, 0x06040200u);
  const int xo = (int)__builtin_amdgcn_perm((unsigned)x1, (unsigned)x0, 0x07050301u);
  const long b = (long)(uint32_t)xe | ((long)(uint32_t)xo << 32);
  acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(minus8, b, acc, 0, 0, 0);
}

template <int STEPS, bool WIDE>
__global__ __launch_bounds__(256) void k_gemv_w4_mfma(const int8_t* __restrict__ xq,
                                                      const double* __restrict__ sx, int sx_stride,
                                                      const uint8_t* __restrict__ wq4,
                                                      const double* __restrict__ sw, int M, int N,
                                                      int K, int group,
                                                      const float* __restrict__ bias, int act,
                                                      float* __restrict__ y) {
  constexpr int SPAN = WIDE ? 128 : 32;                 // elements per wave step
  constexpr int LANE = SPAN / 4;                        // elements per lane and step
  extern __shared__ double lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int G = K / group, KB = K >> 1;
  const int NO = 16 * M;                                // outputs of the workgroup
  double* sc = lds;                                     // [16][G] group scales
  int* accs = reinterpret_cast<int*>(lds + 16 * G);     // [G][NO] group sums

  const int steps = (K >> 2) / SPAN;                    // steps per wave (<= STEPS)
  const int kbase = wave * (K >> 2);
  const uint32_t rows = (uint32_t)min(16, N - n0);
  const __amdgpu_buffer_rsrc_t rw = w4_rsrc(wq4 + (int64_t)n0 * KB, rows * (uint32_t)KB);
  const __amdgpu_buffer_rsrc_t rx = w4_rsrc(xq, (uint32_t)M * (uint32_t)K);
  // lane's weight row r16 (past the last row: offset past the end) and
  // token r16 (>= M: past the end): both read zero
  const uint32_t wrow = (uint32_t)r16 < rows ? (uint32_t)r16 : rows;
  const uint32_t xtok = r16 < M ? (uint32_t)r16 : (uint32_t)M;
  v4i wv[WIDE ? STEPS : 1];
  v4i xv[WIDE ? 2 * STEPS : 1];
  int wn[WIDE ? 1 : STEPS];
  v2i xn[WIDE ? 1 : STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const uint32_t k = (uint32_t)(kbase + SPAN * (s < steps ? s : 0) + LANE * q);
    const uint32_t wo = wrow * (uint32_t)KB + k / 2, xo = xtok * (uint32_t)K + k;
    if constexpr (WIDE) {
      wv[s] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, wo, 0, 2));
      xv[2 * s] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0));
      xv[2 * s + 1] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16, 0, 0));
    } else {
      wn[s] = __builtin_bit_cast(int, __builtin_amdgcn_raw_buffer_load_b32(rw, wo, 0, 2));
      xn[s] = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rx, xo, 0, 0));
    }
  }
  // group scales of the workgroup's 16 rows
  for (int i = tid; i < 16 * G; i += 256) {
    const int r = i / G, g = i - r * G;
    sc[i] = n0 + r < N ? sw[(int64_t)(n0 + r) * G + g] : 0.0;
  }
  // this lane's output: (row o / M, token o % M)
  const int o = tid, orow = o / M, otok = o - orow * M;
  const bool out_lane = o < NO && n0 + orow < N;
  const double sxo = out_lane ? sx[(int64_t)otok * sx_stride] : 0.0;
  const float bo = (out_lane && bias) ? bias[n0 + orow] : 0.0f;
  __builtin_amdgcn_sched_barrier(0);

  const int gsteps = group / SPAN;                      // steps per group
  int g = kbase / group, left = 0;                      // the wave starts on a group boundary
  v4i acc = {0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    if (s < steps) {                                    // uniform
      if (left == 0) {                                  // a group starts
        acc = v4i{0, 0, 0, 0};
        left = gsteps;
      }
      if constexpr (WIDE) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc = w4_mma8(wv[s][j], xv[2 * s + j / 2][2 * (j & 1)], xv[2 * s + j / 2][2 * (j & 1) + 1], acc);
      } else {
        acc = w4_mma8(wn[s], xn[s].x, xn[s].y, acc);
      }
      if (--left == 0) {                                // a group ends: D[4q + r][r16]
        if (r16 < M) {
#pragma unroll
          for (int r = 0; r < 4; ++r) accs[g * NO + (4 * q + r) * M + r16] = acc[r];
        }
        ++g;
      }
    }
  }
  __syncthreads();
  if (out_lane) {
    double S = -0.0;                                    // -0.0 + t = t exactly
    for (int gi = 0; gi < G; ++gi) S = S + (double)accs[gi * NO + o] * sc[orow * G + gi];
    float v = (float)(S * sxo);
    if (bias) v = v + bo;
    if (act == 1) v = relu_js(v);
    else if (act == 2) v = silu_js(v);
    y[(int64_t)otok * N + n0 + orow] = v;
  }
}

bool gemv_w4_mfma_ok(int64_t M, int64_t K, int64_t group) {
  if (M < 2 || M > 16 || K % 128 != 0 || K > 4096 || group % 32 != 0 || K % group != 0) return false;
  const int64_t G = K / group;
  if ((K / 4) % group != 0) return false;               // whole groups per wave
  return (size_t)16 * G * 8 + (size_t)G * 16 * M * 4 <= 65536;
}

__global__ __launch_bounds__(256) void k_gemv_w4_generic(const int8_t* __restrict__ xq,
                                                         const double* __restrict__ sx,
                                                         int sx_stride,
                                                         const uint8_t* __restrict__ wq4,
                                                         const double* __restrict__ sw, int64_t M,
                                                         int64_t N, int64_t K, int64_t group,
                                                         const float* __restrict__ bias, int act,
                                                         float* __restrict__ y) {
  const int64_t idx = blockIdx.x * 256LL + threadIdx.x;
  if (idx >= M * N) return;
  const int64_t m = idx / N, n = idx % N;
  const int64_t G = K / group, KB = (K + 1) / 2;
  double S = 0.0;
  for (int64_t g = 0; g < G; ++g) {
    int acc = 0;
    for (int64_t k = g * group; k < (g + 1) * group; ++k) {
      const int nib = (wq4[n * KB + (k >> 1)] >> (4 * (k & 1))) & 0xF;
      acc += (int)xq[m * K + k] * (nib >= 8 ? nib - 16 : nib);
    }
    const double t = (double)acc * sw[n * G + g];
    S = g == 0 ? t : S + t;
  }
  float v = (float)(S * sx[m * sx_stride]);
  if (bias) v = v + bias[n];
  if (act == 1) v = relu_js(v);
  else if (act == 2) v = silu_js(v);
  y[idx] = v;
}

hipError_t launch_pack_w4(const float* W, int64_t N, int64_t K, int64_t group, uint8_t* wq4,
                          double* scales, hipStream_t st) {
  const int64_t ngroups = N * K / group;
  if (ngroups == 0) return hipSuccess;
  hipLaunchKernelGGL(k_pack_w4, dim3((unsigned)((ngroups + 255) / 256)), dim3(256), 0, st, W,
                     N * K, group, wq4, scales);
  return hipGetLastError();
}

constexpr int W4_P = 4;                          // passes per block

namespace {
int ilog2_ceil(int64_t v) {
  int l = 0;
  while ((int64_t(1) << l) < v) ++l;
  return l;
}

struct W4Plan {
  int mt, ncp_log2, rpp_log2, lpg_log2;
  size_t lds;
  int64_t rows;
};

// Block shape of the fast kernel: outputs per block (ROWS x MT) <= 256,
// two LDS buffers of G x (ROWS x MT + 1) doubles within 64 KiB.
bool w4_plan(int64_t M, int64_t K, int64_t group, W4Plan* pl) {
  const bool pow2 = group >= 32 && group <= 2048 && (group & (group - 1)) == 0;
  if (!(M >= 1 && M <= 4 && pow2 && K % group == 0 && K <= 8192)) return false;
  pl->mt = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
  pl->ncp_log2 = ilog2_ceil(K / 32);
  pl->lpg_log2 = ilog2_ceil(group / 32);
  pl->rpp_log2 = std::min(8 - pl->ncp_log2, ilog2_ceil(256 / (W4_P * pl->mt)));
  pl->rows = (int64_t)W4_P << pl->rpp_log2;
  const int64_t G = K / group;
  pl->lds = 2 * (size_t)G * (size_t)(pl->rows * pl->mt + 1) * sizeof(double);
  return pl->lds <= 65536;
}
}  // namespace

bool gemv_w4_fast_ok(int64_t M, int64_t K, int64_t group) {
  W4Plan pl;
  return w4_plan(M, K, group, &pl);
}

hipError_t launch_gemv_w4(const int8_t* xq, const double* sx, int sx_stride, const uint8_t* wq4,
                          const double* sw, int64_t M, int64_t N, int64_t K, int64_t group,
                          const float* bias, int act, float* y, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  W4Plan pl;
  const bool dot4 = w4_plan(M, K, group, &pl);
  // the MFMA kernel from 3 tokens on with 16-byte weight loads (groups of a
  // multiple of 128); dot4 below that, or where the MFMA kernel does not apply
  if (gemv_w4_mfma_ok(M, K, group) && (!dot4 || (M >= 3 && group % 128 == 0))) {
    const int64_t G = K / group;
    const size_t lds = (size_t)16 * G * 8 + (size_t)G * 16 * M * 4;
    const dim3 grid((unsigned)((N + 15) / 16)), block(256);
#define Q8_W4M(ST, WD)                                                                          \
  hipLaunchKernelGGL((k_gemv_w4_mfma<ST, WD>), grid, block, lds, st, xq, sx, sx_stride, wq4, sw, \
                     (int)M, (int)N, (int)K, (int)group, bias, act, y)
    if (group % 128 == 0) {                             // 16-byte weight loads
      const int steps = (int)(K >> 9);
      if (steps <= 4) Q8_W4M(4, true);
      else Q8_W4M(8, true);
    } else {
      const int steps = (int)(K >> 7);
      if (steps <= 8) Q8_W4M(8, false);
      else if (steps <= 16) Q8_W4M(16, false);
      else Q8_W4M(32, false);
    }
#undef Q8_W4M
    return hipGetLastError();
  }
  if (!dot4) {
    hipLaunchKernelGGL(k_gemv_w4_generic, dim3((unsigned)((M * N + 255) / 256)), dim3(256), 0, st,
                       xq, sx, sx_stride, wq4, sw, M, N, K, group, bias, act, y);
    return hipGetLastError();
  }
  // one block per workgroup while they all fit at once (4 resident
  // workgroups per CU), else two
  const int64_t nblk = (N + pl.rows - 1) / pl.rows, slots = 4 * (int64_t)cu_count();
  const dim3 grid((unsigned)(nblk <= slots ? nblk : (nblk + 1) / 2)), block(256);
#define Q8_W4(MT)                                                                                \
  hipLaunchKernelGGL((k_gemv_w4<MT, W4_P>), grid, block, pl.lds, st, xq, sx, sx_stride, wq4, sw, \
                     (int)M, (int)N, (int)K, pl.ncp_log2, pl.rpp_log2, pl.lpg_log2, bias, act, y)
  if (pl.mt == 1) Q8_W4(1);
  else if (pl.mt == 2) Q8_W4(2);
  else Q8_W4(4);
#undef Q8_W4
  return hipGetLastError();
}

}  // namespace q8
