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

// A team of L lanes per group (L = the largest power of two <= 64 that
// divides group / 2, teams aligned within the wave): lane j of the team
// takes the code pairs j, j + L, j + 2L, ... so the team's loads and byte
// stores are contiguous; the absmax is combined across the team by xor
// shuffles (NaN never compares greater, so it never becomes the max), then
// every lane rounds its own pairs.
__global__ __launch_bounds__(256) void k_pack_w4(const float* __restrict__ W, int64_t total,
                                                 int64_t group, int L, uint8_t* __restrict__ wq,
                                                 double* __restrict__ scales) {
  const int64_t t = blockIdx.x * 256LL + threadIdx.x;
  const int64_t ngroups = total / group;
  const int64_t g = t / L;
  const int j = (int)(t - g * L);
  const bool live = g < ngroups;                 // dead lanes still join the shuffles
  const int64_t pairs = group / 2;
  const float* w = W + (live ? g : 0) * group;   // 4-byte aligned only: two dword loads per pair
  double amax = 0.0;
  if (live) {
    for (int64_t p = j; p < pairs; p += L) {
      const double a = fabs((double)w[2 * p]), b = fabs((double)w[2 * p + 1]);
      if (a > amax) amax = a;
      if (b > amax) amax = b;
    }
  }
  for (int o = L >> 1; o >= 1; o >>= 1) {
    const double other = __shfl_xor(amax, o, 64);
    if (other > amax) amax = other;
  }
  if (!live) return;
  double s = amax / 7.0;
  if (s == 0.0 || s != s) s = 1e-10;
  if (j == 0) scales[g] = s;
  uint8_t* out = wq + g * pairs;
  for (int64_t p = j; p < pairs; p += L)
    out[p] = (uint8_t)((w4_code(w[2 * p], s) & 0xF) | ((w4_code(w[2 * p + 1], s) & 0xF) << 4));
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

// 16 bytes per lane from buffer offset voff to LDS dst + 16 * lane.
__device__ __forceinline__ void w4_copy16_to_lds(__amdgpu_buffer_rsrc_t r, int8_t* dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16, voff, 0, 0, 0);
}

// Slot of 16-byte unit u of staged row r (LPR units per row): a bijection
// of the row's units, chosen so that the 16 rows' reads of one unit fall in
// 16 different bank groups.
template <int LPR>
__device__ __forceinline__ int w4_slot(int u, int r) {
  return u ^ (LPR == 8 ? (r >> 1) & 7 : r & 15);
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
        for (; g + 16 <= G; g += 16) {                  // 16 products per LDS round trip
          double v[16];
#pragma unroll
          for (int j = 0; j < 16; ++j) v[j] = t[(g + j) * pitch];
#pragma unroll
          for (int j = 0; j < 16; ++j) S = S + v[j];
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

// ---- MFMA W4A8 GEMV: any M (blocks of 16 tokens), K a multiple of 32,
// groups of a multiple of 32.  One v_mfma_i32_16x16x32_i8 per 16 weight
// rows x 32 codes x 16 token columns: lane l holds row (resp. token) l % 16
// and 8 of the 32 codes, in A and B alike (the order of K inside an
// instruction is free as long as both operands use the same one).  The 4
// packed bytes of a lane become two dot operands without sign extension --
// the low nibbles (codes 0, 2, 4, 6) and the high ones (1, 3, 5, 7), each
// `(n ^ 8)` = q + 8 -- and the activations are regrouped into the same
// even / odd order (v_perm); a second MFMA with the constant -8 as A adds
// -8 * sum(x), so the accumulator holds sum x * q exactly.
//
// Loads: in a step of 128 codes, lane (r, q) of a wave reads the 16 packed
// bytes of chunk q (32 codes) of row r, so one instruction covers 64
// contiguous bytes of each of 16 rows, and lane (t, q) the 32 activation
// bytes of the same chunk of token t.  With groups of a multiple of 128
// codes the whole step lies in one group and MFMA j takes dword j (codes
// 8j..8j+7) of every lane's chunk.  Otherwise (TR) a 4 x 4 transpose of the
// dwords between the 4 lanes of a row (v_permlane32_swap, then
// v_permlane16_swap), of codes and activations alike, makes MFMA j consume
// chunk j whole, so no MFMA mixes two groups.
//
// K is walked in rounds: in round r, wave w of the workgroup's NW takes the
// span of PS codes at (NW r + w) * PS -- PS a multiple of the group, or a
// divisor of it, of at most 128 * RS codes (one round covers K = 4096 with
// groups of 128) -- and splits it into segments of SL = min(PS, group)
// codes.  Each segment's int32 sum (exact) goes to an LDS window
// [segment][token][row], with the scales of the groups that end in the
// round.  After one barrier, lane o = (token, row) walks the round's
// segments in order, adds the pieces of a group in int32 and, when the
// group is complete, adds acc_g * sw_g to its f64 sum -- groups in
// ascending order, as the definition asks.  With more than one round, LDS
// holds two windows used alternately, so one barrier per round suffices.
__device__ __forceinline__ v4i w4_mma8(int w, int x0, int x1, v4i acc) {
  const long minus8 = (long)0xF8F8F8F8F8F8F8F8ull;
  const int lo = (w & 0x0F0F0F0F) ^ 0x08080808;         // codes 0,2,4,6 of 8: q + 8
  const int hi = ((w >> 4) & 0x0F0F0F0F) ^ 0x08080808;  // codes 1,3,5,7
  const long a = (long)(uint32_t)lo | ((long)(uint32_t)hi << 32);
  const int xe = (int)__builtin_amdgcn_perm((unsigned)x1, (unsigned)x0, 0x06040200u);
  const int xo = (int)__builtin_amdgcn_perm((unsigned)x1, (unsigned)x0, 0x07050301u);
  const long b = (long)(uint32_t)xe | ((long)(uint32_t)xo << 32);
  acc = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_i32_16x16x32_i8(minus8, b, acc, 0, 0, 0);
}

// Register j of lane (r, q) <- dword q of lane (r, j)'s v[0..3].
__device__ __forceinline__ v4i w4_transpose4(v4i v) {
  const auto s02 = __builtin_amdgcn_permlane32_swap((unsigned)v[0], (unsigned)v[2], false, false);
  const auto s13 = __builtin_amdgcn_permlane32_swap((unsigned)v[1], (unsigned)v[3], false, false);
  const auto t01 = __builtin_amdgcn_permlane16_swap(s02[0], s13[0], false, false);
  const auto t23 = __builtin_amdgcn_permlane16_swap(s02[1], s13[1], false, false);
  return v4i{(int)t01[0], (int)t01[1], (int)t23[0], (int)t23[1]};
}

template <int NW, int RS, bool TR, bool ONE, bool XH>
__global__ __launch_bounds__(64 * NW) void k_gemv_w4_mfma(const int8_t* __restrict__ xq,
                                                          const double* __restrict__ sx,
                                                          int sx_stride,
                                                          const uint8_t* __restrict__ wq4,
                                                          const double* __restrict__ sw, int M,
                                                          int N, int K, int group, int PS,
                                                          int segw, int ng,
                                                          const float* __restrict__ bias, int act,
                                                          float* __restrict__ y) {
  constexpr int NT = 64 * NW;
  extern __shared__ double lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, q = lane >> 4;
  const int n0 = blockIdx.x * 16, t0 = blockIdx.y * 16;
  const int MB = min(16, M - t0);                       // tokens of this block
  const int NO = 16 * MB;                               // outputs: o = token * 16 + row
  const int G = K / group, KB = K >> 1;
  const int SL = min(PS, group);                        // segment length (codes)
  const int nseg = NW * segw;                           // segments per round
  const int ngp = ng | 1;                               // scale row pitch (doubles): odd, so
                                                        // the 16 rows' reads hit distinct banks
  const int win = nseg * NO + 2 * 16 * ngp;             // ints per LDS window: sums, then the
                                                        // scales of the <= ng groups that end
  const int RC = NW * PS;                               // codes per round
  const int rounds = (K + RC - 1) / RC;

  const uint32_t rows = (uint32_t)min(16, N - n0);
  const __amdgpu_buffer_rsrc_t rw = w4_rsrc(wq4 + (int64_t)n0 * KB, rows * (uint32_t)KB);
  const __amdgpu_buffer_rsrc_t rx = w4_rsrc(xq + (int64_t)t0 * K, (uint32_t)MB * (uint32_t)K);
  const __amdgpu_buffer_rsrc_t rs = w4_rsrc(sw + (int64_t)n0 * G, rows * (uint32_t)G * 8u);
  const uint32_t wrow = (uint32_t)r16 < rows ? (uint32_t)r16 : rows;    // past the end: zero
  // XH (at most 8 tokens): lane (t, q) loads half t >> 3 of token t & 7's
  // 32-byte chunk, and lanes t < 8 take the other half from lane t + 8 of
  // their row; B's columns 8..15 then hold data of no token and their
  // outputs are never stored
  const int xr = XH ? (r16 & 7) : r16;
  const uint32_t xtok = xr < MB ? (uint32_t)xr : (uint32_t)MB;

  // this lane's output
  const int o = tid, otok = o >> 4, orow = o & 15;
  const bool out_lane = o < NO && n0 + orow < N;
  const double sxo = out_lane ? sx[(int64_t)(t0 + otok) * sx_stride] : 0.0;
  const float bo = (out_lane && bias) ? bias[n0 + orow] : 0.0f;
  // scale slots u = tid + NT * u2 of a window: row u / ng, group u % ng
  constexpr int NSC = (16 * 64 + NT - 1) / NT;          // ng <= 64
  uint32_t sc_off[NSC];
  int sc_g[NSC], sc_w[NSC];
#pragma unroll
  for (int u2 = 0; u2 < NSC; ++u2) {
    const int u = tid + NT * u2, rr = u / ng;
    sc_g[u2] = u < 16 * ng ? u - rr * ng : G;          // G: past the end
    sc_w[u2] = rr * ngp + (u - rr * ng);                // LDS slot
    sc_off[u2] = (uint32_t)(rr < 16 ? rr : 16) * (uint32_t)G;
  }

  double S = -0.0;                                      // -0.0 + t = t exactly
  int gacc = 0, pieces = 0, gdone = 0;                  // groups split over spans
  const int P = group > PS ? group / PS : 1;            // spans per group
  int* const win0 = reinterpret_cast<int*>(lds);
  // Weight staging: each round, the wave copies its 16 rows x 64 RS packed
  // bytes (its span) into LDS after the windows with direct-to-LDS buffer
  // loads, RPC rows of LPR contiguous 16-byte units per instruction, and
  // reads its fragments back (unit u of row r in slot w4_slot(u, r)).
  // Loaded straight into the fragment layout, each instruction reads 64
  // bytes of each of 16 rows.  Units outside the span or K, and rows past
  // N, read zero.  Staged where the 32 KiB of copies keep the workgroups a
  // CU holds: 16 waves (one per CU), and 8 waves for up to 8 tokens (small
  // windows); for 16 tokens, and with 4 waves, they would cost a resident
  // workgroup per CU and run slower (N = 11008, M = 16: 12.6 -> 13.1 us).
  constexpr bool STAGE = NW == 16 || (NW == 8 && XH);
  constexpr int LPR = 4 * RS, RPC = 64 / LPR;
  const int nwin = (ONE || rounds == 1) ? 1 : 2;
  int8_t* const stg = reinterpret_cast<int8_t*>(lds) + ((nwin * win * 4 + 15) & ~15) +
                      RS * 1024 * __builtin_amdgcn_readfirstlane(wave);
  // ONE: a single round (K <= NW * PS), known at compile time: no loop, and
  // the registers of the round are allocated as straight-line code
  for (int r = 0; r < (ONE ? 1 : rounds); ++r) {
    int* wbuf = ONE ? win0 : win0 + (r & 1) * win;     // two windows (one if one round):
                                                        // one barrier per round
    const int k0 = (NW * r + wave) * PS;                // this wave's span
    const int gfirst = (NW * r * PS) / group;           // first group that can end in round r
    v4i wv[RS], xv[RS][2];
    double scv[NSC];
    if constexpr (STAGE) {
      // the previous round's fragment reads from the staging have returned
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int c = 0; c < RS; ++c) {
        const int row = RPC * c + lane / LPR, u = w4_slot<LPR>(lane % LPR, row);
        const bool ok = 32 * u < PS && k0 + 32 * u < K;
        w4_copy16_to_lds(rw, stg + 1024 * c,
                         ok ? (uint32_t)row * (uint32_t)KB + (uint32_t)(k0 / 2 + 16 * u) : 0x80000000u);
      }
    }
#pragma unroll
    for (int s = 0; s < RS; ++s) {
      const int kc = k0 + 128 * s + 32 * q;             // the lane's chunk
      // a chunk outside the span or K reads from the row (token) past the
      // end: selecting the row, not the offset, keeps the load unconditional
      const bool ok = 128 * s + 32 * q < PS && kc < K;
      const uint32_t kk = ok ? (uint32_t)kc : 0u;
      const uint32_t wr = ok ? wrow : rows, xt = ok ? xtok : (uint32_t)MB;
      if constexpr (!STAGE)
        wv[s] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, wr * (uint32_t)KB + kk / 2, 0, 0));
      const uint32_t xo = xt * (uint32_t)K + kk;
      if constexpr (XH) {
        xv[s][0] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16u * (uint32_t)(r16 >> 3), 0, 0));
      } else {
        xv[s][0] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0));
        xv[s][1] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rx, xo + 16, 0, 0));
      }
    }
#pragma unroll
    for (int u2 = 0; u2 < NSC; ++u2) {
      const int g = gfirst + sc_g[u2] < G ? gfirst + sc_g[u2] : G;          // G: past the row
      scv[u2] = __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(
                    rs, (sc_off[u2] + (uint32_t)g) * 8u, 0, 0));
    }
    if constexpr (STAGE) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int s = 0; s < RS; ++s)
        wv[s] = *reinterpret_cast<const v4i*>(stg + r16 * (16 * LPR) + 16 * w4_slot<LPR>(4 * s + q, r16));
    }
    // an unconditional use of every loaded value: the compiler would
    // otherwise sink a step's loads into the branch that consumes them,
    // behind all the others, and wait for every load before the first MFMA
#pragma unroll
    for (int s = 0; s < RS; ++s) {
      if constexpr (XH) asm volatile("" ::"v"(wv[s]), "v"(xv[s][0]));
      else asm volatile("" ::"v"(wv[s]), "v"(xv[s][0]), "v"(xv[s][1]));
    }
    __builtin_amdgcn_sched_barrier(0);
    auto x_second_half = [&](int s) {                  // XH: row rotate by 8 lanes
      if constexpr (XH) {
#pragma unroll
        for (int d = 0; d < 4; ++d) xv[s][1][d] = __builtin_amdgcn_update_dpp(0, xv[s][0][d], 0x128, 0xF, 0xF, false);
      }
    };

    // MFMAs over the span's chunks; segment sums to LDS [segment][token][row]
    const int nch = max(0, min(PS, K - k0)) >> 5;       // chunks of this span inside K
    v4i acc = {0, 0, 0, 0};
    int seg = wave * segw, left = 0;
    auto seg_end = [&]() {
      if (r16 < MB) *reinterpret_cast<v4i*>(wbuf + seg * NO + r16 * 16 + 4 * q) = acc;
      ++seg;
    };
    if constexpr (!TR) {
      // groups of a multiple of 128 codes, spans of whole steps: MFMA j takes
      // dword j (codes 8j..8j+7) of every lane's chunk, all in one group
#pragma unroll
      for (int s = 0; s < RS; ++s) {
        if (4 * s < nch) {                              // uniform
          x_second_half(s);
          if (left == 0) {                              // a segment starts
            acc = v4i{0, 0, 0, 0};
            left = SL >> 7;
          }
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc = w4_mma8(wv[s][j], xv[s][j >> 1][2 * (j & 1)], xv[s][j >> 1][2 * (j & 1) + 1], acc);
          if (--left == 0) seg_end();
        }
      }
    } else {
#pragma unroll
    for (int s = 0; s < RS; ++s) {
      if (4 * s < nch) {                                // uniform
        x_second_half(s);
        const v4i wt = w4_transpose4(wv[s]);
        // chunk j's codes 8q..8q+7 = dwords 2q, 2q+1 of lane (t, j)'s 32 bytes
        const v4i xe = w4_transpose4(v4i{xv[s][0][0], xv[s][0][2], xv[s][1][0], xv[s][1][2]});
        const v4i xo = w4_transpose4(v4i{xv[s][0][1], xv[s][0][3], xv[s][1][1], xv[s][1][3]});
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (4 * s + j < nch) {                        // uniform
            if (left == 0) {                            // a segment starts
              acc = v4i{0, 0, 0, 0};
              left = SL >> 5;
            }
            acc = w4_mma8(wt[j], xe[j], xo[j], acc);
            if (--left == 0) seg_end();                 // segment complete
          }
        }
      }
    }
    }
    double* scw = reinterpret_cast<double*>(wbuf + nseg * NO);
#pragma unroll
    for (int u2 = 0; u2 < NSC; ++u2)
      if (tid + NT * u2 < 16 * ng) scw[sc_w[u2]] = scv[u2];
    w4_lds_barrier();

    // lane o adds the round's groups in order
    if (out_lane) {
      const double* sco = scw + orow * ngp;
      const int kr = NW * r * PS;                       // the round's first code
      if (group <= PS) {                                // uniform: every segment is a group
        const int nv = min(nseg, (K - kr) / group);
        // 16 segments per batch: one LDS round trip per 16 products (the
        // registers of the loads above are free by now; 32 per batch would
        // raise the kernel's VGPR count and cost a workgroup per CU)
        for (int i = 0; i < nv; i += 16) {
          int a16[16];
          double t16[16];
#pragma unroll
          for (int u = 0; u < 16; ++u) {                // reads stay inside the window
            const int iu = min(i + u, nseg - 1);
            a16[u] = wbuf[iu * NO + o];
            t16[u] = sco[iu];
          }
#pragma unroll
          for (int u = 0; u < 16; ++u)
            if (i + u < nv) S = S + (double)a16[u] * t16[u];
        }
      } else {                                          // a group spans P wave spans
        for (int w = 0; w < NW; ++w) {
          if (kr + w * PS >= K) break;
          gacc += wbuf[w * NO + o];                     // int32, exact
          if (++pieces == P) {
            S = S + (double)gacc * sco[gdone - gfirst];
            gacc = 0;
            pieces = 0;
            ++gdone;
          }
        }
      }
    }
  }
  if (out_lane) {
    float v = (float)(S * sxo);
    if (bias) v = v + bo;
    if (act == 1) v = relu_js(v);
    else if (act == 2) v = silu_js(v);
    y[(int64_t)(t0 + otok) * N + n0 + orow] = v;
  }
}

namespace {
struct W4MPlan {
  int nw, rs;                             // waves per workgroup, 128-code steps per span
  int PS, segw, ng;                       // span per wave and round, segments per span,
  size_t lds;                             // groups that can end in a round; LDS bytes
  bool tr;                                // chunk transpose (groups not a multiple of 128)
  bool one;                               // one round covers K
};

// Span per wave and round: a multiple of the group (as many groups as fit
// in 4 steps = 512 codes and the LDS budget) or, for groups above 512
// codes, the largest divisor of the group of at most 512 codes.
// Workgroup shape: 8 waves of 4-step spans while the grid fits the chip
// (two workgroups per CU at 94 VGPRs, three when one round covers K and the
// kernel needs 68), else 4 waves of 8-step spans (three per CU) for groups
// of a multiple of 128.
bool w4m_plan(int64_t M, int64_t N, int64_t K, int64_t group, W4MPlan* pl, int nw = 8);

bool w4m_plan(int64_t M, int64_t N, int64_t K, int64_t group, W4MPlan* pl, int nw) {
  if (M < 1 || K < 32 || K % 32 != 0 || group < 32 || group % 32 != 0 || K % group != 0) return false;
  if (K > (int64_t)1 << 24) return false;                     // 32-bit buffer offsets
  if ((M + 15) / 16 > 65535) return false;                    // token blocks: grid.y
  const int64_t NO = 16 * std::min<int64_t>(M, 16);
  // groups of a multiple of 128 codes need no chunk transpose, with spans of
  // whole 128-code steps; other groups work in 32-code chunks
  pl->tr = group % 128 != 0;
  pl->nw = nw;
  pl->rs = nw == 16 ? 2 : nw == 8 ? 4 : 8;
  const int64_t NW = pl->nw, span = 128 * pl->rs;
  const int64_t unit = pl->tr ? 32 : 128;
  // LDS: one window of segment sums and scales per round in flight (two
  // when there is more than one round)
  auto lds_of = [&](int64_t PS, int64_t segw, int64_t ng) {
    const int64_t nwin = K > NW * PS ? 2 : 1;
    return nwin * (NW * segw * NO + 2 * 16 * (ng | 1)) * 4;
  };
  int64_t PS = 0;
  if (group <= span) {
    // as many whole groups per span as fit (ng <= 64)
    for (int64_t k = span / group; k >= 1; --k)
      if (NW * k <= 64 && lds_of(k * group, k, NW * k) <= 65536) { PS = k * group; break; }
  } else {
    // the largest divisor of the group of at most `span` codes, in whole units
    for (int64_t c = span / unit; c >= 1; --c)
      if ((group / unit) % c == 0) { PS = unit * c; break; }
  }
  if (PS == 0) return false;
  pl->PS = (int)PS;
  pl->segw = PS >= group ? (int)(PS / group) : 1;
  // a round of NW * PS codes holds NW * PS / group group ends when the group
  // divides it, else at most one more
  const int64_t rc = NW * PS;
  pl->ng = (int)(rc / group + (rc % group != 0));
  pl->lds = (size_t)lds_of(PS, pl->segw, pl->ng);
  pl->one = K <= NW * PS;
  if (!(pl->ng <= 64 && pl->lds <= 65536)) return false;
  if (nw == 16 || (nw == 8 && M <= 8))   // the kernels that stage their weights (XH: M <= 8)
    pl->lds = ((pl->lds + 15) & ~(size_t)15) + (size_t)NW * pl->rs * 1024;
  // Waves per workgroup by the number of (row, token) blocks: 16 while
  // every block has a CU to itself, 4 when they outnumber the resident
  // 8-wave workgroups.  Measured with groups of 128 at K = 4096, M 3..16:
  // N = 4096 (256 blocks) 5.5 / 6.7 us at M = 4 / 16 with 16 waves against
  // 6.0 / 7.1 with 8; N = 11008 (688 blocks) 8 waves up to 8 tokens (16
  // are 4-5% slower there), and 16 above: with its weights staged the
  // 16-wave form beats the 8-wave one, which cannot stage at 16 tokens
  // (M = 16: 12.5 -> 12.0 us).
  if (nw == 8 && !pl->tr) {
    const int64_t blocks = ((N + 15) / 16) * ((M + 15) / 16);
    const int64_t cus = cu_count() > 0 ? cu_count() : 256;
    if (blocks > (pl->one ? 3 : 2) * cus) {
      W4MPlan p4;
      if (w4m_plan(M, N, K, group, &p4, 4)) *pl = p4;
    } else if (blocks <= cus || M > 8) {
      W4MPlan p16;
      if (w4m_plan(M, N, K, group, &p16, 16)) *pl = p16;
    }
  }
  return true;
}
}  // namespace

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
  int L = 1;                                     // lanes per group: a power of two dividing group / 2
  while (L < 64 && (group / 2) % (2 * L) == 0) L *= 2;
  const int64_t threads = ngroups * L;
  hipLaunchKernelGGL(k_pack_w4, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st, W,
                     N * K, group, L, wq4, scales);
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

hipError_t launch_gemv_w4(const int8_t* xq, const double* sx, int sx_stride, const uint8_t* wq4,
                          const double* sw, int64_t M, int64_t N, int64_t K, int64_t group,
                          const float* bias, int act, float* y, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  W4Plan pl;
  const bool dot4 = w4_plan(M, K, group, &pl);
  W4MPlan mp;
  const bool mfma = w4m_plan(M, N, K, group, &mp);
  // dot4 for one and two tokens (and up to four where the MFMA kernel does
  // not apply), the MFMA kernel from three tokens on
  if (mfma && (!dot4 || M >= 3)) {
    const dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16)), block(64 * mp.nw);
#define Q8_W4M1(NW, RS, TR, ONE, XH)                                                              \
  hipLaunchKernelGGL((k_gemv_w4_mfma<NW, RS, TR, ONE, XH>), grid, block, mp.lds, st, xq, sx,      \
                     sx_stride, wq4, sw, (int)M, (int)N, (int)K, (int)group, mp.PS, mp.segw,      \
                     mp.ng, bias, act, y)
#define Q8_W4M(NW, RS, TR)                                                                        \
  do {                                                                                            \
    if (mp.one) {                                                                                 \
      if (M <= 8) Q8_W4M1(NW, RS, TR, true, true);                                                \
      else Q8_W4M1(NW, RS, TR, true, false);                                                      \
    } else {                                                                                      \
      if (M <= 8) Q8_W4M1(NW, RS, TR, false, true);                                               \
      else Q8_W4M1(NW, RS, TR, false, false);                                                     \
    }                                                                                             \
  } while (0)
    if (mp.nw == 4) Q8_W4M(4, 8, false);
    else if (mp.nw == 16) Q8_W4M(16, 2, false);
    else if (mp.tr) Q8_W4M(8, 4, true);
    else Q8_W4M(8, 4, false);
#undef Q8_W4M
#undef Q8_W4M1
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

// The MFMA kernel's dynamic LDS (windows of up to 64 KiB plus 32 KiB of
// weight staging) can pass 64 KiB, which needs each launched
// instantiation's limit raised; done once per device at set-up.
hipError_t setup_w4_attributes() {
  hipError_t err;
#define Q8_W4M_LDS(NW, RS, TR, ONE, XH)                                                            \
  err = hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemv_w4_mfma<NW, RS, TR, ONE, XH>),    \
                            hipFuncAttributeMaxDynamicSharedMemorySize, 96 * 1024 + 16);          \
  if (err != hipSuccess) return err;
#define Q8_W4M_LDS4(NW, RS, TR)                                                                    \
  Q8_W4M_LDS(NW, RS, TR, true, true) Q8_W4M_LDS(NW, RS, TR, true, false)                          \
  Q8_W4M_LDS(NW, RS, TR, false, true) Q8_W4M_LDS(NW, RS, TR, false, false)
  Q8_W4M_LDS4(4, 8, false)
  Q8_W4M_LDS4(16, 2, false)
  Q8_W4M_LDS4(8, 4, true)
  Q8_W4M_LDS4(8, 4, false)
#undef Q8_W4M_LDS4
#undef Q8_W4M_LDS
  return hipSuccess;
}

}  // namespace q8
