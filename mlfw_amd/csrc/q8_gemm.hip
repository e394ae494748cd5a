// q8_gemm.hip -- int8 x int8 -> int32 matmul with the dequant epilogue fused,
// for gfx950 (CDNA4).
//
// GEMM (M > 16): C[M,N] = A[M,K] . B[N,K]^T, both operands K-contiguous
// (A = activations [M,K], B = the nn.Linear weight [N,K]).
//   * Tiles of BM x BN outputs per workgroup of 4 waves (2 x 2); each wave
//     owns a (BM/2) x (BN/2) sub-tile as a grid of 32x32 blocks computed
//     with v_mfma_i32_32x32x32_i8 (16 int32 accumulators per lane per block,
//     kept in AGPRs).  A lane feeds 16 K-bytes of one row of A and the same
//     16 K-bytes of one row of B per instruction, so fragments are single
//     128-bit LDS reads.
//   * K is walked in BK = 128-byte stages held in a ring of two LDS
//     buffers (2 x 64 KiB for the 256 x 256 tile).  Global -> LDS copies
//     use the buffer_load_dwordx4 ... lds form (no VGPR staging): each
//     instruction moves 8 tile rows x 128 B, lane l landing at LDS byte
//     16*l of the wave's destination, so every row segment is one whole
//     128-byte line.  Measured against 64-byte stages in a ring of four on
//     the 4096^3 GEMM: the same cycles per tile, half the L1 -> L2 requests
//     and barriers, and a part that holds a ~5% higher clock under the
//     MFMA load (power-limited at ~1.7 GHz): 63-64 us instead of 67 us.
//     Out-of-range rows and the K tail are fetched through offsets past
//     the buffer resource's num_records, which the hardware returns as
//     zero -- edge tiles need no separate code.
//   * LDS layout: tile row r occupies 128 B; its logical 16-byte K chunk c
//     is stored at chunk position c ^ swz(r), swz(r) = (r>>1) & 7: rows
//     r, r+2, ..., r+14 start on the same bank (128-byte rows over 256
//     bytes of banks) and the swizzle puts their chunks on eight distinct
//     16-byte bank groups.  (The 64-byte-row form of the same rule,
//     (r>>2) & 3, measured SQ_LDS_BANK_CONFLICT 0 where ((r>>1) ^ (r>>3)) & 3
//     read 4.2M conflict cycles.)  The swizzle is applied on the global side
//     (each lane fetches the chunk its LDS slot must hold), so the DMA
//     writes stay linear.
//   * Pipeline: a stage is four 32-byte K sub-steps and one barrier, before
//     its last sub-step: after it every wave is done with the stage's
//     buffer and the next stage has landed.  The refill of that buffer with
//     the stage after next goes out in two halves, in the last sub-step and
//     in the next stage's first, spread between their MFMAs (a burst of
//     copies backs up the address unit and stalls MFMA issue), and lands
//     within the two sub-steps that follow.  Fragments are double-buffered
//     in registers: every sub-step reads the next one's.
//   * Workgroup -> tile order undoes the round-robin dispatch over the 8
//     XCDs (consecutive workgroup ids land on different XCDs), then walks
//     groups of 4 tile rows column by column, so the tiles resident on one
//     XCD share rows of A and columns of B in that XCD's L2.
//   * The epilogue converts the int32 accumulators with the reference's
//     arithmetic (fround(acc * fround(sA[m] * sB[n])) or fround(acc * s_out),
//     f64 where the reference is f64), adds the bias and applies ReLU /
//     SiLU before the only store of the output.
// GEMV (M <= 16): HBM-bound on B.  M <= 4: packed int8 dot products
// (v_dot4_i32_i8), no MFMA; 4 < M <= 16: one 16x16x64 MFMA per 16 weight
// rows x 64 K-bytes (dot4 would make it VALU-bound); see the kernels' own
// comments.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <type_traits>

#include "q8_device.h"
#include "q8_internal.h"

namespace q8 {

// ------------------------------------------------------------------ epilogue
// y = fround(acc * sv) for an f32 scale sv.  When acc is exactly an f32
// (|acc| <= 2^24) the f32 multiply rounds the exact product once, which is
// what Math.fround((+acc) * sv) does in f64 (a binary32 product of two
// binary32 values is exact in binary64); otherwise the f64 form is used.
__device__ __forceinline__ float mul_acc_f32scale(int acc, float sv) {
  if ((unsigned)(acc + (1 << 24)) <= (2u << 24)) return (float)acc * sv;
  return (float)((double)acc * (double)sv);
}

__device__ __forceinline__ float epi_finish(float y, int64_t n, const GemmEpi& e) {
  if (e.bias) y = y + e.bias[n];   // binary32 add == Math.fround(f64 add) for f32 operands
  if (e.act == 1) y = relu_js(y);
  else if (e.act == 2) y = silu_js(y);
  return y;
}

__device__ __forceinline__ float epi_value(int acc, int64_t m, int64_t n, const GemmEpi& e) {
  float y;
  if (e.mode == 0) {
    y = (float)((double)acc * e.s_out);
  } else {
    const float sv = (float)(e.sA[m * e.sA_stride] * e.sB[n * e.sB_stride]);
    y = mul_acc_f32scale(acc, sv);
  }
  return epi_finish(y, n, e);
}

// The compiled `quantize` (quant_math.ts:16-27) of an epilogue value with the
// next layer's static scale: q = (min(max(Math.round(fround(y / s)), -128), 127) | 0).
__device__ __forceinline__ int requant(float y, const GemmEpi& e) {
  return e.q_fast ? quant_sym_fast(y, e.rq32, e.s_q) : quant_exact(y, e.s_q, 0.0, -128, 127);
}

// Final store of one output element of the GEMV / generic kernels.
__device__ __forceinline__ void store_out(void* out, int64_t idx, int acc, int64_t m, int64_t n,
                                          const GemmEpi& e) {
  if (e.col_blk > 0) idx = (n / e.col_blk) * e.blk_stride + m * e.ld_out + n % e.col_blk;
  if (e.out_i32) static_cast<int32_t*>(out)[idx] = acc;
  else if (e.out_q8) static_cast<int8_t*>(out)[idx] = (int8_t)requant(epi_value(acc, m, n, e), e);
  else static_cast<float*>(out)[idx] = epi_value(acc, m, n, e);
}

// ------------------------------------------------------------------ MFMA GEMM
constexpr int BK = 128;                 // K bytes per LDS stage
constexpr int NBUF = 2;                 // LDS stages in the ring
constexpr int GEMM_THREADS = 256;       // 4 waves, 2 x 2
constexpr uint32_t OOB = 0x80000000u;   // voffset past every buffer's num_records

template <int BM, int BN>
struct GemmCfg {
  static constexpr int WM = BM / 2, WN = BN / 2;      // per-wave sub-tile
  static constexpr int TM = WM / 32, TN = WN / 32;    // 32x32 blocks per wave
  static constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int LDS = NBUF * STAGE;              // the stage ring
  static constexpr int LDS_TOTAL = LDS + 8 * (BM + BN);  // + the tile's f64 scales
  static constexpr int A_LOADS = BM / 32;              // 8-row copies per wave per stage
  static constexpr int B_LOADS = BN / 32;
  static_assert(TM >= 1 && TN >= 1 && BM % 64 == 0 && BN % 64 == 0, "tile shape");
};

__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

// Buffer resource (V#) of a raw byte range: base, stride 0, num_records
// bytes, gfx9 data-format word.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const int8_t* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// 16 bytes per lane from buffer offset voff to LDS dst + 16 * lane.
__device__ __forceinline__ void copy16_to_lds(__amdgpu_buffer_rsrc_t r, int8_t* dst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      r, (__attribute__((address_space(3))) void*)dst, 16, voff, 0, 0, 0);
}

// End of a stage: this wave's LDS copies have landed and its fragment reads
// have returned, then all waves meet.  Written as one asm statement because
// the compiler's wait-count pass would otherwise relax an explicit
// lgkmcnt(0) whose results it sees as not yet needed; the next stage's
// copies overwrite the buffer those reads came from.
__device__ __forceinline__ void stage_sync() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// As stage_sync, but up to N of this wave's most recent copies (later
// stages) may still be in flight: vector-memory loads complete in issue
// order, so vmcnt(N) means every older copy has landed.
template <int N>
__device__ __forceinline__ void stage_sync_keep() {
  static_assert(N >= 0 && N <= 63, "vmcnt immediate");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Instruction order of one sub-step (compiler schedule groups): NF
// fragment reads paired with the first MFMAs, then NC copies spread evenly
// over the remaining MFMAs.  Keeps the LDS reads one sub-step ahead of
// their use and never lets a burst of copies back up the address unit
// while the MFMAs wait behind them.
template <int NF, int NM, int NC>
__device__ __forceinline__ void sched_substep() {
  constexpr int G1 = NF < NM ? NF : NM;
#pragma unroll
  for (int x = 0; x < G1; ++x) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
  }
  if constexpr (NF > G1) __builtin_amdgcn_sched_group_barrier(0x100, NF - G1, 0);
  constexpr int R = NM - G1;
  if constexpr (NC == 0) {
    if constexpr (R > 0) __builtin_amdgcn_sched_group_barrier(0x008, R, 0);
  } else if constexpr (R == 0) {
    __builtin_amdgcn_sched_group_barrier(0x020, NC, 0);
  } else if constexpr (NC <= R) {
    constexpr int PER = R / NC;
#pragma unroll
    for (int x = 0; x < NC; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, PER, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM (copy)
    }
    if constexpr (R - PER * NC > 0) __builtin_amdgcn_sched_group_barrier(0x008, R - PER * NC, 0);
  } else {
    constexpr int PER = NC / R;
#pragma unroll
    for (int x = 0; x < R; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, PER, 0);
    }
    if constexpr (NC - PER * R > 0) __builtin_amdgcn_sched_group_barrier(0x020, NC - PER * R, 0);
  }
}

// Workgroup id -> (tile row, tile col).  Dispatch places consecutive ids on
// consecutive XCDs (id % 8); the remap gives each XCD a contiguous run of
// the grouped tile order below.
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int G = tiles_m * tiles_n;
  const int xcd = bid & 7, k = bid >> 3;
  const int per = G >> 3, rem = G & 7;
  const int id = xcd < rem ? xcd * (per + 1) + k : rem * (per + 1) + (xcd - rem) * per + k;
  constexpr int GROUP = 4;
  const int group = id / (GROUP * tiles_n);
  const int first = group * GROUP;
  const int gm = min(tiles_m - first, GROUP);
  const int in = id - group * GROUP * tiles_n;
  tm = first + in % gm;
  tn = in / gm;
}

// Maximum over each half of the wave (lanes 0-31, 32-63), in the last lane
// of the half (lanes 31 and 63; other lanes hold partial maxima).  DPP row
// operations stay in the VALU: quad swaps, the half-row and row mirrors
// reduce each 16-lane row, then row_bcast:15 feeds lane 15 of rows 0 and 2
// into rows 1 and 3.  (A ds_bpermute butterfly takes an LDS round trip per
// step.)
__device__ __forceinline__ int half_wave_max(int v) {
  auto mx = [](int a, int b) { return a > b ? a : b; };
  v = mx(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  v = mx(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  v = mx(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  v = mx(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false));  // row_mirror
  v = mx(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xA, 0xF, false));  // row_bcast:15 into rows 1, 3
  return v;
}

// Compile-time epilogue variant of the MFMA kernel:
//   bit 4 int32 output (raw accumulators), else fp32 output with
//   bit 3 MODE (0: fround(acc * s_out), 1: fround(acc * fround(sA[m] * sB[n]))),
//   bit 2 bias, bits 0-1 activation (0 none, 1 ReLU, 2 SiLU);
//   bit 5 int8 output: the fp32 value (MODE as above, bias and activation
//   taken from the runtime epilogue) requantized with a static scale;
//   bit 6 int8 output requantized per row with the row's dynamic absmax
//   scale (every tile resident at once; the OUT_DQ branch of k_qgemm's
//   epilogue).
template <int EPI>
struct Epi {
  static constexpr bool OUT_I32 = (EPI & 16) != 0;
  static constexpr bool OUT_Q8 = (EPI & 32) != 0;
  static constexpr bool OUT_DQ = (EPI & 64) != 0;
  static constexpr bool COLBLK = (EPI & 128) != 0;   // GemmEpi::col_blk addressing
  static constexpr bool IMPL = (EPI & 256) != 0;     // B is a conv frame (GemmEpi::cb)
  static constexpr bool GLU = (EPI & 512) != 0;      // gate|up interleaved, h = silu(g) * u out
  static constexpr int MODE = (EPI >> 3) & 1;
  static constexpr bool BIAS = (EPI & 4) != 0;
  static constexpr int ACT = EPI & 3;
};

inline int epi_code(const GemmEpi& e) {
  if (e.out_dq) return 64 | (e.mode << 3);
  const int cb = e.col_blk > 0 ? 128 : 0;
  if (e.out_i32) return 16 | cb;
  if (e.out_q8) return 32 | (e.mode << 3);
  return (e.mode << 3) | (e.bias ? 4 : 0) | e.act | cb;
}

// Implicit conv B operand (GemmEpi::ConvB): frame offset of tap t relative
// to tap 0, in positions.
__device__ __forceinline__ uint32_t convb_tap(const GemmEpi::ConvB& c, uint32_t t) {
  const uint32_t k2 = t % c.K2, r = t / c.K2, k1 = r % c.K1, k0 = r / c.K1;
  return (k0 * c.dl0 * c.E1 + k1 * c.dl1) * c.E2 + k2 * c.dl2;
}
// frame byte offset of GEMM column n's contraction byte 0 (tap 0, channel 0)
__device__ __forceinline__ uint32_t convb_row(const GemmEpi::ConvB& c, uint32_t n) {
  const uint32_t y = n / c.Pn, p = n - y * c.Pn;
  const uint32_t o2 = p % c.P2, q = p / c.P2, o1 = q % c.P1, o0 = q / c.P1;
  return (y * c.Ep + (o0 * c.st0 * c.E1 + o1 * c.st1) * c.E2 + o2 * c.st2) * c.Cg;
}
// byte offsets, relative to a column's convb_row, of the two 64-byte halves
// of K stage s (contraction bytes 128 s .. 128 s + 127): Cg is a multiple of
// 64, so a half never straddles two taps.  A half past the last tap
// repeats the first (its lanes read out of range there).
__device__ __forceinline__ void convb_stage(const GemmEpi::ConvB& c, uint32_t s, uint32_t& lo,
                                            uint32_t& hi) {
  const uint32_t k = 128u * s, t = k / c.Cg, ch = k - t * c.Cg;
  lo = convb_tap(c, t) * c.Cg + ch;
  hi = ch + 64 < c.Cg ? lo + 64 : (t + 1 < c.Kn ? convb_tap(c, t + 1) * c.Cg : lo);
}

template <int BM, int BN, int EPI>
__global__ __launch_bounds__(GEMM_THREADS, 1)
void k_qgemm(const int8_t* __restrict__ A, const int8_t* __restrict__ B, int M, int N, int K,
             int tiles_m, int tiles_n, GemmEpi e, void* __restrict__ out) {
  using C = GemmCfg<BM, BN>;
  constexpr bool OUT_I32 = Epi<EPI>::OUT_I32;
  constexpr int MODE = Epi<EPI>::MODE;
  constexpr bool IMPL = Epi<EPI>::IMPL;
  extern __shared__ __attribute__((aligned(1024))) int8_t lds[];
  // the wave index is uniform: kept in an SGPR, the LDS destinations of the
  // copies (M0) follow without a VGPR round trip
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int tm, tn;
  // IMPL: blockIdx.x = split * tiles + tile; split s takes K stages
  // [s * kps, (s + 1) * kps) and, with more than one split, writes its raw
  // partial sums to out + s * M * N (row-major int32)
  const int split = IMPL ? (int)(blockIdx.x / (unsigned)(tiles_m * tiles_n)) : 0;
  tile_of(IMPL ? (int)blockIdx.x - split * tiles_m * tiles_n : (int)blockIdx.x, tiles_m, tiles_n, tm, tn);
  if constexpr (IMPL) out = static_cast<int32_t*>(out) + (int64_t)split * M * N;
  const int m0 = tm * BM, n0 = tn * BN;
  const int rows_a = min(BM, M - m0), rows_b = min(BN, N - n0);
  const int8_t* Ab = A + (int64_t)m0 * K;
  const int8_t* Bb = B + (int64_t)n0 * K;

  // The tile's epilogue scales: loaded now, stored to LDS behind the two
  // stages once the prologue copies are issued.
  double* s_rows = reinterpret_cast<double*>(lds + C::LDS);
  double* s_cols = s_rows + BM;
  constexpr int NSC = (BM + BN + GEMM_THREADS - 1) / GEMM_THREADS;
  double scv[NSC];
#pragma unroll
  for (int u = 0; u < NSC; ++u) {
    const int t = tid + u * GEMM_THREADS;
    double v = 0.0;
    if (!OUT_I32 && MODE == 1) {
      if (t < BM) { if (t < rows_a) v = e.sA[(int64_t)(m0 + t) * e.sA_stride]; }
      else if (t < BM + BN && t - BM < rows_b) v = e.sB[(int64_t)(n0 + t - BM) * e.sB_stride];
    }
    scv[u] = v;
  }

  // Copy plan: wave w fills tile rows [w*BM/4, (w+1)*BM/4) of A and the
  // same share of B, 8 rows per instruction.  Lane l lands in row
  // 8j + l/8 at chunk position l%8 and so fetches logical chunk
  // (l%8) ^ swz(row).
  uint32_t offa[C::A_LOADS], offb[C::B_LOADS];
  int kca[C::A_LOADS], kcb[C::B_LOADS];
#pragma unroll
  for (int j = 0; j < C::A_LOADS; ++j) {
    const int row = wave * (BM / 4) + 8 * j + (lane >> 3);
    kca[j] = 16 * ((lane & 7) ^ swz(row));
    offa[j] = row < rows_a ? (uint32_t)(row * K + kca[j]) : OOB;
  }
#pragma unroll
  for (int j = 0; j < C::B_LOADS; ++j) {
    const int row = wave * (BN / 4) + 8 * j + (lane >> 3);
    kcb[j] = 16 * ((lane & 7) ^ swz(row));
    if constexpr (IMPL)   // the column's frame row; the stage adds its tap offset
      offb[j] = row < rows_b ? convb_row(e.cb, (uint32_t)(n0 + row)) + (uint32_t)(kcb[j] & 63) : OOB;
    else
      offb[j] = row < rows_b ? (uint32_t)(row * K + kcb[j]) : OOB;
  }
  // IMPL: lane l holds the half offsets of K stages l and l + 64
  uint32_t stg_lo[2] = {0u, 0u}, stg_hi[2] = {0u, 0u};
  if constexpr (IMPL) {
#pragma unroll
    for (int r = 0; r < 2; ++r) convb_stage(e.cb, (uint32_t)(lane + 64 * r), stg_lo[r], stg_hi[r]);
  }
  const uint32_t bytes_a = (uint32_t)rows_a * (uint32_t)K;
  const uint32_t bytes_b = (uint32_t)rows_b * (uint32_t)K;
  const int KT = (K + BK - 1) / BK;
  const int kt0 = IMPL ? split * (int)e.cb.kps : 0;                    // this split's stages
  const int KTe = IMPL ? min(KT, kt0 + (int)e.cb.kps) : KT;
  // offsets for the last stage when K is not a multiple of BK: the lane's
  // chunk past K reads past the buffer's end (zero) instead of the next row
  const int kb_last = (KT - 1) * BK;
  uint32_t offa_t[C::A_LOADS], offb_t[C::B_LOADS];
#pragma unroll
  for (int j = 0; j < C::A_LOADS; ++j) offa_t[j] = kb_last + kca[j] >= K ? OOB : offa[j];
#pragma unroll
  for (int j = 0; j < C::B_LOADS; ++j) offb_t[j] = kb_last + kcb[j] >= K ? OOB : offb[j];

  // Copies j0 <= j < j1 of the A (resp. B) part of K stage kt into
  // `stage`.  kt >= KT copies nothing: with num_records 0 every lane is out
  // of range and writes zeros into a stage that is no longer read, which
  // keeps the loop body branch-free.
  auto issue_a = [&](int kt, int8_t* stage, int j0, int j1) {
    const bool live = kt < KTe;
    const int kb = live ? kt * BK : 0;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(Ab + kb, live ? bytes_a - (uint32_t)kb : 0u);
    int8_t* sa = stage + wave * (BM / 4) * BK;
    const bool tail = kb + BK > K;
#pragma unroll
    for (int j = 0; j < C::A_LOADS; ++j)
      if (j >= j0 && j < j1) copy16_to_lds(ra, sa + j * 8 * BK, tail ? offa_t[j] : offa[j]);
  };
  auto issue_b = [&](int kt, int8_t* stage, int j0, int j1) {
    if constexpr (IMPL) {
      // the stage's two halves sit at frame offsets lo and hi from each
      // column's row; the resource starts at the lower one
      // (both lanes read, then a bit select: no branch in the loop)
      const bool live = kt < KTe;
      const int s = live ? kt : 0;
      const uint32_t up = 0u - (uint32_t)(s >> 6);   // all ones for stages 64 .. 127
      const uint32_t lo0 = __builtin_amdgcn_readlane(stg_lo[0], s & 63);
      const uint32_t lo1 = __builtin_amdgcn_readlane(stg_lo[1], s & 63);
      const uint32_t hi0 = __builtin_amdgcn_readlane(stg_hi[0], s & 63);
      const uint32_t hi1 = __builtin_amdgcn_readlane(stg_hi[1], s & 63);
      const uint32_t lo = lo0 ^ ((lo0 ^ lo1) & up), hi = hi0 ^ ((hi0 ^ hi1) & up);
      const uint32_t base = lo < hi ? lo : hi;
      const __amdgpu_buffer_rsrc_t rb = make_rsrc(B + base, live ? e.cb.frame_bytes - base : 0u);
      const uint32_t dlo = lo - base, dhi = hi - base;
      int8_t* sb = stage + C::A_BYTES + wave * (BN / 4) * BK;
      const bool tail = s * BK + BK > K;
#pragma unroll
      for (int j = 0; j < C::B_LOADS; ++j)
        if (j >= j0 && j < j1)
          copy16_to_lds(rb, sb + j * 8 * BK, (tail ? offb_t[j] : offb[j]) + (kcb[j] >= 64 ? dhi : dlo));
    } else {
      const bool live = kt < KTe;
      const int kb = live ? kt * BK : 0;
      const __amdgpu_buffer_rsrc_t rb = make_rsrc(Bb + kb, live ? bytes_b - (uint32_t)kb : 0u);
      int8_t* sb = stage + C::A_BYTES + wave * (BN / 4) * BK;
      const bool tail = kb + BK > K;
#pragma unroll
      for (int j = 0; j < C::B_LOADS; ++j)
        if (j >= j0 && j < j1) copy16_to_lds(rb, sb + j * 8 * BK, tail ? offb_t[j] : offb[j]);
    }
  };

  // Fragment addresses: byte offset of the fragment row within a stage and
  // the lane's swizzle (sub-step kk reads logical chunk 2*kk + kh, which
  // sits at position (2*kk) ^ (kh ^ swz(row))).
  const int wm = (wave >> 1) * C::WM, wn = (wave & 1) * C::WN;
  const int r32 = lane & 31, kh = lane >> 5;
  int fa_off[C::TM], fa_sw[C::TM], fb_off[C::TN], fb_sw[C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i) {
    const int row = wm + 32 * i + r32;
    fa_off[i] = row * BK;
    fa_sw[i] = kh ^ swz(row);
  }
#pragma unroll
  for (int j = 0; j < C::TN; ++j) {
    const int row = wn + 32 * j + r32;
    fb_off[j] = C::A_BYTES + row * BK;
    fb_sw[j] = kh ^ swz(row);
  }
  auto read_frags = [&](const int8_t* st, int kk, v4i* fa, v4i* fb) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
      fa[i] = *reinterpret_cast<const v4i*>(st + fa_off[i] + 16 * ((2 * kk) ^ fa_sw[i]));
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
      fb[j] = *reinterpret_cast<const v4i*>(st + fb_off[j] + 16 * ((2 * kk) ^ fb_sw[j]));
  };

  v16i acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
  auto mfma_all = [&](const v4i* fa, const v4i* fb) {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
  };

  // Pipeline over a ring of NBUF = 2 stages (stage kt in buffer kt % 2).
  // A stage is four 32-byte K sub-steps.  The barrier of stage kt sits
  // before its last sub-step: every fragment read of buffer kt % 2 has
  // returned (the last sub-step's fragments were read one sub-step ahead)
  // and stage kt+1 has landed.  The refill of buffer kt % 2 with stage
  // kt+2 goes out in two halves: with the last sub-step of stage kt and the
  // first of stage kt+1, so every copy has at least two sub-steps to land
  // before the next barrier.
  int8_t* const ring = lds;
  auto buf = [&](int kt) { return ring + (kt & (NBUF - 1)) * C::STAGE; };
  constexpr int NV = C::A_LOADS + C::B_LOADS;    // copies per stage
  constexpr int HA = C::A_LOADS / 2, HB = C::B_LOADS / 2;
  static_assert(C::A_LOADS % 2 == 0 && C::B_LOADS % 2 == 0, "copies split in halves");
  issue_a(kt0, buf(kt0), 0, C::A_LOADS);
  issue_b(kt0, buf(kt0), 0, C::B_LOADS);
  issue_a(kt0 + 1, buf(kt0 + 1), 0, C::A_LOADS);
  issue_b(kt0 + 1, buf(kt0 + 1), 0, C::B_LOADS);
  if (!OUT_I32 && MODE == 1) {
#pragma unroll
    for (int u = 0; u < NSC; ++u)
      if (tid + u * GEMM_THREADS < BM + BN) s_rows[tid + u * GEMM_THREADS] = scv[u];
  }
  stage_sync_keep<NV>();                          // stage 0 landed
  v4i fa0[C::TM], fb0[C::TN], fa1[C::TM], fb1[C::TN];
  read_frags(buf(kt0), 0, fa0, fb0);
  for (int kt = kt0; kt < KTe; ++kt) {
    int8_t* cur = buf(kt);
    // sub-step 0; the second half of stage kt+1's copies (stage 1 went out
    // whole in the prologue)
    read_frags(cur, 1, fa1, fb1);
    if (kt >= kt0 + 1) {
      issue_a(kt + 1, buf(kt + 1), HA, C::A_LOADS);
      issue_b(kt + 1, buf(kt + 1), HB, C::B_LOADS);
    }
    mfma_all(fa0, fb0);
    sched_substep<C::TM + C::TN, C::TM * C::TN, NV / 2>();
    // sub-steps 1 and 2
    read_frags(cur, 2, fa0, fb0);
    mfma_all(fa1, fb1);
    sched_substep<C::TM + C::TN, C::TM * C::TN, 0>();
    read_frags(cur, 3, fa1, fb1);
    mfma_all(fa0, fb0);
    sched_substep<C::TM + C::TN, C::TM * C::TN, 0>();
    // every read of `cur` returned everywhere; stage kt+1 landed
    stage_sync();
    // sub-step 3; the first half of stage kt+2's copies into `cur`
    read_frags(buf(kt + 1), 0, fa0, fb0);
    issue_a(kt + 2, cur, 0, HA);
    issue_b(kt + 2, cur, 0, HB);
    mfma_all(fa1, fb1);
    sched_substep<C::TM + C::TN, C::TM * C::TN, NV / 2>();
  }
  // The last iterations issued zero-filling copies for stages past KT into
  // the stage buffers the epilogue reuses: drain them first.
  stage_sync();

  // Epilogue, one 32-row strip of the wave's sub-tile at a time:
  //  1. the scales, bias and activation are applied in the accumulator
  //     layout (lane l holds column 32j + l%32 and rows (r/4)*8 + (l/32)*4
  //     + r%4 of each 32x32 block), with one exactness test per strip;
  //  2. the 32 x WN results go through this wave's own LDS region (row
  //     pitch WN + 8 words; the stage buffers are free after the last
  //     barrier) and come back as 4-column quads, so every lane stores 16
  //     bytes.  Stores are non-temporal: the kernel never reads them back.
  using P = Epi<EPI>;
  constexpr int PITCH = C::WN + 8;                    // 32-bit words per strip row
  constexpr int LPR = C::WN / 4;                      // lanes per strip row
  constexpr int RPI = 64 / LPR;                       // strip rows per read
  constexpr int NQ = 32 / RPI;                        // quads per lane per strip
  static_assert(4 * 32 * PITCH * 4 <= C::LDS, "epilogue strips fit in the stage buffers");
  int32_t* strip = reinterpret_cast<int32_t*>(lds) + wave * 32 * PITCH;
  const int qcol = 4 * (lane % LPR), qrow = lane / LPR;
  const bool qlane = 64 % LPR == 0 || lane < LPR * RPI;   // lanes that own quads of the strip
  const int gcol = n0 + wn + qcol;
  // COLBLK: 16-byte quads need column blocks, and so the rows of every
  // block, that start on multiples of 4 elements
  const bool interior = m0 + BM <= M && n0 + BN <= N && (N % 4 == 0) &&
                        (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
                        (!P::COLBLK || ((e.col_blk | e.blk_stride | e.ld_out) & 3) == 0);
  // COLBLK: the column part of this lane's output offset (fixed for the lane)
  const int64_t colblk_base =
      P::COLBLK ? ((int64_t)gcol / e.col_blk) * e.blk_stride + (int64_t)gcol % e.col_blk : 0;
  double sbj[C::TN];
  float bj[C::TN];
#pragma unroll
  for (int j = 0; j < C::TN; ++j) {
    const int lc = wn + 32 * j + r32;
    sbj[j] = (!OUT_I32 && MODE == 1) ? s_cols[lc] : 0.0;
    if constexpr (P::BIAS) bj[j] = e.bias[n0 + lc < N ? n0 + lc : N - 1];
    else if constexpr (P::OUT_Q8 || P::OUT_DQ || P::GLU) bj[j] = e.bias ? e.bias[n0 + lc < N ? n0 + lc : N - 1] : 0.0f;
    else bj[j] = 0.0f;
  }
  auto strip_out = [&](auto ic) {
    constexpr int i = decltype(ic)::value;
    auto slot = [&](int j, int r) -> int32_t& {
      return strip[((r >> 2) * 8 + kh * 4 + (r & 3)) * PITCH + 32 * j + r32];
    };
    if constexpr (OUT_I32) {
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) slot(j, r) = acc[i][j][r];
    } else {
      double sar[16];
      if constexpr (MODE == 1) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sar[r] = s_rows[wm + 32 * i + (r >> 2) * 8 + kh * 4 + (r & 3)];
      }
      // binary32 multiply when every accumulator of the strip is exactly a
      // binary32 value (|acc| <= 2^24), the f64 form otherwise
      bool exact = true;
      if constexpr (MODE == 1) {
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) exact &= (unsigned)(acc[i][j][r] + (1 << 24)) <= (2u << 24);
      }
      const bool fast = __all(exact);
      auto finish = [&](float y, int j) {
        if constexpr (P::BIAS) y = y + bj[j];
        if constexpr (P::ACT == 1) y = relu_js(y);
        if constexpr (P::ACT == 2) y = silu_js(y);
        return y;
      };
      if (MODE == 0 || fast) {
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float y;
            if constexpr (MODE == 0) y = (float)((double)acc[i][j][r] * e.s_out);
            else y = (float)acc[i][j][r] * (float)(sar[r] * sbj[j]);
            slot(j, r) = __float_as_int(finish(y, j));
          }
      } else {
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float y = mul_acc_f32scale(acc[i][j][r], (float)(sar[r] * sbj[j]));
            slot(j, r) = __float_as_int(finish(y, j));
          }
      }
    }
    // a strip row of WN = 96 columns is 24 lanes' quads: 48 lanes read two
    // rows at a time and lanes 48-63 sit out
    if (!qlane) return;
    v4i q[NQ];
#pragma unroll
    for (int it = 0; it < NQ; ++it)
      q[it] = *reinterpret_cast<const v4i*>(strip + (it * RPI + qrow) * PITCH + qcol);
    int32_t* o = static_cast<int32_t*>(out);
    if (interior) {
#pragma unroll
      for (int it = 0; it < NQ; ++it) {
        const int64_t row = m0 + wm + 32 * i + it * RPI + qrow;
        // COLBLK: a quad never straddles two column blocks (col_blk % 4 == 0)
        const int64_t at = P::COLBLK ? colblk_base + row * e.ld_out : row * N + gcol;
        __builtin_nontemporal_store(q[it], reinterpret_cast<v4i*>(o + at));
      }
    } else {
#pragma unroll
      for (int it = 0; it < NQ; ++it) {
        const int row = m0 + wm + 32 * i + it * RPI + qrow;
        if (row < M) {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (gcol + c < N) {
              int64_t at = (int64_t)row * N + gcol + c;
              if constexpr (P::COLBLK) {   // N < 2^31: 32-bit division
                const unsigned j = (unsigned)(gcol + c), cb = (unsigned)e.col_blk;
                const unsigned blk = j / cb;
                at = (int64_t)blk * e.blk_stride + (int64_t)row * e.ld_out + (j - blk * cb);
              }
              o[at] = q[it][c];
            }
        }
      }
    }
  };
  if constexpr (P::GLU) {
    // Gate|up with SiLU(gate) * up (decomposition_pass.ts:197-230): B holds
    // the gate and up weights interleaved in groups of 32 rows (packed
    // column 64 g + c is gate feature 32 g + c, 64 g + 32 + c is up feature
    // 32 g + c), and BN is a multiple of 128, so the wave's 32x32 blocks 2p
    // and 2p + 1 hold the gate and up accumulators of the same 32 features.
    // Per strip of 32 rows the accumulators go to the wave's LDS strip
    // (accumulator layout, static register indices), then a rolled loop over
    // the lane's 4-feature quads reads each quad's gate and up accumulators,
    // takes both epilogues (E-rowcol, bias), h = fround(silu(g) * u) (a
    // binary32 product of binary32 values is the rounded exact product) and
    // stores the 16-byte quad of h ([M, N/2] fp32).  Rolled, so the code
    // the wave runs stays small: the f64 exp of every SiLU inlined over the
    // 256 values a lane holds would overflow the instruction cache.
    static_assert(C::TN % 2 == 0 && MODE == 1, "GLU needs pairs of column blocks and the row x column scales");
    constexpr int WH = C::WN / 2;                  // h columns of the wave
    constexpr int LPRH = WH / 4, RPIH = 64 / LPRH, NQH = 32 / RPIH;
    static_assert(64 % LPRH == 0, "whole strip rows per lane set");
    static_assert(NQH % 2 == 0, "quads in pairs");
    const int64_t F = N / 2;
    const int qcolh = 4 * (lane % LPRH), qrowh = lane / LPRH;
    // the lane's four h columns are features qcolh .. qcolh + 3 of the wave:
    // pair p = qcolh / 32, gate strip columns 64 p + qcolh % 32 + c, up 32 after
    const int gcs = 64 * (qcolh / 32) + (qcolh % 32);
    const int64_t hcol = (int64_t)(n0 + wn) / 2 + qcolh;
    double sg4[4], su4[4];
    float bg4[4], bu4[4];
    const bool has_bias = e.bias != nullptr;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int lg = wn + gcs + c, lu = lg + 32;
      sg4[c] = s_cols[lg];
      su4[c] = s_cols[lu];
      bg4[c] = has_bias ? e.bias[n0 + lg < N ? n0 + lg : N - 1] : 0.0f;
      bu4[c] = has_bias ? e.bias[n0 + lu < N ? n0 + lu : N - 1] : 0.0f;
    }
    float* hout = static_cast<float*>(out);
    const bool interior_h = m0 + BM <= M && n0 + BN <= N && (F % 4 == 0) &&
                            (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    auto glu_strip = [&](auto ic) {
      constexpr int i = decltype(ic)::value;
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) strip[((r >> 2) * 8 + kh * 4 + (r & 3)) * PITCH + 32 * j + r32] = acc[i][j][r];
#pragma unroll 1
      for (int it0 = 0; it0 < NQH; it0 += 2) {
        float h[2][4];
        int64_t rowg[2];
#pragma unroll
        for (int u2 = 0; u2 < 2; ++u2) {
          const int srow = (it0 + u2) * RPIH + qrowh;           // strip row
          rowg[u2] = m0 + wm + 32 * i + srow;
          const v4i ag = *reinterpret_cast<const v4i*>(strip + srow * PITCH + gcs);
          const v4i au = *reinterpret_cast<const v4i*>(strip + srow * PITCH + gcs + 32);
          const double sr = s_rows[wm + 32 * i + srow];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            float g = mul_acc_f32scale(ag[c], (float)(sr * sg4[c]));
            float u = mul_acc_f32scale(au[c], (float)(sr * su4[c]));
            if (has_bias) {
              g = g + bg4[c];
              u = u + bu4[c];
            }
            h[u2][c] = silu_js(g) * u;
          }
        }
        if (interior_h) {
#pragma unroll
          for (int u2 = 0; u2 < 2; ++u2) {
            const v4i hv{__float_as_int(h[u2][0]), __float_as_int(h[u2][1]), __float_as_int(h[u2][2]),
                         __float_as_int(h[u2][3])};
            v4i* dst = reinterpret_cast<v4i*>(hout + rowg[u2] * F + hcol);
            if (e.h_plain) *dst = hv;
            else __builtin_nontemporal_store(hv, dst);
          }
        } else {
#pragma unroll
          for (int u2 = 0; u2 < 2; ++u2)
            if (rowg[u2] < M) {
#pragma unroll
              for (int c = 0; c < 4; ++c)
                if (hcol + c < F) hout[rowg[u2] * F + hcol + c] = h[u2][c];
            }
        }
      }
    };
    glu_strip(std::integral_constant<int, 0>{});
    if constexpr (C::TM > 1) glu_strip(std::integral_constant<int, 1>{});
    if constexpr (C::TM > 2) glu_strip(std::integral_constant<int, 2>{});
    if constexpr (C::TM > 3) glu_strip(std::integral_constant<int, 3>{});
    static_assert(C::TM <= 4, "glu_strip calls cover TM <= 4");
  } else if constexpr (P::OUT_DQ) {
    // Dynamic per-row requant: the row's scale is S-abs over all N columns,
    // so every tile of a row block must have seen its values first.
    //  A. per strip: the accumulators go to the wave's LDS strip; a rolled
    //     loop over the lane's 4-column quads (one row each) applies the
    //     scales, bias and activation, takes the quad's absmax key, reduces
    //     it over the lanes of the row and max-es it into the tile's row
    //     keys (LDS); the fp32 values go back to the accumulator registers
    //     in quad order;
    //  B. the tile's row keys are max-ed into the caller's workspace (one
    //     32-bit atomic per row) and all workgroups (co-resident: one per
    //     CU, no more than the chip holds) meet once: an arrival counter, polled with a
    //     bound (a timed-out wait sets the status word and carries on with
    //     the keys it sees);
    //  C. each row's scale, and its binary32 reciprocal (NaN where the f32
    //     fast path does not apply), is computed once into LDS; per strip
    //     the values return to the LDS strip and a rolled loop quantizes
    //     each quad like q8_quantize_rows does (R1 with the row scale) and
    //     stores its 4 codes; the tiles of column 0 store the scales.
    // The per-element work runs in rolled loops reading LDS, so the code a
    // wave executes stays small: unrolled over the 256 values a lane holds
    // (with the exact-path and activation code between them) it overflows
    // the instruction cache and costs more than the main loop.
    constexpr int STRIP_WORDS = 4 * 32 * PITCH;
    static_assert((STRIP_WORDS + BM) % 2 == 0, "row scales are 8-byte aligned");
    static_assert((STRIP_WORDS + BM) * 4 + BM * 12 <= C::LDS, "row keys and scales fit in the stage buffers");
    int* tkey = reinterpret_cast<int32_t*>(lds) + STRIP_WORDS;                 // [BM] row keys
    double* rscale = reinterpret_cast<double*>(lds + (STRIP_WORDS + BM) * 4);  // [BM] row scales
    float* rrcp = reinterpret_cast<float*>(rscale + BM);                      // [BM] f32 reciprocals
    if (tid < BM) tkey[tid] = -1;
    __syncthreads();
    // the lane's four columns, the same in every quad it handles
    double sc4[4];
    float b4[4];
    bool col_ok[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int lc = wn + qcol + c;
      col_ok[c] = n0 + lc < N;
      sc4[c] = MODE == 1 ? s_cols[lc] : 0.0;
      b4[c] = e.bias ? e.bias[col_ok[c] ? n0 + lc : N - 1] : 0.0f;
    }
    auto quad_ptr = [&](int it) { return reinterpret_cast<v4i*>(strip + (it * RPI + qrow) * PITCH + qcol); };
    // U quads per iteration: U independent LDS / shuffle chains in flight
    // (one wave per SIMD leaves nothing else to hide their latency), each
    // step a straight-line block over the U quads.
    constexpr int U = 8;
    static_assert(NQ % U == 0, "whole groups of quads");
    static_assert(LPR == 32, "a strip row is one half of the wave (half_wave_max)");
    auto dq_values = [&](auto ic) {
      constexpr int i = decltype(ic)::value;
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) strip[((r >> 2) * 8 + kh * 4 + (r & 3)) * PITCH + 32 * j + r32] = acc[i][j][r];
#pragma unroll 1
      for (int it0 = 0; it0 < NQ; it0 += U) {
        const int trow0 = wm + 32 * i + it0 * RPI + qrow;    // tile row of quad it0 (+ RPI per quad)
        v4i a[U];
        double sr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          a[u] = *quad_ptr(it0 + u);
          sr[u] = MODE == 1 ? s_rows[trow0 + u * RPI] : 0.0;
        }
        float y[U][4];
        bool exact = true;
        if constexpr (MODE == 1) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) exact &= (unsigned)(a[u][c] + (1 << 24)) <= (2u << 24);
        }
        if (MODE == 0 || __all(exact)) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              if constexpr (MODE == 0) y[u][c] = (float)((double)a[u][c] * e.s_out);
              else y[u][c] = (float)a[u][c] * (float)(sr[u] * sc4[c]);
            }
        } else {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) y[u][c] = mul_acc_f32scale(a[u][c], (float)(sr[u] * sc4[c]));
        }
        if (e.bias) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) y[u][c] = y[u][c] + b4[c];
        }
        if (e.act == 1) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) y[u][c] = relu_js(y[u][c]);
        } else if (e.act == 2) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) y[u][c] = silu_js(y[u][c]);
        }
        // columns past N are never stored and rows past M never published,
        // so neither changes a real row's key
        int k[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          k[u] = -1;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int kc = col_ok[c] ? absmax_key(y[u][c]) : -1;
            k[u] = kc > k[u] ? kc : k[u];
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) k[u] = half_wave_max(k[u]);
        if (lane % LPR == LPR - 1) {
#pragma unroll
          for (int u = 0; u < U; ++u) atomicMax(&tkey[trow0 + u * RPI], k[u]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
          *quad_ptr(it0 + u) = v4i{__float_as_int(y[u][0]), __float_as_int(y[u][1]), __float_as_int(y[u][2]),
                                   __float_as_int(y[u][3])};
      }
#pragma unroll
      for (int it = 0; it < NQ; ++it) {
        const v4i v = *quad_ptr(it);
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[i][(4 * it + c) >> 4][(4 * it + c) & 15] = v[c];
      }
    };
    dq_values(std::integral_constant<int, 0>{});
    if constexpr (C::TM > 1) dq_values(std::integral_constant<int, 1>{});
    if constexpr (C::TM > 2) dq_values(std::integral_constant<int, 2>{});
    if constexpr (C::TM > 3) dq_values(std::integral_constant<int, 3>{});
    static_assert(C::TM <= 4 && C::TN * 16 == 4 * NQ, "dq_values covers TM <= 4; a strip is NQ quads per lane");
    __syncthreads();
    // Publication of the tile's row keys, then the grid-wide meeting.
    // Ordering argument:
    //  1. each publishing lane's agent-scope fetch_max is followed by that
    //     lane's own agent-scope release fence, which waits until the
    //     wave's atomics are performed at the device-coherent level
    //     (vmcnt(0)) -- a workgroup barrier alone does not: its release is
    //     workgroup-scoped and waits only for LDS traffic, so waves 1-3
    //     could still have their atomics in flight;
    //  2. the workgroup barrier then orders every wave's fence before
    //     thread 0's release increment of the arrival counter;
    //  3. a workgroup that sees the counter reach nwg (relaxed polls: an
    //     acquire per poll would invalidate this XCD's L2 each time) runs
    //     one agent-scope acquire fence before reading any key, so it sees
    //     every key published before every increment it counted.
    if (tid < rows_a && tkey[tid] >= 0)
      __hip_atomic_fetch_max(&e.row_keys[m0 + tid], tkey[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (tid == 0) {
      __hip_atomic_fetch_add(e.sync, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
      int polls = 0;
      while (__hip_atomic_load(e.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (unsigned)e.nwg) {
        if (++polls > e.spin_limit) {
          __hip_atomic_store(e.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    __syncthreads();
    if (tid < BM) {
      const int key = tid < rows_a
                          ? __hip_atomic_load(&e.row_keys[m0 + tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                          : -1;
      const double s = scale_from_key(key);
      rscale[tid] = s;
      rrcp[tid] = fast_scale_ok(s) ? (float)(1.0 / s) : __builtin_nanf("");
      if (tn == 0 && tid < rows_a) e.q_scales[m0 + tid] = s;
    }
    __syncthreads();
    int8_t* o8 = static_cast<int8_t*>(out);
    auto dq_store = [&](auto ic) {
      constexpr int i = decltype(ic)::value;
#pragma unroll
      for (int it = 0; it < NQ; ++it) {
        v4i v;
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = acc[i][(4 * it + c) >> 4][(4 * it + c) & 15];
        *quad_ptr(it) = v;
      }
#pragma unroll 1
      for (int it0 = 0; it0 < NQ; it0 += U) {
        const int trow0 = wm + 32 * i + it0 * RPI + qrow;
        float f[U][4];
        float rcp[U];
        double sc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const v4i v = *quad_ptr(it0 + u);
#pragma unroll
          for (int c = 0; c < 4; ++c) f[u][c] = __int_as_float(v[c]);
          rcp[u] = rrcp[trow0 + u * RPI];
          sc[u] = rscale[trow0 + u * RPI];
        }
        // the f32 decision for every value; a NaN reciprocal (scale outside
        // the fast path's range) flags all of its row's values
        int code[U][4];
        bool bad[U][4];
        bool any_bad = false;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            code[u][c] = quant_sym_try(f[u][c], rcp[u], bad[u][c]);
            any_bad |= bad[u][c];
          }
        if (__any(any_bad)) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (bad[u][c]) code[u][c] = quant_exact(f[u][c], sc[u], 0.0, -128, 127);
        }
        if (interior) {
#pragma unroll
          for (int u = 0; u < U; ++u)
            *reinterpret_cast<int*>(o8 + (m0 + trow0 + u * RPI) * (int64_t)N + gcol) =
                pack4(code[u][0], code[u][1], code[u][2], code[u][3]);
        } else {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int64_t row = m0 + trow0 + u * RPI;
            if (row < M) {
#pragma unroll
              for (int c = 0; c < 4; ++c)
                if (gcol + c < N) o8[row * N + gcol + c] = (int8_t)code[u][c];
            }
          }
        }
      }
    };
    dq_store(std::integral_constant<int, 0>{});
    if constexpr (C::TM > 1) dq_store(std::integral_constant<int, 1>{});
    if constexpr (C::TM > 2) dq_store(std::integral_constant<int, 2>{});
    if constexpr (C::TM > 3) dq_store(std::integral_constant<int, 3>{});
  } else if constexpr (P::OUT_Q8 || (!OUT_I32 && P::ACT == 2)) {
    // Static requant (int8 out) and fp32 out with SiLU: per strip the
    // accumulators go to the wave's LDS strip, then a rolled loop over the
    // lane's 4-column quads (one row each) applies the epilogue (scales,
    // bias, activation) and stores the quad: as fp32 values, or quantized
    // with the next layer's static scale (the f32 decision for every value,
    // the exact path only where it is needed) as 4 codes.  Rolled for the
    // reason given for the dynamic path: written in the accumulator layout,
    // with the exact-path, SiLU and exact-quantize code inlined for each of
    // the 256 values a lane holds, the int8 kernel's code is ~500 KB and the
    // 4096^3 GEMM takes 117 us instead of 64.
    double sc4[4];
    float b4[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int lc = wn + qcol + c;
      sc4[c] = MODE == 1 ? s_cols[lc] : 0.0;
      b4[c] = e.bias ? e.bias[n0 + lc < N ? n0 + lc : N - 1] : 0.0f;
    }
    static_assert(64 % LPR == 0, "whole strip rows per lane set");
    auto quad_ptr = [&](int it) { return reinterpret_cast<const v4i*>(strip + (it * RPI + qrow) * PITCH + qcol); };
    int8_t* o8 = static_cast<int8_t*>(out);
    constexpr int U = 4;
    static_assert(NQ % U == 0, "whole groups of quads");
    auto q8_strip = [&](auto ic) {
      constexpr int i = decltype(ic)::value;
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) strip[((r >> 2) * 8 + kh * 4 + (r & 3)) * PITCH + 32 * j + r32] = acc[i][j][r];
#pragma unroll 1
      for (int it0 = 0; it0 < NQ; it0 += U) {
        const int trow0 = wm + 32 * i + it0 * RPI + qrow;    // tile row of quad it0 (+ RPI per quad)
        v4i a[U];
        double sr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          a[u] = *quad_ptr(it0 + u);
          sr[u] = MODE == 1 ? s_rows[trow0 + u * RPI] : 0.0;
        }
        float y[U][4];
        bool exact = true;
        if constexpr (MODE == 1) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) exact &= (unsigned)(a[u][c] + (1 << 24)) <= (2u << 24);
        }
        if (MODE == 0 || __all(exact)) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              if constexpr (MODE == 0) y[u][c] = (float)((double)a[u][c] * e.s_out);
              else y[u][c] = (float)a[u][c] * (float)(sr[u] * sc4[c]);
            }
        } else {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) y[u][c] = mul_acc_f32scale(a[u][c], (float)(sr[u] * sc4[c]));
        }
        // int8 out: bias and activation from the runtime epilogue; fp32 out:
        // the variant's bias bit, then SiLU
        if (P::OUT_Q8 ? e.bias != nullptr : P::BIAS) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) y[u][c] = y[u][c] + b4[c];
        }
        if (P::OUT_Q8 && e.act == 1) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) y[u][c] = relu_js(y[u][c]);
        } else if (!P::OUT_Q8 || e.act == 2) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c) y[u][c] = silu_js(y[u][c]);
        }
        if constexpr (!P::OUT_Q8) {
          float* of = static_cast<float*>(out);
          if (interior) {
#pragma unroll
            for (int u = 0; u < U; ++u)
              __builtin_nontemporal_store(
                  v4i{__float_as_int(y[u][0]), __float_as_int(y[u][1]), __float_as_int(y[u][2]),
                      __float_as_int(y[u][3])},
                  reinterpret_cast<v4i*>(of + (m0 + trow0 + u * RPI) * (int64_t)N + gcol));
          } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
              const int64_t row = m0 + trow0 + u * RPI;
              if (row < M) {
#pragma unroll
                for (int c = 0; c < 4; ++c)
                  if (gcol + c < N) of[row * N + gcol + c] = y[u][c];
              }
            }
          }
          continue;
        }
        // requant(y, e), with the exact quantize taken out of the straight line
        int code[U][4];
        bool bad[U][4];
        bool any_bad = false;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            if (e.q_fast) {
              code[u][c] = quant_sym_try(y[u][c], e.rq32, bad[u][c]);
            } else {
              code[u][c] = 0;
              bad[u][c] = true;
            }
            any_bad |= bad[u][c];
          }
        if (__any(any_bad)) {
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int c = 0; c < 4; ++c)
              if (bad[u][c]) code[u][c] = quant_exact(y[u][c], e.s_q, 0.0, -128, 127);
        }
        if (interior) {
#pragma unroll
          for (int u = 0; u < U; ++u)
            __builtin_nontemporal_store(pack4(code[u][0], code[u][1], code[u][2], code[u][3]),
                                        reinterpret_cast<int*>(o8 + (m0 + trow0 + u * RPI) * (int64_t)N + gcol));
        } else {
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int64_t row = m0 + trow0 + u * RPI;
            if (row < M) {
#pragma unroll
              for (int c = 0; c < 4; ++c)
                if (gcol + c < N) o8[row * N + gcol + c] = (int8_t)code[u][c];
            }
          }
        }
      }
    };
    q8_strip(std::integral_constant<int, 0>{});
    if constexpr (C::TM > 1) q8_strip(std::integral_constant<int, 1>{});
    if constexpr (C::TM > 2) q8_strip(std::integral_constant<int, 2>{});
    if constexpr (C::TM > 3) q8_strip(std::integral_constant<int, 3>{});
    static_assert(C::TM <= 4, "q8_strip calls cover TM <= 4");
  } else {
    strip_out(std::integral_constant<int, 0>{});
    if constexpr (C::TM > 1) strip_out(std::integral_constant<int, 1>{});
    if constexpr (C::TM > 2) strip_out(std::integral_constant<int, 2>{});
    if constexpr (C::TM > 3) strip_out(std::integral_constant<int, 3>{});
    static_assert(C::TM <= 4, "strip_out calls cover TM <= 4");
  }
}

template <int BM, int BN>
constexpr int qgemm_lds() { return GemmCfg<BM, BN>::LDS_TOTAL; }

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
  store_out(out, idx, (int)s, m, n, e);
}

#define Q8_EPI_CODES(X) \
  X(16) X(0) X(1) X(2) X(4) X(5) X(6) X(8) X(9) X(10) X(12) X(13) X(14) X(32) X(40) X(128) X(144)

// The 256 x 192 tile (three 32-column blocks per wave; a strip row of 96
// columns): the plain fp32 and int32 epilogues only -- the rolled epilogues
// (int8 out, SiLU, dynamic requant, GLU) assume whole strip rows per 64 lanes.
#define Q8_EPI_CODES_192(X) X(16) X(0) X(1) X(4) X(5) X(8) X(9) X(12) X(13)

static bool epi_192_ok(const GemmEpi& e) {
  switch (epi_code(e)) {
#define Q8_CASE(code) case code:
    Q8_EPI_CODES_192(Q8_CASE)
#undef Q8_CASE
    return true;
    default:
      return false;
  }
}

template <int BM, int BN>
static hipError_t launch_qgemm_tile(const int8_t* A, const int8_t* B, int M, int N, int K,
                                    const GemmEpi& e, void* out, hipStream_t st) {
  const int tm = (M + BM - 1) / BM, tn = (N + BN - 1) / BN;
  const dim3 grid((unsigned)(tm * tn)), block(GEMM_THREADS);
  constexpr int lds = qgemm_lds<BM, BN>();
#define Q8_LAUNCH_EPI(code)                                                                  \
  case code:                                                                                 \
    hipLaunchKernelGGL((k_qgemm<BM, BN, code>), grid, block, lds, st, A, B, M, N, K, tm, tn, \
                       e, out);                                                              \
    break;
  if constexpr (BN == 192) {
    switch (epi_code(e)) {
      Q8_EPI_CODES_192(Q8_LAUNCH_EPI)
      default:
        return hipErrorInvalidValue;
    }
  } else {
    switch (epi_code(e)) {
      Q8_EPI_CODES(Q8_LAUNCH_EPI)
      default:
        return hipErrorInvalidValue;
    }
  }
#undef Q8_LAUNCH_EPI
  return hipGetLastError();
}

// Implicit conv GEMM (B a conv frame): column-blocked i32 and per-tensor f32
// dequant outputs, and the raw row-major partial sums of a K split, on the
// tiles whose register budget has room for the per-column frame offsets.
#define Q8_EPI_CODES_CONV(X) X(272) X(384) X(400)   // 272: a split's raw partial sums

std::atomic<long long> g_generic_gemm_launches{0};

// Tile choice by a fill-aware cost of the launch's rounds.  A tile shape
// has `slots` workgroups resident at once (CUs x the workgroups per CU its
// LDS allows: 1 for 256x256 and 256x128, 2 for 128x128, 4 for 64x64); a
// round of it costs tmin + (tfull - tmin) * fill, fill = its tiles / slots
// (a partial round is cheaper but not free).  The constants are
// microseconds at K = 4096, fitted to measurements of every shape on M in
// 256..4096 x N in 2048..22016 (they pick the fastest tile on all 56); K
// scales every shape alike, so it does not enter the choice.  Two resident
// 128x128 workgroups per CU overlap one's epilogue with the other's main
// loop, which is why they win many mid-size shapes.  256x192 (the plain
// epilogues only; allowed bit 4) fits N = 6144 / 12288 in whole rounds
// where 256x256 leaves half a round: 9% less work per second than 256x256
// but no idle half round (fitted on eleven shapes, M 1024..4096 x N
// 4096..22016: C4's QKV 110.6 -> 103.5 us, 4096 x 6144 110.5 -> 102.3 us;
// the rule keeps the fastest tile on all eleven).  Returns the index of the
// chosen tile in cands.
static int gemm_tile_choice(int64_t M, int64_t N, unsigned allowed = 0xF) {
  struct Cand { int bm, bn, per_cu; double tmin, tfull; };
  const Cand cands[] = {{256, 256, 1, 44.0, 63.0}, {256, 128, 1, 27.5, 40.0},
                        {128, 128, 2, 19.0, 36.0}, {64, 64, 4, 9.0, 28.0},
                        {256, 192, 1, 44.0, 51.5}};
  const int cus = cu_count() > 0 ? cu_count() : 256;
  int best = 0;
  double best_cost = 1e300;
  for (int c = 0; c < 5; ++c) {
    if (!((allowed >> c) & 1u)) continue;
    const int64_t tiles = ((M + cands[c].bm - 1) / cands[c].bm) * ((N + cands[c].bn - 1) / cands[c].bn);
    const int64_t slots = (int64_t)cus * cands[c].per_cu;
    const int64_t full = tiles / slots, rest = tiles % slots;
    double cost = (double)full * cands[c].tfull;
    if (rest) cost += cands[c].tmin + (cands[c].tfull - cands[c].tmin) * (double)rest / (double)slots;
    if (cost < best_cost * 0.995) { best_cost = cost; best = c; }   // near ties keep the larger tile
  }
  return best;
}

ConvGemmPlan conv_gemm_plan(int64_t M, int64_t N, int64_t K, size_t part_cap_bytes) {
  // Measured on ResNet-style layers at batch 32: with few tiles per CU the
  // K loop is bound by load latency, which four resident 64x64 workgroups
  // per CU hide better than two 128x128 ones; with two or more 64x64 tiles
  // per CU the 64x64 tile is bound by its L2 traffic (64 operations per
  // staged byte) and 128x128 (128 per byte) is faster.
  const int64_t cus = cu_count() > 0 ? cu_count() : 256;
  const int64_t tiles64 = ((M + 63) / 64) * ((N + 63) / 64);
  ConvGemmPlan p;
  p.bm = M >= 128 && tiles64 >= 2 * cus ? 128 : 64;
  const int64_t tiles = ((M + p.bm - 1) / p.bm) * ((N + p.bm - 1) / p.bm);
  const int64_t KT = (K + BK - 1) / BK;
  // Split only when the tiles leave CUs idle and K is long: the partial
  // sums cost 8 * splits bytes of traffic per output element, against
  // 2 * K operations.  Aim at two workgroups per CU, 8 stages per split.
  int64_t splits = 1;
  if (tiles < cus && K >= 4096) {
    splits = (2 * cus + tiles - 1) / tiles;
    splits = splits < 8 ? splits : 8;
    splits = splits < KT / 8 ? splits : KT / 8;
    splits = splits > 1 ? splits : 1;
  }
  while (splits > 1 && (size_t)splits * (size_t)M * (size_t)N * 4 > part_cap_bytes) --splits;
  p.kps = (int)((KT + splits - 1) / splits);
  p.splits = (int)((KT + p.kps - 1) / p.kps);   // no empty split
  return p;
}

// Sum of the splits' partial sums, stored with the column-blocked mapping
// and output kind of e (int32, or fround(acc * s_out) as the GEMM epilogue).
// Row m = blockIdx.y (+ multiples of gridDim.y); a thread takes 4
// consecutive columns.  M * N < 2^31 (split plans only go to small outputs).
__global__ __launch_bounds__(256) void k_conv_splitk_finish(const int32_t* __restrict__ part, int splits,
                                                            int M, int N, GemmEpi e,
                                                            void* __restrict__ out) {
  const int j0 = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (j0 >= N) return;
  const int cb = (int)e.col_blk;
  const int nj = N - j0 < 4 ? N - j0 : 4;
  const bool vec = (N & 3) == 0;   // 16-byte rows of partial sums
  const int blk0 = j0 / cb, p0 = j0 - blk0 * cb;
  for (int m = blockIdx.y; m < M; m += gridDim.y) {
    uint32_t acc[4] = {0u, 0u, 0u, 0u};
    const int32_t* src = part + (int64_t)m * N + j0;
    // at most 8 splits: unrolled, so that their loads are in flight together
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (s < splits) {
        const int32_t* ps = src + (int64_t)s * M * N;
        if (vec) {
          const v4i v = *reinterpret_cast<const v4i*>(ps);
#pragma unroll
          for (int c = 0; c < 4; ++c) acc[c] += (uint32_t)v[c];
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (c < nj) acc[c] += (uint32_t)ps[c];
        }
      }
    }
    int blk = blk0, p = p0;
    int64_t at = (int64_t)blk * e.blk_stride + (int64_t)m * e.ld_out + p;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if (c < nj) {
        if (e.out_i32) static_cast<int32_t*>(out)[at] = (int32_t)acc[c];
        else static_cast<float*>(out)[at] = (float)((double)(int32_t)acc[c] * e.s_out);
      }
      ++at;
      if (++p == cb) {   // next image's block
        p = 0;
        ++blk;
        at = (int64_t)blk * e.blk_stride + (int64_t)m * e.ld_out;
      }
    }
  }
}

hipError_t launch_gemm_conv(const int8_t* A, const int8_t* frame, int64_t M, int64_t N, int64_t K,
                            const GemmEpi& e, const ConvGemmPlan& plan, int32_t* part, void* out,
                            hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  const int64_t KT = (K + BK - 1) / BK;
  if (K % 64 != 0 || K <= 0 || K > 16384 || (e.cb.Cg % 64) != 0 || e.col_blk <= 0 || M > INT32_MAX ||
      N > INT32_MAX || ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(frame)) & 15) != 0 ||
      plan.splits < 1 || plan.splits > 8 || plan.kps < 1 || (int64_t)plan.splits * plan.kps < KT ||
      (plan.splits > 1 && (part == nullptr || (reinterpret_cast<uintptr_t>(part) & 15) != 0 ||
                           M * N >= ((int64_t)1 << 31))) ||
      (plan.bm != 64 && plan.bm != 128))
    return hipErrorInvalidValue;
  GemmEpi eg = e;
  eg.cb.kps = (uint32_t)(plan.splits > 1 ? plan.kps : KT);
  void* dst = out;
  if (plan.splits > 1) {   // raw partial sums, row-major [M, N] per split
    eg.col_blk = 0;
    eg.out_i32 = 1;
    dst = part;
  }
  const int tm = (int)((M + plan.bm - 1) / plan.bm), tn = (int)((N + plan.bm - 1) / plan.bm);
  if ((int64_t)tm * tn * plan.splits >= ((int64_t)1 << 31) / GEMM_THREADS) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(tm * tn * plan.splits)), block(GEMM_THREADS);
  const int code = epi_code(eg) | 256;
  hipError_t err = hipErrorInvalidValue;
  constexpr int lds128 = qgemm_lds<128, 128>(), lds64 = qgemm_lds<64, 64>();
#define Q8_CONV_LAUNCH(BMV, codev)                                                                \
  if (plan.bm == BMV && code == codev) {                                                          \
    hipLaunchKernelGGL((k_qgemm<BMV, BMV, codev>), grid, block, BMV == 128 ? lds128 : lds64, st, A, \
                       frame, (int)M, (int)N, (int)K, tm, tn, eg, dst);                           \
    err = hipGetLastError();                                                                      \
  }
#define Q8_CONV_LAUNCH_BOTH(codev) Q8_CONV_LAUNCH(128, codev) Q8_CONV_LAUNCH(64, codev)
  Q8_EPI_CODES_CONV(Q8_CONV_LAUNCH_BOTH)
#undef Q8_CONV_LAUNCH_BOTH
#undef Q8_CONV_LAUNCH
  if (err != hipSuccess || plan.splits == 1) return err;
  const unsigned gy = (unsigned)(M < 65535 ? M : 65535);
  hipLaunchKernelGGL(k_conv_splitk_finish, dim3((unsigned)((N + 1023) / 1024), gy), dim3(256), 0, st,
                     part, plan.splits, (int)M, (int)N, e, out);
  return hipGetLastError();
}

hipError_t launch_gemm(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                       const GemmEpi& e, void* out, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  // The MFMA kernel needs 16-byte K chunks and 32-bit buffer offsets within
  // a 256-row tile (offsets up to 256 * K, plus the OOB marker 2^31).
  const bool vec = (K % 16 == 0) && K > 0 && (256 * K < (int64_t)OOB) &&
                   ((reinterpret_cast<uintptr_t>(A) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(B) & 15) == 0);
  if (!vec) {
    const int64_t n = M * N;
    g_generic_gemm_launches.fetch_add(1, std::memory_order_relaxed);
    hipLaunchKernelGGL(k_gemm_i8_generic, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       A, B, (int)M, (int)N, (int)K, e, out);
    return hipGetLastError();
  }
  switch (gemm_tile_choice(M, N, epi_192_ok(e) ? 0x1Fu : 0xFu)) {
    case 0: return launch_qgemm_tile<256, 256>(A, B, (int)M, (int)N, (int)K, e, out, st);
    case 1: return launch_qgemm_tile<256, 128>(A, B, (int)M, (int)N, (int)K, e, out, st);
    case 2: return launch_qgemm_tile<128, 128>(A, B, (int)M, (int)N, (int)K, e, out, st);
    case 4: return launch_qgemm_tile<256, 192>(A, B, (int)M, (int)N, (int)K, e, out, st);
    default: return launch_qgemm_tile<64, 64>(A, B, (int)M, (int)N, (int)K, e, out, st);
  }
}

// ------------------------------------------------------------------ gate|up GEMM (GLU)
// One output element h[m, f] per thread for the shapes the MFMA kernel does
// not take (K % 16 != 0, unaligned operands): the gate and up dot products of
// feature f over the interleaved weight, then the same arithmetic as the
// MFMA epilogue.
__global__ __launch_bounds__(256) void k_glu_generic(const int8_t* __restrict__ A,
                                                     const int8_t* __restrict__ B, int M, int F, int K,
                                                     GemmEpi e, float* __restrict__ h) {
  const int64_t idx = blockIdx.x * 256LL + threadIdx.x;
  if (idx >= (int64_t)M * F) return;
  const int64_t m = idx / F, f = idx % F;
  const int64_t pg = 64 * (f / 32) + f % 32, pu = pg + 32;
  uint32_t sg = 0, su = 0;
  for (int k = 0; k < K; ++k) {
    sg += (uint32_t)((int)A[m * K + k] * (int)B[pg * K + k]);
    su += (uint32_t)((int)A[m * K + k] * (int)B[pu * K + k]);
  }
  GemmEpi en = e;
  en.act = 0;
  const float g = epi_value((int)sg, m, pg, en), u = epi_value((int)su, m, pu, en);
  h[idx] = silu_js(g) * u;
}

// h from the epilogue values of the interleaved columns ([M, 2F], bias
// already added): h[m, f] = fround(silu(y[m, pg]) * y[m, pg + 32]).
__global__ __launch_bounds__(256) void k_glu_combine(const float* __restrict__ y, int64_t M, int64_t F,
                                                     float* __restrict__ h) {
  const int64_t idx = blockIdx.x * 256LL + threadIdx.x;
  if (idx >= M * F) return;
  const int64_t m = idx / F, f = idx % F;
  const int64_t pg = 64 * (f / 32) + f % 32;
  const float* row = y + m * 2 * F;
  h[idx] = silu_js(row[pg]) * row[pg + 32];
}

// Interleave per-channel packed gate and up weights (and their scales, and
// optionally biases) into the layout of the GLU GEMM: packed row 64 g + c is
// gate row 32 g + c, 64 g + 32 + c is up row 32 g + c.  F % 32 == 0.
__global__ __launch_bounds__(256) void k_glu_interleave(const int8_t* __restrict__ Wg,
                                                        const int8_t* __restrict__ Wu, int64_t F,
                                                        int64_t K, int8_t* __restrict__ W) {
  // one 16-byte chunk per thread (K % 16 == 0, 16-byte aligned rows)
  const int64_t per_row = K / 16;
  const int64_t total = 2 * F * per_row;
  for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t pr = i / per_row, c = i % per_row;
    const int64_t g = pr / 64, w = pr % 64;
    const int8_t* src = (w < 32 ? Wg : Wu) + (32 * g + (w & 31)) * K;
    *reinterpret_cast<v4i*>(W + pr * K + 16 * c) = *reinterpret_cast<const v4i*>(src + 16 * c);
  }
}

__global__ __launch_bounds__(256) void k_glu_interleave_bytes(const int8_t* __restrict__ Wg,
                                                              const int8_t* __restrict__ Wu, int64_t F,
                                                              int64_t K, int8_t* __restrict__ W) {
  const int64_t total = 2 * F * K;
  for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    const int64_t pr = i / K, c = i % K;
    const int64_t g = pr / 64, w = pr % 64;
    W[i] = ((w < 32 ? Wg : Wu) + (32 * g + (w & 31)) * K)[c];
  }
}

__global__ __launch_bounds__(256) void k_glu_interleave_vec(const double* __restrict__ sg,
                                                            const double* __restrict__ su,
                                                            const float* __restrict__ bg,
                                                            const float* __restrict__ bu, int64_t F,
                                                            double* __restrict__ s, float* __restrict__ b) {
  const int64_t pr = blockIdx.x * 256LL + threadIdx.x;
  if (pr >= 2 * F) return;
  const int64_t g = pr / 64, w = pr % 64, f = 32 * g + (w & 31);
  s[pr] = w < 32 ? sg[f] : su[f];
  if (b) b[pr] = w < 32 ? bg[f] : bu[f];
}

hipError_t launch_glu_interleave(const int8_t* Wg, const int8_t* Wu, const double* sg, const double* su,
                                 const float* bg, const float* bu, int64_t F, int64_t K, int8_t* W,
                                 double* s, float* b, hipStream_t st) {
  if (F == 0) return hipSuccess;
  const bool vec = (K % 16) == 0 && ((reinterpret_cast<uintptr_t>(Wg) | reinterpret_cast<uintptr_t>(Wu) |
                                      reinterpret_cast<uintptr_t>(W)) & 15) == 0;
  if (K > 0) {
    if (vec) {
      const int64_t total = 2 * F * (K / 16);
      const unsigned g = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
      hipLaunchKernelGGL(k_glu_interleave, dim3(g), dim3(256), 0, st, Wg, Wu, F, K, W);
    } else {
      // byte copies: the same kernel with K seen as not a multiple of 16
      const int64_t total = 2 * F * K;
      const unsigned g = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
      hipLaunchKernelGGL(k_glu_interleave_bytes, dim3(g), dim3(256), 0, st, Wg, Wu, F, K, W);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  hipLaunchKernelGGL(k_glu_interleave_vec, dim3((unsigned)((2 * F + 255) / 256)), dim3(256), 0, st, sg, su,
                     bg, bu, F, s, b);
  return hipGetLastError();
}

size_t gemm_glu_ws_bytes(int64_t M, int64_t F, int64_t K) {
  (void)K;
  return M <= 16 ? (size_t)((M * 2 * F * 4 + 255) / 256 * 256) : 0;
}

hipError_t launch_gemm_glu(const int8_t* A, const int8_t* B, int64_t M, int64_t F, int64_t K,
                           const GemmEpi& e, float* h, void* ws, hipStream_t st) {
  if (M == 0 || F == 0) return hipSuccess;
  const int64_t N = 2 * F;
  if (M <= 16) {
    // decode: the GEMV's epilogue values of the interleaved columns into the
    // workspace, then h from pairs of them
    float* y = static_cast<float*>(ws);
    hipError_t err = launch_gemv(A, B, M, N, K, e, y, st);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(k_glu_combine, dim3((unsigned)((M * F + 255) / 256)), dim3(256), 0, st, y, M, F, h);
    return hipGetLastError();
  }
  GemmEpi eg = e;
  eg.act = 0;
  const bool vec = (K % 16 == 0) && K > 0 && (256 * K < (int64_t)OOB) &&
                   ((reinterpret_cast<uintptr_t>(A) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(B) & 15) == 0);
  if (!vec) {
    g_generic_gemm_launches.fetch_add(1, std::memory_order_relaxed);
    hipLaunchKernelGGL(k_glu_generic, dim3((unsigned)((M * F + 255) / 256)), dim3(256), 0, st, A, B, (int)M,
                       (int)F, (int)K, eg, h);
    return hipGetLastError();
  }
  // 256 x 256 or 128 x 128: the 64 x 64 tile has one 32-column block per
  // wave (no gate/up pairs), and the cost model picks 256 x 128 for no
  // shape of interest
  const int c = gemm_tile_choice(M, N, 0x5u);
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
  switch (c) {
    case 0: {
      const int tm = (Mi + 255) / 256, tn = (Ni + 255) / 256;
      constexpr unsigned lds = (unsigned)qgemm_lds<256, 256>();
      hipLaunchKernelGGL((k_qgemm<256, 256, 520>), dim3((unsigned)(tm * tn)), dim3(GEMM_THREADS), lds, st, A,
                         B, Mi, Ni, Ki, tm, tn, eg, (void*)h);
      break;
    }
    default: {
      const int tm = (Mi + 127) / 128, tn = (Ni + 127) / 128;
      constexpr unsigned lds = (unsigned)qgemm_lds<128, 128>();
      hipLaunchKernelGGL((k_qgemm<128, 128, 520>), dim3((unsigned)(tm * tn)), dim3(GEMM_THREADS), lds, st, A,
                         B, Mi, Ni, Ki, tm, tn, eg, (void*)h);
      break;
    }
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------ dynamic requant GEMM
// Workspace: [M] int32 row keys (rounded up to 256 bytes), then the arrival
// counter and the status word.
size_t gemm_dq_ws_bytes(int64_t M) { return (size_t)((M * 4 + 255) / 256 * 256) + 256; }

__global__ void k_dq_init(int* keys, int64_t M, unsigned* sync, int* status) {
  for (int64_t i = blockIdx.x * 256LL + threadIdx.x; i < M; i += (int64_t)gridDim.x * 256) keys[i] = -1;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    *sync = 0u;
    *status = 0;
  }
}

// Workgroups of the 256 x 256 dynamic-requant kernel that fit the chip at
// once (one per CU at its LDS size), cached per device.
static int dq_capacity() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int c = cache[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)k_qgemm<256, 256, 72>,
                                                     GEMM_THREADS, qgemm_lds<256, 256>()) != hipSuccess)
      per_cu = 0;
    c = per_cu * cu_count();
    cache[dev].store(c > 0 ? c : -1, std::memory_order_relaxed);
  }
  return c > 0 ? c : 0;
}

bool gemm_dq_fits(int64_t M, int64_t N) {
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
  return tiles <= dq_capacity();
}

// Test hook (q8_debug_dq_force_timeout): while set, the arrival count a
// launch waits for is one more than its workgroups, so every wait runs out
// after a few polls and the status word reports it (the kernel still ends
// normally; its output is then unreliable).
std::atomic<int> g_dq_force_timeout{0};

hipError_t launch_gemm_dq(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                          GemmEpi e, int8_t* out, double* scales, void* ws, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  const int tm = (int)((M + 255) / 256), tn = (int)((N + 255) / 256);
  const int nwg = tm * tn;
  if (nwg > dq_capacity()) return hipErrorCooperativeLaunchTooLarge;
  char* w = static_cast<char*>(ws);
  const size_t keys_bytes = (size_t)((M * 4 + 255) / 256 * 256);
  e.out_dq = 1;
  e.row_keys = reinterpret_cast<int*>(w);
  e.sync = reinterpret_cast<unsigned*>(w + keys_bytes);
  e.status = reinterpret_cast<int*>(w + keys_bytes + 4);
  e.q_scales = scales;
  e.nwg = nwg;
  e.spin_limit = 1 << 18;      // a poll is a device-coherent load (~1 us) and a short sleep: < 1 s in all
  if (g_dq_force_timeout.load(std::memory_order_relaxed)) {
    e.nwg = nwg + 1;
    e.spin_limit = 64;
  }
  const int ig = (int)((M + 255) / 256 < 1024 ? (M + 255) / 256 : 1024);
  hipLaunchKernelGGL(k_dq_init, dim3(ig), dim3(256), 0, st, e.row_keys, M, e.sync, e.status);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  // An ordinary launch.  Every workgroup needs a CU of its own (LDS) and
  // nwg <= dq_capacity(), so on a device that runs nothing else all of them
  // are dispatched at once: the kernels of one stream run one after another,
  // and the kernel before this one has ended before its first workgroup
  // starts.  Work on other streams or processes can hold CUs for a while;
  // the bounded wait then runs out instead of hanging, and the status word
  // (q8_gemm_requant_dynamic_status) reports it.  A cooperative launch
  // would guarantee co-residency instead, at ~20 us per call on MI355X (the
  // fused O projection of C4: 121 vs 101 us), which is more than the
  // fusion saves.
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
  constexpr unsigned lds = (unsigned)qgemm_lds<256, 256>();
  if (e.mode == 1)
    hipLaunchKernelGGL((k_qgemm<256, 256, 72>), dim3((unsigned)nwg), dim3(GEMM_THREADS), lds, st, A, B, Mi,
                       Ni, Ki, tm, tn, e, (void*)out);
  else
    hipLaunchKernelGGL((k_qgemm<256, 256, 64>), dim3((unsigned)nwg), dim3(GEMM_THREADS), lds, st, A, B, Mi,
                       Ni, Ki, tm, tn, e, (void*)out);
  return hipGetLastError();
}

// ------------------------------------------------------------------ GEMV (M <= 16)
// Sum of value a[lane >> (6 - log2 V)] over the 64 lanes of the wave, for
// V values per lane (V a power of two <= 64): each halving step trades the
// half of the values a lane gives away with its partner (lane ^ OFF), so V
// totals cost V - 1 shuffles instead of 6 V.  Written as compile-time
// recursion so every array index is a constant (the values stay in VGPRs).
template <int N, int OFF>
__device__ __forceinline__ void butterfly_step(int* a, int lane) {
  if constexpr (OFF >= 1) {
    if constexpr (N > 1) {
      constexpr int H = N / 2;
      const bool up = (lane & OFF) != 0;
#pragma unroll
      for (int i = 0; i < H; ++i) {
        const int give = up ? a[i] : a[i + H];
        const int keep = up ? a[i + H] : a[i];
        a[i] = keep + __shfl_xor(give, OFF, 64);
      }
      butterfly_step<H, OFF / 2>(a, lane);
    } else {
      a[0] += __shfl_xor(a[0], OFF, 64);
      butterfly_step<1, OFF / 2>(a, lane);
    }
  }
}

template <int V>
__device__ __forceinline__ int wave_butterfly_sum(int (&a)[V], int lane) {
  static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "power of two <= 64");
  butterfly_step<V, 32>(a, lane);
  return a[0];
}

// ---- dot4 GEMV, M <= 4 tokens.  One workgroup (4 waves) per group of
// GV_ROWS = 4 weight rows.  K is cut into 16-byte chunks spread over all
// 256 lanes (CPT chunks per lane), so every load instruction of a wave
// reads 1 KiB of one weight row, and a lane's activation chunks for all MT
// tokens stay in registers for the group.  Small groups and many
// workgroups keep the load ramp short and the reduction tail of each
// workgroup small (measured against 16-row groups, which re-read the
// activations 4x less but ran slower at every M <= 4).  All weight loads
// of a group are issued before the first dot product.  Partial dot products
// (v_dot4_i32_i8) are reduced across the wave by a butterfly and across the
// 4 waves through a small LDS array; lanes of wave 0 apply the epilogue.
constexpr int GV_ROWS = 4;

template <int MT, int CPT>
__global__ __launch_bounds__(256)
void k_gemv_i8(const int8_t* __restrict__ A, const int8_t* __restrict__ B, int M, int N, int K,
               GemmEpi e, void* __restrict__ out) {
  constexpr int V = GV_ROWS * MT;
  static_assert(V <= 64, "butterfly width");
  __shared__ int red[4][V];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int C = K >> 4;                                // 16-byte chunks per row
  const int n0 = blockIdx.x * GV_ROWS;

  // Buffer loads, every one issued unconditionally: the weight resource
  // starts at row n0 and ends after the group's last row, the activation
  // resource ends after token M - 1, and chunks past the row end take an
  // offset past num_records -- all of those read zero.
  const uint32_t rows = (uint32_t)min(GV_ROWS, N - n0);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(B + (int64_t)n0 * K, rows * (uint32_t)K);
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (uint32_t)M * (uint32_t)K);
  v4i w[GV_ROWS][CPT];
#pragma unroll
  for (int r = 0; r < GV_ROWS; ++r)
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int ch = tid + 256 * c;
      const uint32_t off = ch < C ? (uint32_t)r * (uint32_t)K + 16u * (uint32_t)ch : OOB;
      w[r][c] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rb, off, 0, 2));
    }
  v4i xa[CPT][MT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int ch = tid + 256 * c;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      const uint32_t off = ch < C ? (uint32_t)m * (uint32_t)K + 16u * (uint32_t)ch : OOB;
      xa[c][m] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0));
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  int acc[V];
#pragma unroll
  for (int r = 0; r < GV_ROWS; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      int a = 0;
#pragma unroll
      for (int c = 0; c < CPT; ++c) {
        a = __builtin_amdgcn_sdot4(xa[c][m].x, w[r][c].x, a, false);
        a = __builtin_amdgcn_sdot4(xa[c][m].y, w[r][c].y, a, false);
        a = __builtin_amdgcn_sdot4(xa[c][m].z, w[r][c].z, a, false);
        a = __builtin_amdgcn_sdot4(xa[c][m].w, w[r][c].w, a, false);
      }
      acc[r * MT + m] = a;
    }
  const int total = wave_butterfly_sum<V>(acc, lane);
  constexpr int SHIFT = V == 64 ? 0 : V == 32 ? 1 : V == 16 ? 2 : V == 8 ? 3 : V == 4 ? 4 : 5;
  if ((lane & ((1 << SHIFT) - 1)) == 0) red[wave][lane >> SHIFT] = total;
  __syncthreads();
  if (tid < V) {
    // lanes of one token write consecutive outputs: tid -> (token, row)
    const int m = tid / GV_ROWS, r = tid % GV_ROWS, n = n0 + r, i = r * MT + m;
    if (m < M && n < N) {
      // int32 wrap-around sum, as the reference's Int32Array store
      const int s = (int)((uint32_t)red[0][i] + (uint32_t)red[1][i] + (uint32_t)red[2][i] +
                          (uint32_t)red[3][i]);
      store_out(out, (int64_t)m * N + n, s, m, n, e);
    }
  }
}

// ---- Fused dynamic qlinear for one-token decode (K <= 4096): the per-token
// (or per-tensor) int8 quantize of the fp32 activations and the dot4 GEMV
// in one kernel.  Every workgroup reads the whole activation row (16 fp32
// elements per lane; cached, it is the same for all workgroups), takes its
// absmax key (wave max, then LDS across the 4 waves), derives the scale and
// codes with the same functions as q8_quantize_rows -- so codes and scale
// are identical to that kernel's -- and goes on as k_gemv_i8 with R weight
// rows per workgroup.  One launch and one dependent memory round trip less
// than quantize + GEMV.  The template also takes MT <= 4 tokens; only
// MT = 1 is launched (the quantize repeated per workgroup grows with MT).
// R1's exact form, symmetric int8 -- out of line: it runs only for
// near-ties (and non-normal scales), and inlining it at each of a lane's
// 16 x MT elements would multiply the kernel's code size.
__device__ __noinline__ int quant_exact_sym_call(float x, double s) {
  return quant_exact(x, s, 0.0, -128, 127);
}

// quant4_sym with the exact path out of line.
__device__ __forceinline__ int quant4_sym_call(v4f v, bool fast, float r32, double s) {
  if (fast) {
    bool b0, b1, b2, b3;
    int c0 = quant_sym_try(v.x, r32, b0), c1 = quant_sym_try(v.y, r32, b1);
    int c2 = quant_sym_try(v.z, r32, b2), c3 = quant_sym_try(v.w, r32, b3);
    if (b0 | b1 | b2 | b3) {
      if (b0) c0 = quant_exact_sym_call(v.x, s);
      if (b1) c1 = quant_exact_sym_call(v.y, s);
      if (b2) c2 = quant_exact_sym_call(v.z, s);
      if (b3) c3 = quant_exact_sym_call(v.w, s);
    }
    return pack4(c0, c1, c2, c3);
  }
  return pack4(quant_exact_sym_call(v.x, s), quant_exact_sym_call(v.y, s),
               quant_exact_sym_call(v.z, s), quant_exact_sym_call(v.w, s));
}

template <int MT, int R>
__global__ __launch_bounds__(256)
void k_qlinear_dot4(const float* __restrict__ x, int M, int K, int per_tensor,
                    const int8_t* __restrict__ W, const double* __restrict__ sW, int sW_stride,
                    int N, const float* __restrict__ bias, int act, float* __restrict__ y,
                    double* __restrict__ sx_out, int8_t* __restrict__ xq_out) {
  constexpr int V = R * MT;
  static_assert(V <= 64, "butterfly width");
  __shared__ int kred[4][MT];
  __shared__ int red[4][V];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int C = K >> 4;                               // 16-element chunks per row (<= 256)
  const bool live = tid < C;                          // this lane's chunk exists
  const int n0 = blockIdx.x * R;

  // activations first (the reduction needs them first), then the weights,
  // then the epilogue operands; every load issued before any arithmetic
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x), (short)0, (int)((uint32_t)M * (uint32_t)K * 4u),
                                        0x00020000);
  v4f xv[MT][4];
#pragma unroll
  for (int m = 0; m < MT; ++m)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t off = (live && m < M) ? ((uint32_t)m * (uint32_t)K + 16u * (uint32_t)tid) * 4u + 16u * j : OOB;
      xv[m][j] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
    }
  const uint32_t rows = (uint32_t)min(R, N - n0);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(W + (int64_t)n0 * K, rows * (uint32_t)K);
  v4i w[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t off = live ? (uint32_t)r * (uint32_t)K + 16u * (uint32_t)tid : OOB;
    w[r] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 2));
  }
  // output lane tid < V finishes (token tid / R, row n0 + tid % R)
  const int om = tid / R, on = n0 + tid % R;
  const bool out_lane = tid < V && om < M && on < N;
  const double sw = out_lane ? sW[(int64_t)on * sW_stride] : 0.0;
  const float bv = (out_lane && bias) ? bias[on] : 0.0f;
  __builtin_amdgcn_sched_barrier(0);

  // absmax keys: -1 (no value) for absent chunks and tokens
  int key[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    int k = -1;
    if (live && m < M) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kj = key4(make_float4(xv[m][j].x, xv[m][j].y, xv[m][j].z, xv[m][j].w));
        k = k > kj ? k : kj;
      }
    }
    key[m] = wave_max_i32(k);
  }
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < MT; ++m) kred[wave][m] = key[m];
  }
  __syncthreads();
  int kt = -1;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    int k = kred[0][m];
#pragma unroll
    for (int v = 1; v < 4; ++v) k = k > kred[v][m] ? k : kred[v][m];
    key[m] = k;
    if (m < M) kt = kt > k ? kt : k;
  }
  // scales and codes (q8_quantize_rows' arithmetic)
  double s[MT];
  v4i xa[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    s[m] = scale_from_key(per_tensor ? kt : key[m]);
    const bool fast = fast_scale_ok(s[m]);
    const float r32 = (float)(1.0 / s[m]);
    int c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      c[j] = quant4_sym_call(xv[m][j], fast, r32, s[m]);
    xa[m] = v4i{c[0], c[1], c[2], c[3]};
    if (xq_out && blockIdx.x == 0 && live && m < M)
      *reinterpret_cast<v4i*>(xq_out + (int64_t)m * K + 16 * tid) = xa[m];
  }
  if (sx_out && blockIdx.x == 0 && tid < (per_tensor ? 1 : M)) {
    double v = s[0];
#pragma unroll
    for (int m = 1; m < MT; ++m)
      if (tid == m) v = s[m];
    sx_out[tid] = v;
  }
  int acc[V];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      int a = 0;
      a = __builtin_amdgcn_sdot4(xa[m].x, w[r].x, a, false);
      a = __builtin_amdgcn_sdot4(xa[m].y, w[r].y, a, false);
      a = __builtin_amdgcn_sdot4(xa[m].z, w[r].z, a, false);
      a = __builtin_amdgcn_sdot4(xa[m].w, w[r].w, a, false);
      acc[r * MT + m] = a;
    }
  const int total = wave_butterfly_sum<V>(acc, lane);
  constexpr int SHIFT = V == 64 ? 0 : V == 32 ? 1 : V == 16 ? 2 : V == 8 ? 3 : V == 4 ? 4 : 5;
  if ((lane & ((1 << SHIFT) - 1)) == 0) red[wave][lane >> SHIFT] = total;
  __syncthreads();
  if (out_lane) {
    const int i = (tid % R) * MT + om;
    const int a = (int)((uint32_t)red[0][i] + (uint32_t)red[1][i] + (uint32_t)red[2][i] +
                        (uint32_t)red[3][i]);
    double sm = s[0];
#pragma unroll
    for (int m = 1; m < MT; ++m)
      if (om == m) sm = s[m];
    // E-rowcol: fround(acc * fround(sx[m] * sW[n])), then bias and activation
    float v = mul_acc_f32scale(a, (float)(sm * sw));
    if (bias) v = v + bv;
    if (act == 1) v = relu_js(v);
    else if (act == 2) v = silu_js(v);
    y[(int64_t)om * N + on] = v;
  }
}

// ---- MFMA GEMV, 4 < M <= 16 tokens.  At 16 tokens a v_dot4 kernel spends
// 64 VALU instructions per 16 weight bytes per lane and stops being
// HBM-bound; one v_mfma_i32_16x16x64_i8 does the same work for 16 weight
// rows x 64 K-bytes x all 16 tokens.  Weights are the A operand (lane l:
// row l%16, K bytes 16*(l/16) of each 64-byte block), the tokens the B
// operand in the same lane layout (rows >= M zero), so both operands
// pair the same K bytes.  The workgroup's NW waves split each pass over K
// into NW slices of KB 64-byte blocks; each wave keeps its activation
// fragments in registers for all the weight-row blocks it visits
// (grid-stride over blocks of 16 rows), and the NW partial 16x16 results
// meet in LDS (double-buffered: one barrier per block).  Output element (row n0 + 4*(l/16) + r, token l%16)
// is accumulator r of lane l.  NW = 4: at most 168 VGPRs (3 waves per
// SIMD), so 3 workgroups per CU are resident (K < 4096).  NW = 16 (KB = 4):
// a 1024-lane workgroup, each wave a sixteenth of K with 32 VGPRs of
// operands; one per row block while the blocks fit the CUs, else one per CU
// walking several row blocks (N = 11008, M = 16: 14.8 -> 13.3 us against
// three 4-wave workgroups per CU, unstaged).
template <int KB, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW == 4 ? 3 : 4)))
void k_gemv_mfma(const int8_t* __restrict__ A, const int8_t* __restrict__ B, int M, int N, int K,
                 GemmEpi e, void* __restrict__ out) {
  __shared__ int red[2][NW][256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const int nblk = (N + 15) >> 4;
  const int passes = (K + 64 * NW * KB - 1) / (64 * NW * KB);  // K bytes per pass: NW x KB x 64
  // Buffer loads: offsets past num_records return zeros.  Activation
  // chunks past K are masked explicitly (zeros); weight chunks past K then
  // only ever meet zero activations, so they need no mask.
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (uint32_t)M * (uint32_t)K);
  v4i xf[KB];
  auto load_x = [&](int pass) {
    const int kw = pass * 64 * NW * KB + wave * 64 * KB + 16 * g;
    const uint32_t xrow = r16 < M ? (uint32_t)(r16 * K) : OOB;
#pragma unroll
    for (int j = 0; j < KB; ++j) {
      const int k = kw + 64 * j;
      const uint32_t off = k < K ? xrow + (uint32_t)k : OOB;   // OOB + k stays past num_records
      xf[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0));
    }
  };
  // Weight fragments.  Fragment j of lane (g, r16) is K chunk 4 j + g (16
  // bytes) of the wave's K slice of row r16, as the activation fragments.
  // Loaded straight into that layout, each load instruction reads 64 bytes
  // of each of 16 rows.  The staged forms instead copy the wave's 16 rows x
  // 64 KB bytes into LDS (direct-to-LDS buffer loads), 4 rows x 256
  // contiguous bytes per instruction, then read the fragments from LDS.
  // The slice is kept as KB / 4 regions of 16 rows x 256 bytes; in a
  // region, row r's chunk c sits in slot c ^ r, so a row still arrives as
  // one contiguous run and the 16 lanes of a fragment read fall in 16
  // different bank groups.  Each wave reads back only its own copies (its
  // vmcnt, no barrier).  Staged where the copies fit beside the workgroups
  // a CU holds: 16 waves (one per CU, 64 KiB) and 4 waves with KB <= 8
  // (three per CU, up to 32 KiB each); N = 11008, M = 16: 13.3 -> 12.4 us.
  constexpr bool STAGE = (NW == 16 && KB == 4) || (NW == 4 && KB <= 8);
  __shared__ __align__(16) int8_t wst[STAGE ? NW * KB * 1024 : 16];
  auto load_w = [&](v4i* w, const __amdgpu_buffer_rsrc_t& rw, uint32_t kpass) {
    if constexpr (STAGE) {
      int8_t* base = wst + KB * 1024 * __builtin_amdgcn_readfirstlane(wave);
      const int rl = lane >> 4, q = lane & 15;
      // the previous fragment reads from this region have returned
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int h = 0; h < KB / 4; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int row = 4 * j + rl;
          copy16_to_lds(rw, base + 4096 * h + 1024 * j,
                        (uint32_t)(row * K) + kpass + (uint32_t)(wave * 64 * KB + 256 * h + 16 * (q ^ row)));
        }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int j = 0; j < KB; ++j) {
        const int c = 4 * j + g;
        w[j] = *reinterpret_cast<const v4i*>(base + 4096 * (c >> 4) + 256 * r16 + 16 * ((c & 15) ^ r16));
      }
    } else {
      const uint32_t wo = (uint32_t)(r16 * K) + kpass + (uint32_t)(wave * 64 * KB + 16 * g);
#pragma unroll
      for (int j = 0; j < KB; ++j)
        w[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, wo + 64 * j, 0, 0));
    }
  };
  if constexpr (KB <= 8) {
    if (passes == 1 && (int)gridDim.x >= nblk) {
      // One pass covers K and every workgroup has one row block: straight
      // line, the activation and weight loads issued together before the
      // first MFMA (0.3-0.5 us less than the block loop below on the same
      // launch at N = 4096, K = 1024..4096).  With several blocks per
      // workgroup the loop below stays: walking balanced row ranges, or
      // issuing the next block's weights before this block's MFMAs, was
      // slower there (N = 11008, M <= 8: 12.0 -> 12.5-13.5 us).
      load_x(0);
      const int n0 = (int)blockIdx.x * 16;
      const int rows = N - n0 < 16 ? N - n0 : 16;
      const __amdgpu_buffer_rsrc_t rw = make_rsrc(B + (int64_t)n0 * K, (uint32_t)rows * (uint32_t)K);
      v4i w[KB];
      load_w(w, rw, 0u);
      __builtin_amdgcn_sched_barrier(0);
      v4i acc = {0, 0, 0, 0}, acc2 = {0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < KB; j += 2) {
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[j], xf[j], acc, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[j + 1], xf[j + 1], acc2, 0, 0, 0);
      }
      acc += acc2;
#pragma unroll
      for (int r = 0; r < 4; ++r) red[0][wave][r16 * 16 + 4 * g + r] = acc[r];
      __syncthreads();
      const int t = tid >> 4, i = tid & 15, n = n0 + i;
      if (tid < 256 && t < M && n < N) {
        uint32_t su = 0;
#pragma unroll
        for (int w2 = 0; w2 < NW; ++w2) su += (uint32_t)red[0][w2][tid];
        store_out(out, (int64_t)t * N + n, (int)su, t, n, e);
      }
      return;
    }
  }
  if (passes == 1) load_x(0);
  int rb = 0;
  for (int blk = blockIdx.x; blk < nblk; blk += gridDim.x, rb ^= 1) {
    const int n0 = blk * 16;
    const int rows = N - n0 < 16 ? N - n0 : 16;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(B + (int64_t)n0 * K, (uint32_t)rows * (uint32_t)K);
    v4i acc = {0, 0, 0, 0}, acc2 = {0, 0, 0, 0};     // two chains of dependent MFMAs
    for (int pass = 0; pass < passes; ++pass) {
      if (passes > 1) load_x(pass);
      v4i w[KB];
      load_w(w, rw, (uint32_t)(pass * 64 * NW * KB));
      // all KB weight loads in flight before the first MFMA waits on one
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < KB; j += 2) {
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[j], xf[j], acc, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[j + 1], xf[j + 1], acc2, 0, 0, 0);
      }
    }
    acc += acc2;   // int32 wrap-around sums: exact in any order
    // token-major: red[.][t * 16 + i] holds (token t, row i) of this block
#pragma unroll
    for (int r = 0; r < 4; ++r) red[rb][wave][r16 * 16 + 4 * g + r] = acc[r];
    __syncthreads();
    const int t = tid >> 4, i = tid & 15, n = n0 + i;
    if (tid < 256 && t < M && n < N) {
      uint32_t su = 0;
#pragma unroll
      for (int w = 0; w < NW; ++w) su += (uint32_t)red[rb][w][tid];
      store_out(out, (int64_t)t * N + n, (int)su, t, n, e);
    }
  }
}

template <int MT>
static hipError_t launch_gemv_mt(const int8_t* A, const int8_t* B, int M, int N, int K,
                                 const GemmEpi& e, void* out, hipStream_t st) {
  const dim3 grid((unsigned)((N + GV_ROWS - 1) / GV_ROWS)), block(256);
  const int cpt = (K / 16 + 255) / 256;               // <= 2 (K <= 8192)
  if (cpt <= 1)
    hipLaunchKernelGGL((k_gemv_i8<MT, 1>), grid, block, 0, st, A, B, M, N, K, e, out);
  else
    hipLaunchKernelGGL((k_gemv_i8<MT, 2>), grid, block, 0, st, A, B, M, N, K, e, out);
  return hipGetLastError();
}

static hipError_t launch_gemv_mfma(const int8_t* A, const int8_t* B, int M, int N, int K,
                                   const GemmEpi& e, void* out, hipStream_t st) {
  // K >= 4096 (one pass of 16 waves x 4 x 64 bytes covers 4096): one
  // 16-wave workgroup per row block while the blocks fit the CUs, else one
  // per CU walking several blocks.  With its weights staged through LDS
  // this form beats two 8-wave workgroups per CU (unstaged: they would not
  // fit their copies beside each other) at every token count: N = 11008,
  // M = 8: 12.2 -> 11.6 us; N = 14336: 16.1 -> 14.6 us.
  const int nblk = (N + 15) / 16;
  const int cus = cu_count() > 0 ? cu_count() : 256;
  if (K >= 4096) {
    hipLaunchKernelGGL((k_gemv_mfma<4, 16>), dim3((unsigned)(nblk < cus ? nblk : cus)), dim3(1024), 0, st,
                       A, B, M, N, K, e, out);
    return hipGetLastError();
  }
  // every workgroup resident at once (3 per CU): weight loads of all row
  // blocks are in flight together
  const int cap = 3 * cu_count();
  const dim3 grid((unsigned)(nblk < cap ? nblk : cap)), block(256);
  if (K <= 1024)
    hipLaunchKernelGGL((k_gemv_mfma<4, 4>), grid, block, 0, st, A, B, M, N, K, e, out);
  else if (K <= 2048)
    hipLaunchKernelGGL((k_gemv_mfma<8, 4>), grid, block, 0, st, A, B, M, N, K, e, out);
  else
    hipLaunchKernelGGL((k_gemv_mfma<16, 4>), grid, block, 0, st, A, B, M, N, K, e, out);
  return hipGetLastError();
}

hipError_t launch_gemv(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                       const GemmEpi& e, void* out, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  // 16-byte chunks and aligned rows, else the GEMM kernels (which handle
  // any M).  The dot4 kernel keeps 16 weight rows of K <= 2 * 256 * 16
  // bytes in registers; the MFMA kernel walks any K in passes.
  const bool vec = (K % 16 == 0) && K > 0 && K < (int64_t)1 << 30 &&
                   ((reinterpret_cast<uintptr_t>(A) & 15) == 0) &&
                   ((reinterpret_cast<uintptr_t>(B) & 15) == 0);
  if (!vec) return launch_gemm(A, B, M, N, K, e, out, st);
  if (M > 4 || K > 8192) {
    if (16 * K >= (int64_t)OOB) return launch_gemm(A, B, M, N, K, e, out, st);
    return launch_gemv_mfma(A, B, (int)M, (int)N, (int)K, e, out, st);
  }
  if (M <= 1) return launch_gemv_mt<1>(A, B, (int)M, (int)N, (int)K, e, out, st);
  if (M <= 2) return launch_gemv_mt<2>(A, B, (int)M, (int)N, (int)K, e, out, st);
  return launch_gemv_mt<4>(A, B, (int)M, (int)N, (int)K, e, out, st);
}

bool qlinear_fused_ok(const float* x, const int8_t* W, int64_t M, int64_t K) {
  return M == 1 && K >= 16 && K <= 4096 && K % 16 == 0 &&
         (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(W) & 15) == 0;
}

hipError_t launch_qlinear_fused(const float* x, int64_t M, int64_t K, int per_tensor,
                                const int8_t* W, const double* sW, int sW_stride, int64_t N,
                                const float* bias, int act, float* y, double* sx_out,
                                int8_t* xq_out, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
#define Q8_QLF(MT, R)                                                                            \
  hipLaunchKernelGGL((k_qlinear_dot4<MT, R>), dim3((unsigned)((N + (R)-1) / (R))), dim3(256), 0, \
                     st, x, (int)M, (int)K, per_tensor, W, sW, sW_stride, (int)N, bias, act, y,   \
                     sx_out, xq_out)
  // one token: 16 weight rows per workgroup (measured against 4, 8, 32 and
  // 64: fewer, larger workgroups repeat the quantize less often but stream
  // fewer rows at once).  With more tokens the quantize repeated in every
  // workgroup costs more than the launch it saves, so M > 1 runs as two
  // kernels (see qlinear_fused_ok).
  Q8_QLF(1, 16);
#undef Q8_QLF
  return hipGetLastError();
}

hipError_t setup_kernel_attributes() {
  hipError_t err;
#define Q8_SET_LDS(kern, bytes)                                                              \
  err = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),                             \
                            hipFuncAttributeMaxDynamicSharedMemorySize, (bytes));            \
  if (err != hipSuccess) return err;
#define Q8_SET_256(code) Q8_SET_LDS((k_qgemm<256, 256, code>), (qgemm_lds<256, 256>()));
#define Q8_SET_256x128(code) Q8_SET_LDS((k_qgemm<256, 128, code>), (qgemm_lds<256, 128>()));
#define Q8_SET_128(code) Q8_SET_LDS((k_qgemm<128, 128, code>), (qgemm_lds<128, 128>()));
#define Q8_SET_64(code) Q8_SET_LDS((k_qgemm<64, 64, code>), (qgemm_lds<64, 64>()));
#define Q8_SET_256x192(code) Q8_SET_LDS((k_qgemm<256, 192, code>), (qgemm_lds<256, 192>()));
  Q8_EPI_CODES_192(Q8_SET_256x192)
  Q8_EPI_CODES(Q8_SET_256)
  Q8_EPI_CODES(Q8_SET_256x128)
  Q8_EPI_CODES(Q8_SET_128)
  Q8_EPI_CODES(Q8_SET_64)
  Q8_SET_256(64)
  Q8_SET_256(72)
  Q8_SET_256(520)
  Q8_SET_128(520)
  Q8_EPI_CODES_CONV(Q8_SET_128)
  Q8_EPI_CODES_CONV(Q8_SET_64)
#undef Q8_SET_256
#undef Q8_SET_256x128
#undef Q8_SET_256x192
#undef Q8_SET_128
#undef Q8_SET_64
#undef Q8_SET_LDS
  return hipSuccess;
}

}  // namespace q8
