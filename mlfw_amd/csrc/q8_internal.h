// q8_internal.h -- launchers shared between the kernel files and the C ABI.
// Every launcher assumes its arguments were validated by q8_capi.hip and
// returns the hipError_t of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/q8hip.h"

namespace q8 {

// Epilogue description passed by value to the GEMM / GEMV kernels.
struct GemmEpi {
  const double* sA;     // per-row (stride 1) or scalar (stride 0); ROWCOL only
  const double* sB;     // per-column (stride 1) or scalar (stride 0); ROWCOL only
  int64_t sA_stride;
  int64_t sB_stride;
  double s_out;         // PT only
  const float* bias;    // may be null
  int mode;             // 0 = PT, 1 = ROWCOL
  int act;              // 0 none, 1 relu, 2 silu
  int out_i32;          // 1: write the raw int32 accumulator
  int out_q8;           // 1: requantize the fp32 result to int8 with the static scale s_q
  double s_q;           // next layer's quantize scale (out_q8)
  float rq32;           // (float)(1 / s_q), for the f32 fast path of R1
  int q_fast;           // s_q admits the fast path (normal, in [2^-100, 2^100])
  // out_dq: the fp32 value is requantized per row with the row's own
  // absmax scale (q8_gemm_requant_dynamic).  All workgroups are co-resident
  // (one per CU, no more than the chip holds): each publishes its rows'
  // absmax keys, they meet once grid-wide (a bounded wait), then quantize
  // the values they still hold.
  int out_dq;
  int* row_keys;        // [M] absmax keys, -1 at launch
  unsigned* sync;       // arrival counter, 0 at launch
  int* status;          // set to 1 if the bounded wait ran out
  double* q_scales;     // [M] row scales, written by the tiles of column 0
  int nwg;              // workgroups of the launch
  int spin_limit;       // bound of the wait (polls)
  // column-blocked output (quantized_conv over a batch of images): GEMM
  // column j is position j % col_blk of image j / col_blk, and element
  // (row, j) is stored at (j / col_blk) * blk_stride + row * ld_out +
  // j % col_blk.  col_blk = 0: plain row-major [M, N].
  // GLU output (q8_gemm_glu): 1 stores h with plain stores (kept in the
  // caches for the quantize that reads it next), 0 non-temporal
  int h_plain;
  int64_t col_blk;
  int64_t blk_stride;
  int64_t ld_out;
  // implicit-GEMM B operand of quantized_conv (EPI bit 256): B is the
  // channel-last frame of a batch of images.  GEMM column j is output
  // position p = j % Pn of image y = j / Pn, and its contraction byte
  // k = t * Cg + c (tap t, channel c) is frame byte
  // (y * Ep + e(p) + off(t)) * Cg + c, e(p) the frame position of p's tap 0
  // and off(t) that of tap t relative to it.  All offsets fit 31 bits.
  struct ConvB {
    uint32_t Pn, P1, P2;       // positions per image; output sizes of dims 1, 2
    uint32_t st0, st1, st2;    // strides
    uint32_t E1, E2;           // frame sizes of dims 1, 2
    uint32_t Ep, Cg;           // frame positions per image; channels, a multiple of 64
    uint32_t K1, K2, Kn;       // kernel sizes of dims 1, 2; kernel positions
    uint32_t dl0, dl1, dl2;    // dilations
    uint32_t frame_bytes;      // bytes of the batch's frames
    uint32_t kps;              // K stages per split (split-K), >= all stages for one split
  } cb;
};

// GEMM of quantized_conv's implicit form: A [M, K] (tap-major weight rows),
// B the frames described by e.cb (N = images x Pn columns), column-blocked
// output as set in e.  K a multiple of 64, at most 16384.  The plan picks
// the tile and a split of K when the tiles alone would leave most of the
// chip idle; the splits' int32 partial sums go to `part` (splits * M * N
// words) and a finishing pass adds them (int32 addition does not depend on
// the order) and applies the output mapping and dequant.
struct ConvGemmPlan {
  int bm;       // square tile edge, 128 or 64
  int splits;   // K splits, >= 1
  int kps;      // K stages (of 128) per split
};
ConvGemmPlan conv_gemm_plan(int64_t M, int64_t N, int64_t K, size_t part_cap_bytes);
hipError_t launch_gemm_conv(const int8_t* A, const int8_t* frame, int64_t M, int64_t N, int64_t K,
                            const GemmEpi& e, const ConvGemmPlan& plan, int32_t* part, void* out,
                            hipStream_t st);

hipError_t launch_fill_normal(float* out, int64_t n, uint32_t seed, uint64_t offset,
                              double mean, double std, hipStream_t st);
hipError_t launch_fill_uniform(float* out, int64_t n, uint32_t seed, uint64_t offset,
                               double a, double b, hipStream_t st);
hipError_t launch_apply_outliers(float* x, int64_t n, uint32_t seed, double p, double factor,
                                 hipStream_t st);
hipError_t launch_quant_static(const float* x, int64_t n, double s, double zp, int is_u8,
                               void* q, hipStream_t st);
// x rows start ldx floats apart (K for a contiguous input)
hipError_t launch_quant_rows(const float* x, int64_t ldx, int64_t M, int64_t K, int8_t* q,
                             double* scales, hipStream_t st);
// per-tensor dynamic quantize; its reduction key lives in scales[0]
hipError_t launch_quant_tensor(const float* x, int64_t n, int8_t* q, double* scales,
                               hipStream_t st);
hipError_t launch_dequant(const void* q, int src, int64_t M, int64_t K, const double* scales,
                          int per_row, double zp, float* y, hipStream_t st);
hipError_t launch_pack_weight(const float* W, int64_t rows, int64_t cols, int axis,
                              int per_tensor, int8_t* Wq, double* scales, hipStream_t st);
// g and u rows start ldg / ldu floats apart (K for contiguous inputs)
hipError_t launch_silu_mul_quant_rows(const float* g, int64_t ldg, const float* u, int64_t ldu,
                                      int64_t M, int64_t K, float* h, int8_t* q, double* scales,
                                      hipStream_t st);
// launches of the generic (non-MFMA) GEMM kernel, for q8_generic_gemm_launches
extern std::atomic<long long> g_generic_gemm_launches;
hipError_t launch_gemm(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                       const GemmEpi& e, void* out, hipStream_t st);
// GEMM with the dynamic per-row requant epilogue (e.out_dq fields filled by
// the caller except the meeting point, which comes from `ws`).  Returns
// hipErrorCooperativeLaunchTooLarge when the tiles do not fit the chip at
// once; gemm_dq_fits tells beforehand.  g_dq_force_timeout (test hook) makes
// every launch's grid-wide wait run out.
extern std::atomic<int> g_dq_force_timeout;
// q8_ewise's route (q8_debug_ewise_jit): 0 by size, 1 interpreter, 2 compiled;
// programs compiled and compiled launches so far
extern std::atomic<int> g_ewise_jit_mode;
extern std::atomic<long long> g_ewise_jit_compiled, g_ewise_jit_launches;
// Copies why the last failed ewise compile failed into buf (truncated,
// NUL-terminated; "" if none has) and returns the message's full length.
size_t ewise_jit_error(char* buf, size_t cap);
bool gemm_dq_fits(int64_t M, int64_t N);
size_t gemm_dq_ws_bytes(int64_t M);
hipError_t launch_gemm_dq(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                          GemmEpi e, int8_t* out, double* scales, void* ws, hipStream_t st);
hipError_t launch_gemv(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                       const GemmEpi& e, void* out, hipStream_t st);
// Gate|up GEMM with h = fround(silu(g) * u) fused (B interleaved by
// launch_glu_interleave; e in MODE 1, bias in the interleaved order or null).
// M <= 16 needs gemm_glu_ws_bytes of workspace (the GEMV's values of the
// 2F interleaved columns), other shapes none.
hipError_t launch_glu_interleave(const int8_t* Wg, const int8_t* Wu, const double* sg, const double* su,
                                 const float* bg, const float* bu, int64_t F, int64_t K, int8_t* W,
                                 double* s, float* b, hipStream_t st);
size_t gemm_glu_ws_bytes(int64_t M, int64_t F, int64_t K);
hipError_t launch_gemm_glu(const int8_t* A, const int8_t* B, int64_t M, int64_t F, int64_t K,
                           const GemmEpi& e, float* h, void* ws, hipStream_t st);

// 4-bit per-group weights (q8_w4.hip).
hipError_t launch_pack_w4(const float* W, int64_t N, int64_t K, int64_t group, uint8_t* wq4,
                          double* scales, hipStream_t st);
// quantized_dot with zero points / ui8 operands: byte flip of a ui8
// operand into its int8 form, int8 row sums, and the rank-1 correction of
// the int32 GEMM result.
hipError_t launch_flip_u8(const uint8_t* src, int8_t* dst, int64_t n, hipStream_t st);
hipError_t launch_fill_u8(void* dst, int value, int64_t n, hipStream_t st);
hipError_t launch_row_sums_i8(const int8_t* X, int64_t rows, int64_t K, int32_t* out,
                              hipStream_t st);
hipError_t launch_zp_correct(int32_t* acc, int64_t M, int64_t N, const int32_t* rsA,
                             const int32_t* csB, int32_t cA, int32_t cB, int64_t K,
                             hipStream_t st);
// Dynamic qlinear for one-token decode in one kernel (per-token or
// per-tensor quantize of fp32 x + dot4 GEMV + E-rowcol epilogue);
// qlinear_fused_ok says whether the shape and alignment fit it.
bool qlinear_fused_ok(const float* x, const int8_t* W, int64_t M, int64_t K);
hipError_t launch_qlinear_fused(const float* x, int64_t M, int64_t K, int per_tensor,
                                const int8_t* W, const double* sW, int sW_stride, int64_t N,
                                const float* bias, int act, float* y, double* sx_out,
                                int8_t* xq_out, hipStream_t st);
hipError_t launch_gemv_w4(const int8_t* xq, const double* sx, int sx_stride, const uint8_t* wq4,
                          const double* sw, int64_t M, int64_t N, int64_t K, int64_t group,
                          const float* bias, int act, float* y, hipStream_t st);

// Geometry of a quantized_conv (NC(spatial) input, OI(spatial) kernel);
// unused trailing spatial dimensions have size 1.  Validated by the C ABI:
// every int field and Cg * prod(K) below 2^31.
struct ConvGeom {
  int d;                         // spatial rank, 1..3
  int64_t N, C, O, groups;
  int Cg, Og;                    // input / output channels per group
  int S[3], K[3], P[3];          // input, kernel, output spatial sizes
  int64_t st[3], lo[3], dl[3];   // stride, leading padding, dilation
  int64_t Sn, Pn;                // prod(S), prod(P)
  int Kn, Kc, Kc16;              // prod(K), Cg * prod(K), Kc rounded up to 16
  int zpx = 0, zpw = 0;          // input / kernel zero points
  int x_u8 = 0, w_u8 = 0;        // operands read as ui8 (else i8)
};
// Zero points and ui8 operands run the direct kernel (exact, one thread per
// output); plain i8 convs with Cg * prod(K) >= 64 run im2col + GEMM.
bool conv_direct(const ConvGeom& G);
bool conv_uses_gemm(const ConvGeom& G);
size_t conv_workspace_bytes(const ConvGeom& G);
// w_taps (may be null): the weight already in the channel-last path's
// tap-major form (launch_conv_weight_taps), which then is not permuted per call.
hipError_t launch_conv(const int8_t* x, const int8_t* w, const int8_t* w_taps, const ConvGeom& G,
                       const GemmEpi& e, void* workspace, void* out, hipStream_t st);
// Whether the tap-major weight form is used for weights of G's shape (Cg a
// multiple of 16, 2 <= prod(K) <= 1024), and the permutation that makes it:
// w_taps[o][t * Cg + c] = w[o][c][t], O * Cg * prod(K) bytes.
bool conv_taps_used(const ConvGeom& G);
hipError_t launch_conv_weight_taps(const int8_t* w, const ConvGeom& G, int8_t* w_taps, hipStream_t st);

// Calibration observer state in device memory: this header, then
// num_bins 64-bit bin counts, then num_bins words of re-bucketing scratch.
constexpr size_t Q8_OBS_HEADER = 128;
struct ObsState {
  int min_key, max_key;              // observer min / max as order keys
  int bmin_key, bmax_key;            // the current batch
  int has_hist, num_bins, initialized, mode;
  unsigned long long count;          // ValueObserver.count
  unsigned long long total_count;    // HistogramCollector.totalCount
  double range_min, range_max;       // HistogramCollector range
  double act_min, act_scale;         // range the current batch is binned with
};
static_assert(sizeof(ObsState) <= Q8_OBS_HEADER, "observer header");
__host__ __device__ inline unsigned long long* obs_bins(ObsState* st) {
  return reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(st) + Q8_OBS_HEADER);
}
__host__ __device__ inline unsigned long long* obs_scratch(ObsState* st) {
  return obs_bins(st) + st->num_bins;
}
inline size_t obs_state_bytes(int num_bins) { return Q8_OBS_HEADER + 16 * (size_t)num_bins; }

hipError_t launch_obs_reset(ObsState* st, int num_bins, int has_hist, hipStream_t s);
hipError_t launch_obs_update(ObsState* st, const float* x, int64_t n, hipStream_t s);

// One-time per-device kernel attribute set-up (dynamic LDS limits).
hipError_t setup_kernel_attributes();
hipError_t setup_w4_attributes();   // the 4-bit GEMV kernels' dynamic LDS limits

// Compute units of the current device (cached per device).
int cu_count();

// elementwise loop nests (q8_ewise.hip); q8_ew_prog comes from q8hip.h
const char* ewise_check(const q8_ew_prog& p, const int64_t* in_numel, int64_t out_numel);
hipError_t launch_ewise(const q8_ew_prog& p, const void* const* inputs, void* out, int64_t n,
                        hipStream_t st);

}  // namespace q8
