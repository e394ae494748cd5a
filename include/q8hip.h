/*
 * q8hip.h -- C ABI of the MI355X (gfx950) int8 quantized-inference library
 * (libq8hip.so).
 *
 * This is the boundary the host side binds: the Node N-API addon
 * (mlfw_amd/node/q8hip_napi.c) and the Python ctypes binding
 * (mlfw_amd/_lib.py).  Plain C types only; every device pointer is a raw
 * address in the current HIP device's memory, every `stream` is a
 * hipStream_t (NULL = the null stream).
 *
 * Reference interfaces replaced (paths relative to the slexisvn/mlfw tree):
 *   - the CUDA runtime backend's per-kernel launch path for the int8 ops,
 *     runCudaKernelSync (src/runtime/node/cuda_runtime.ts:85-121) and
 *     launchKernel (src/runtime/node/cuda/launcher.ts:34-54), which run the
 *     NVRTC-compiled kernels CUDACodegen emits for `quantize`,
 *     `quantized_dot` and `dequantize`;
 *   - the device-memory and error conventions of the reference's other
 *     native C ABI, terac (terac/include/Tera/CAPI/Execution.h:40-81:
 *     status codes, teraLastError, teraDeviceAlloc/Upload/Download).
 *
 * Conventions (all entry points):
 *   - return Q8_OK (0) on success, a Q8_ERR_* code otherwise; the message of
 *     the last failure on the calling thread is q8_last_error();
 *   - arguments are validated on the host before anything is launched; a
 *     call that fails validation launches nothing;
 *   - work is enqueued on `stream` and is asynchronous with respect to the
 *     host, except q8_h2d / q8_d2h / q8_stream_sync which block;
 *   - the arithmetic of every op is the reference CPU backend's, bit for bit
 *     (int8 codes, int32 accumulators and fp32 outputs), see each entry.
 */
#ifndef Q8HIP_H
#define Q8HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif
/* The declarations below are the library's whole export list (it is built
 * with hidden visibility by default). */
#pragma GCC visibility push(default)

#define Q8HIP_VERSION 1

/* status codes */
#define Q8_OK               0
#define Q8_ERR_INVALID      1   /* bad argument: null pointer, shape, enum, scale <= 0 */
#define Q8_ERR_DEVICE       2   /* no usable HIP device, or a HIP runtime error */
#define Q8_ERR_UNSUPPORTED  3   /* valid request this build does not implement */
#define Q8_ERR_OOM          4   /* device allocation failed */

/* element types */
#define Q8_I8   0
#define Q8_U8   1
#define Q8_I32  2
#define Q8_F32  3

/* scale granularity */
#define Q8_PER_TENSOR  0   /* one scale */
#define Q8_PER_TOKEN   1   /* one scale per row of an [M,K] tensor */
#define Q8_PER_CHANNEL 2   /* one scale per output channel (weights) */

/* epilogue forms of the GEMM */
#define Q8_EPI_PT      0   /* y = fround(acc * s_out), s_out an f64 scalar (E-pt) */
#define Q8_EPI_ROWCOL  1   /* y = fround(acc * fround(sA[m] * sB[n])) (E-pc / E-rowcol) */

/* activations applied after the optional bias */
#define Q8_ACT_NONE 0
#define Q8_ACT_RELU 1      /* Math.max(v, 0): NaN stays NaN, -0 -> +0 */
#define Q8_ACT_SILU 2      /* v * (1 / (1 + exp(-v))), every step rounded to f32 */

/* calibration modes (CalibrationResult._mode, calibration.ts:192,246-268) */
#define Q8_CALIB_MINMAX     0
#define Q8_CALIB_PERCENTILE 1   /* 99.9th percentile of the histogram, symmetric */
#define Q8_CALIB_ENTROPY    2   /* KL-divergence threshold, symmetric */

/* QuantizationScheme (src/compiler/ir/graph/quantization_types.ts:4-8) */
#define Q8_SCHEME_PER_TENSOR_SYMMETRIC  0
#define Q8_SCHEME_PER_TENSOR_ASYMMETRIC 1
#define Q8_SCHEME_PER_CHANNEL           2

#define Q8_OBS_MAX_BINS 8192    /* largest histogram an observer may keep */
#define Q8_OBS_SUMMARY  9       /* doubles written by q8_observer_read */

/* ---------------------------------------------------------------- runtime */

/* Library version (Q8HIP_VERSION). */
int q8_version(void);

/* Message of the last failed call on this thread ("" if none).
 * Mirrors teraLastError (terac/include/Tera/CAPI/Execution.h:55). */
const char* q8_last_error(void);

/* Number of HIP devices; 0 (and Q8_OK) on a machine without a GPU. */
int q8_device_count(int* count);

/* Make `device` current for this thread and prepare it (checks the device is
 * gfx950 and sets kernel attributes).  Entry points
 * below call it for the current device on first use.  Replaces the CUDA
 * backend's context/stream set-up (src/runtime/node/cuda/device.ts:14-35). */
int q8_init(int device);

/* Device memory that outlives a call: teraDeviceAlloc / Upload / Download
 * (terac/include/Tera/CAPI/Execution.h:62-81), and the reference's pooled
 * device buffers (src/runtime/node/cuda/memory.ts:92-127). */
int q8_alloc(void** dptr, size_t bytes);
int q8_free(void* dptr);
int q8_h2d(void* dst, const void* src, size_t bytes, void* stream);
int q8_d2h(void* dst, const void* src, size_t bytes, void* stream);
int q8_memset(void* dst, int value, size_t bytes, void* stream);
int q8_stream_sync(void* stream);

/* One stream for a host runtime's launches, and whole launch sequences
 * captured on it and replayed: the reference's device stream and eager
 * graphs (src/runtime/node/cuda/device.ts:14-35; cuStreamBeginCapture /
 * cuStreamEndCapture / cuGraphInstantiateWithFlags / cuGraphLaunch /
 * cuGraphExecDestroy through koffi, src/runtime/node/cuda/ffi.ts:80-84,
 * used by eager_graph.ts and the plan runner, device_plan.ts:178-218).
 * The stream has the default priority.  Capture is thread-local; while a
 * stream captures, entry points that block (q8_h2d, q8_d2h,
 * q8_stream_sync) fail on it, and launches are recorded, not run.
 * q8_graph_capture_end instantiates the captured sequence; q8_graph_launch
 * replays it on a stream (the device buffers it names must stay allocated
 * while the graph exists).  No library call records a memset node: buffers
 * that must start at zero are cleared by fill kernels. */
int q8_stream_create(void** stream);
int q8_stream_destroy(void* stream);
int q8_graph_capture_begin(void* stream);
int q8_graph_capture_end(void* stream, void** graph_exec);
int q8_graph_launch(void* graph_exec, void* stream);
int q8_graph_destroy(void* graph_exec);

/* ---------------------------------------------------------------- inputs */

/* Seeded synthetic inputs, counter-based form of mulberry32
 * (src/util/random.ts:5-14): draw i of seed s is a function of
 * s + (i + 1) * 0x6D2B79F5 alone, so the stream is generated in parallel.
 * `offset` = number of draws of the stream already consumed.
 * q8_fill_normal follows normal_ (src/nn/init.ts:40-52: Box-Muller on
 * pairs, 2*ceil(n/2) draws); q8_fill_uniform follows uniform_
 * (src/nn/init.ts:31-37, n draws). */
int q8_fill_normal(float* out, int64_t n, uint32_t seed, uint64_t offset,
                   double mean, double std, void* stream);
int q8_fill_uniform(float* out, int64_t n, uint32_t seed, uint64_t offset,
                    double a, double b, void* stream);

/* Outlier injection of the C5 quantize workload: with a second mulberry32
 * stream (seed, counter form as above, draw i for element i), every element
 * whose draw u satisfies u < p is replaced by fround(x * factor).  The
 * reference has no such generator; it defines the synthetic input only. */
int q8_apply_outliers(float* x, int64_t n, uint32_t seed, double p, double factor,
                      void* stream);

/* ---------------------------------------------------------------- quantize */

/* The compiled `quantize` op with a static scale: the CUDA kernel CUDACodegen
 * emits for the lowering of quant_math.ts:16-27 (rule
 * src/compiler/passes/lowering/rules/quantization.ts:6-12).  Bit-exact with
 * the CPU backend's form
 *   q = (Math.min(Math.max(Math.round(Math.fround(x / s)), lo), hi) | 0)
 * and, for zero_point != 0, Math.round(Math.fround(Math.fround(x/s) + zp)).
 * target Q8_I8 ([-128,127]) or Q8_U8 ([0,255]); scale must be > 0
 * (op verifier, src/compiler/ir/graph/ops/quantization.ts:44-47). */
int q8_quantize_static(const float* x, int64_t n, double scale, double zero_point,
                       int target, void* q, void* stream);

/* Dynamic symmetric int8 quantize of an [M,K] row-major fp32 tensor.
 * mode Q8_PER_TOKEN: scales[m] = S-abs of row m, mode Q8_PER_TENSOR:
 * scales[0] = S-abs of the whole tensor, where S-abs is the reference's
 * calibration scale: ValueObserver min/max (src/compiler/analysis/
 * calibration.ts:24-34, NaN never taken) fed to QuantizationParams.fromRange
 * (src/compiler/ir/graph/quantization_types.ts:248-254):
 *   s = max(|min|, |max|) / 127 || 1e-10   (f64; an empty row gets 6/127).
 * Codes are then the compiled quantize above with that scale.  The
 * reference has this scale only as a static, calibrated one; the dynamic
 * per-token / per-tensor op is this library's composition of the two.
 * scales: 8-byte aligned f64 device array of M (per token) or 1 (per
 * tensor) entries.  The per-tensor reduction keeps its running key in
 * scales[0] until the final scale replaces it, so the call uses no memory
 * besides its arguments: calls with distinct outputs may run concurrently
 * on any streams. */
int q8_quantize_rows(const float* x, int64_t M, int64_t K, int mode,
                     int8_t* q, double* scales, void* stream);

/* q8_quantize_rows with Q8_PER_TOKEN for a row-strided input: row m of x
 * starts at x + m * ldx (ldx >= K), e.g. one slice of a wider projection
 * output; q stays [M, K] contiguous.  No counterpart in the reference (its
 * tensors are contiguous); the codes and scales are those of the
 * contiguous copy. */
int q8_quantize_rows_ld(const float* x, int64_t ldx, int64_t M, int64_t K, int8_t* q,
                        double* scales, void* stream);

/* ---------------------------------------------------------------- dequantize */

/* The compiled `dequantize` op (quant_math.ts:29-34, rule
 * rules/quantization.ts:14-21): y = Math.fround((+q) * s), and for
 * zero_point != 0 y = Math.fround(Math.fround((+q) - zp) * s).
 * src: Q8_I8, Q8_U8 or Q8_I32 (the int32 form is the per-tensor GEMM
 * epilogue).  granularity Q8_PER_TENSOR uses scales[0] for all M*K
 * elements, Q8_PER_TOKEN uses scales[m] for row m.  scales: f64 device. */
int q8_dequantize(const void* q, int src, int64_t M, int64_t K,
                  const double* scales, int granularity, double zero_point,
                  float* y, void* stream);

/* ---------------------------------------------------------------- weights */

/* Host weight quantization moved to the device: QuantizationPass's
 * per-channel weight path (src/compiler/passes/quantization/
 * quantization_pass.ts:390-400) = fromConstantArrayPerChannel
 * (quantization_types.ts:299-317) + quantizeArrayPerChannel (:118-130),
 * all in f64, clamp [-128,127]; or, with granularity Q8_PER_TENSOR,
 * fromConstantArray (:287-297) + quantizeArray (:85-97), clamp [-127,127].
 * W is a row-major [rows, cols] fp32 array.  axis 0: channel = row (the
 * nn.Linear weight [N,K]); axis 1: channel = column (a [K,N] weight).
 * Output Wq is always [N, K] (channel-major, K contiguous: the GEMM's B
 * layout), i.e. W itself for axis 0 and its transpose for axis 1.
 * scales: 8-byte aligned f64 device array of N entries (per channel) or 1
 * (per tensor; its min / max keys are kept in scales[0] until the scale
 * replaces them, as in q8_quantize_rows). */
int q8_pack_weight(const float* W, int64_t rows, int64_t cols, int axis, int granularity,
                   int8_t* Wq, double* scales, void* stream);

/* ---------------------------------------------------------------- matmul */

/* quantized_dot (src/compiler/ir/graph/ops/quantization.ts:103-155, lowering
 * src/compiler/passes/lowering/rules/quantization.ts:57-76) with its
 * dequant epilogue fused:
 *   acc[m,n] = sum_k (A[m,k] - zpA) * (B[n,k] - zpB)   (int32, wraps mod 2^32
 *              exactly like the JS double accumulator stored to an Int32Array)
 * A: [M,K] int8 row-major; B: [N,K] int8 (rhs_contracting = [1], the
 * nn.Linear weight as packed by q8_pack_weight).
 * out_kind Q8_I32: out = acc (the bare quantized_dot result).
 * out_kind Q8_F32: out = act(bias + epilogue(acc)), with
 *   epi Q8_EPI_PT:     fround(acc * s_out)                 (quantization_pass.ts:335-355)
 *   epi Q8_EPI_ROWCOL: fround(acc * fround(sA[m] * sB[n])) (quantization_pass.ts:431-446;
 *                      sA_mode / sB_mode Q8_PER_TENSOR read element 0,
 *                      Q8_PER_TOKEN / Q8_PER_CHANNEL index by m / n)
 *   bias (may be NULL): fround(y + bias[n]); act: Q8_ACT_*.
 * zpA / zpB must be 0 in this build (Q8_ERR_UNSUPPORTED otherwise).
 * Routes M <= 16 to the GEMV kernel.  K % 16 != 0 or A / B not 16-byte
 * aligned take a generic one-thread-per-output kernel (exact, slow);
 * q8_generic_gemm_launches counts those launches. */
int q8_gemm(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
            int32_t zpA, int32_t zpB,
            const double* sA, int sA_mode, const double* sB, int sB_mode,
            int epi, double s_out, const float* bias, int act,
            int out_kind, void* out, void* stream);

/* The skinny (decode) form of q8_gemm for 1 <= M <= 16: same contract,
 * HBM-bound kernels that stream the weight once: packed int8 dot products
 * (v_dot4_i32_i8) for M <= 4, one 16x16x64 int8 MFMA per 16 weight rows x
 * 64 K-bytes for 4 < M <= 16. */
int q8_gemv(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
            const double* sA, int sA_mode, const double* sB, int sB_mode,
            int epi, double s_out, const float* bias, int act,
            int out_kind, void* out, void* stream);

/* Gate and up projections with the SwiGLU product fused: the reference's
 * silu(gate) * up (decomposition_pass.ts:197-230: SiLU as
 * fround(x * fround(1 / fround(1 + fround(exp(-x))))), then
 * fround(silu * up)) applied to two per-channel linears of the same input
 * (quantization_pass.ts:390-459 each), without g or u reaching memory:
 *   g[m,f] = fround(accg * fround(sA[m] * sg[f])) (+ bg[f], fround)
 *   u[m,f] = fround(accu * fround(sA[m] * su[f])) (+ bu[f], fround)
 *   h[m,f] = fround(silu(g[m,f]) * u[m,f])        h: fp32 [M, F]
 * bit for bit two q8_gemm calls and the elementwise chain.  The weights
 * come interleaved by q8_glu_interleave from two q8_pack_weight results
 * (per channel, [F,K] each): B [2F,K], packed row 64 j + c is gate row
 * 32 j + c and 64 j + 32 + c is up row 32 j + c, with the f64 scales
 * (and optional biases) in the same order; F must be a multiple of 32.
 * sB_mode must be Q8_PER_CHANNEL (2F scales) or Q8_PER_TENSOR.  M <= 16
 * runs the GEMV into a workspace of q8_gemm_glu_workspace bytes and forms
 * h from it; larger M needs none (0 bytes, workspace may be NULL).  No
 * single counterpart in the reference, whose graph runs the two linears,
 * the SiLU decomposition and the product as separate ops. */
int q8_glu_interleave(const int8_t* Wg, const double* sg, const float* bg, const int8_t* Wu,
                      const double* su, const float* bu, int64_t F, int64_t K, int8_t* W, double* s,
                      float* b, void* stream);
int q8_gemm_glu_workspace(int64_t M, int64_t F, int64_t K, size_t* bytes);
int q8_gemm_glu(const int8_t* A, const int8_t* B, int64_t M, int64_t F, int64_t K, const double* sA,
                int sA_mode, const double* sB, int sB_mode, const float* bias, float* h, void* workspace,
                size_t workspace_bytes, void* stream);

/* Launches of the generic (non-MFMA) GEMM kernel since the library was
 * loaded, over all devices and threads: q8_gemm / q8_quantized_dot calls
 * whose K is not a multiple of 16 or whose operands are not 16-byte
 * aligned.  No counterpart in the reference (its CPU kernels have one
 * path); it makes the slow route visible to callers and tests. */
int q8_generic_gemm_launches(int64_t* count);

/* quantized_dot as the reference defines it (src/compiler/ir/graph/ops/
 * quantization.ts:103-155, lowering rules/quantization.ts:23-42): operands
 * i8 or ui8 (Q8_I8 / Q8_U8: Int8Array or Uint8Array elements, the
 * verifier's QUANTIZED_INT_DTYPES), zero points, int32 output
 *   out[m,n] = ToInt32( sum_k (A[m,k] - zpA) * (B[n,k] - zpB) )
 * with B in the [N,K] layout (rhs_contracting = [1]).  The reference's
 * QuantizationPass sets non-zero zero points for affine schemes
 * (quantization_pass.ts:303-332, :415-425).  Runs the int8 GEMM / GEMV on
 * operands made signed (ui8 bytes flipped by 128) and adds the exact
 * zero-point correction from row sums; the caller passes a device
 * workspace of q8_quantized_dot_workspace bytes (0 for i8 operands with
 * zero zero points, where this is q8_gemm with Q8_I32 output). */
int q8_quantized_dot_workspace(int64_t M, int64_t N, int64_t K, int a_dtype, int b_dtype,
                               int32_t zpA, int32_t zpB, size_t* bytes);
int q8_quantized_dot(const void* A, int a_dtype, const void* B, int b_dtype, int64_t M,
                     int64_t N, int64_t K, int32_t zpA, int32_t zpB, void* workspace,
                     size_t workspace_bytes, int32_t* out, void* stream);

/* Dynamic int8 linear in one call: QuantizationPass's chain for a linear
 * (quantization_pass.ts:286-459: quantize(x) -> quantized_dot ->
 * convert -> mul(sv) [-> add bias -> max]) with the activation scale taken
 * from x itself, per token or per tensor, as q8_quantize_rows does, on an
 * nn.Linear weight (src/nn/functional/linear.ts:6-16, W [N,K] = Wq with
 * f64 scales sW, Q8_PER_CHANNEL [N] or Q8_PER_TENSOR [1]):
 *   xq, sx  = q8_quantize_rows(x, M, K, x_mode)          (written to xq, sx)
 *   out     = q8_gemm(xq, Wq, ..., Q8_EPI_ROWCOL, bias, act, Q8_F32)
 * bit for bit.  For one-token decode (M == 1, K <= 4096, K % 16 == 0,
 * 16-byte aligned x and Wq) both steps run in one kernel; otherwise as
 * two (the same kernels as the separate calls).
 * xq: int8 [M,K]; sx: 8-byte aligned f64 [M] (per token) or [1] (per
 * tensor; holds the reduction key until the scale replaces it). */
int q8_qlinear_dynamic(const float* x, int64_t M, int64_t K, int x_mode, const int8_t* Wq,
                       const double* sW, int sW_mode, int64_t N, const float* bias, int act,
                       float* out, int8_t* xq, double* sx, void* stream);

/* q8_qlinear_dynamic without caller buffers for xq / sx and without any
 * allocation.  No counterpart in the reference: this entry point is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The codes and
 * scales of x are staged in a file-scope device array of
 * Q8_NOALLOC_SCRATCH_BYTES bytes that each GPU holds until the process
 * ends; x needs round_up(M*K, 256) + 8*M bytes of it (8 for per tensor),
 * and a larger x is rejected with Q8_ERR_INVALID.  out is bit for bit that
 * of q8_qlinear_dynamic.  Every call on one GPU shares that GPU's array and
 * leaves the last call's staging in it: calls that overlap in time on one
 * GPU (two streams, or two host threads) race, so order them on one
 * stream. */
#define Q8_NOALLOC_SCRATCH_BYTES (4u << 20)
int q8_qlinear_dynamic_noalloc(const float* x, int64_t M, int64_t K, int x_mode,
                               const int8_t* Wq, const double* sW, int sW_mode, int64_t N,
                               const float* bias, int act, float* out, void* stream);

/* q8_gemm's fp32 result, requantized in the epilogue with the next layer's
 * static scale and stored as int8: QuantizationPass's calibrated chain
 * dequantize -> [add bias] -> [relu] -> quantize(s_next)
 * (quantization_pass.ts:286-360, :390-459, with the `quantize` of the
 * following dot) evaluated without the fp32 tensor ever reaching memory:
 *   out[m,n] = (Math.min(Math.max(Math.round(Math.fround(y / s_next)), -128), 127) | 0),
 *   y = act(bias + epilogue(acc)) exactly as q8_gemm's Q8_F32 output
 * (the compiled quantize, quant_math.ts:16-27, symmetric int8).  s_next is
 * a static (calibrated) scale: a dynamic per-token or per-tensor requant
 * needs the whole row's / tensor's absmax before any element is rounded,
 * which q8_quantize_rows provides as a separate pass.  Routes M <= 16 to
 * the GEMV kernels. */
int q8_gemm_requant(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                    const double* sA, int sA_mode, const double* sB, int sB_mode,
                    int epi, double s_out, const float* bias, int act,
                    double s_next, int8_t* out, void* stream);

/* q8_gemm's fp32 result requantized per row with the row's own dynamic
 * scale, as the next layer's per-token quantize would take it:
 *   y[m,n]   = act(bias + epilogue(acc))          (exactly q8_gemm's Q8_F32 output)
 *   scale[m] = S-abs of row m of y                (q8_quantize_rows, Q8_PER_TOKEN)
 *   out[m,n] = the compiled quantize of y[m,n] with scale[m]
 * bit for bit equal to q8_gemm followed by q8_quantize_rows, without the
 * fp32 tensor reaching memory when the fused route applies: every 256x256
 * tile of the MFMA GEMM is resident at once (one workgroup per CU; the route
 * is taken only when every tile has a CU), the tiles of a row block publish
 * their rows' absmax through atomics in the workspace, meet once grid-wide
 * (a bounded wait) and quantize the values they hold.  Otherwise (M <= 16, more tiles than fit the chip, K not a
 * multiple of 16) the GEMM writes y into the workspace and q8_quantize_rows
 * follows.  No counterpart in the reference, whose scales are static (it
 * composes quantization_pass.ts:390-459 with a per-token scale); the
 * reference chain it replaces is dequantize -> [add] -> [max] -> quantize.
 * q8_gemm_requant_dynamic_workspace gives the workspace bytes and whether
 * the fused route applies (it then needs 16-byte aligned A and B); calls that
 * share a workspace must be ordered.  q8_gemm_requant_dynamic_status reads
 * (synchronously) whether the fused route's bounded wait ran out; out and
 * out_scales of that call are then unreliable.  On a device that runs
 * nothing else every tile is dispatched at once and the wait cannot run out;
 * a caller that shares the device with other streams or processes (which
 * can hold CUs while the tiles wait) must check the status and, on a
 * timeout, call again or take q8_gemm + q8_quantize_rows. */
int q8_gemm_requant_dynamic_workspace(int64_t M, int64_t N, int64_t K, size_t* bytes, int* fused);
int q8_gemm_requant_dynamic(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                            const double* sA, int sA_mode, const double* sB, int sB_mode, int epi,
                            double s_out, const float* bias, int act, int8_t* out,
                            double* out_scales, void* workspace, size_t workspace_bytes,
                            void* stream);
int q8_gemm_requant_dynamic_status(const void* workspace, int64_t M, int* timed_out, void* stream);

/* Test hook, no counterpart in the reference: while `on` is non-zero every
 * fused q8_gemm_requant_dynamic launch waits for one workgroup more than it
 * has, so its bounded wait runs out and the status word reports it (the
 * kernel still ends normally).  For tests of the timeout report only. */
int q8_debug_dq_force_timeout(int on);

/* ---------------------------------------------------------------- 4-bit weights */

/* fromConstantArrayPerGroup (quantization_types.ts:319-340, numBits 4) +
 * quantizeArrayPerGroup (:143-153) of a row-major fp32 [N, K] weight over
 * its flat element order, on the device: scales[g] = absmax / 7 || 1e-10
 * (f64) for each run of group_size elements, codes
 * Math.max(-8, Math.min(7, Math.round(w / s))) (f64, NaN -> 0), packed two
 * per byte (element 2j in the low nibble, two's complement) into
 * Wq4 [N, K/2].  group_size must be even and divide K, so every group lies
 * in one row; scales has N * K / group_size entries (row n's groups at
 * n * K / group_size).  N * K / 2 must stay below 2^31 (q8_gemv_w4's
 * limit). */
int q8_pack_weight_int4(const float* W, int64_t N, int64_t K, int64_t group_size,
                        uint8_t* Wq4, double* scales, void* stream);

/* Decode-time linear with 4-bit per-group weights and int8 activations
 * (W4A8).  The reference has no op for it; it is defined as a composition
 * that stays exact:
 *   acc_g = sum over group g of xq[m,k] * q[n,k]              (int32)
 *   S     = acc_0*sw[n,0] + acc_1*sw[n,1] + ...  in f64, groups in ascending order
 *   y     = fround(S * sx[m]), then fround(y + bias[n]) and act (Q8_ACT_*)
 * xq: int8 [M, K] (q8_quantize_rows codes); sx: f64, sx_mode Q8_PER_TOKEN
 * ([M]) or Q8_PER_TENSOR ([1]); Wq4 / sw as written by q8_pack_weight_int4.
 * Kernels: packed dot products for M <= 2 (M <= 4 where K or the group
 * rule out the MFMA kernel) with a power-of-two group_size in [32, 2048]
 * and K <= 8192; the MFMA kernel for any M (blocks of 16 tokens) with K and
 * group_size multiples of 32; any other shape (a group that is not a
 * multiple of 32) runs a simple exact kernel.  All give the same bits. */
int q8_gemv_w4(const int8_t* xq, const double* sx, int sx_mode, const uint8_t* Wq4,
               const double* sw, int64_t M, int64_t N, int64_t K, int64_t group_size,
               const float* bias, int act, float* out, void* stream);

/* ---------------------------------------------------------------- conv */

/* quantized_conv (src/compiler/ir/graph/ops/quantization.ts:156-190), as
 * lowered by rules/quantization.ts:44-62 through buildConvNest
 * (src/compiler/passes/lowering/lowering_registry.ts:335-449), with the
 * per-tensor `dequantize` QuantizationPass appends to it fused
 * (quantization_pass.ts:286-360; output_scale = input_scale * kernel_scale).
 * Layouts are the op's default input_layout "NCHW" / kernel_layout "OIHW"
 * and their 1-D / 3-D forms (spatial_dims 1..3):
 *   x: int8 [N, C, S_0..S_{d-1}], w: int8 [O, C/groups, K_0..K_{d-1}],
 *   out: [N, O, P_0..P_{d-1}] with
 *   P_i = floor((S_i + pad_lo_i + pad_hi_i - ((K_i - 1) * dilation_i + 1)) / strides_i) + 1
 *   (inferConvResultTypes, src/compiler/ir/graph/ops/linalg.ts:222-248).
 * acc[n,o,p] = sum over ic < C/groups and kernel positions k of
 *   (x[n, g*C/groups + ic, p*stride + k*dilation - pad_lo] - zp_x) * (w[o, ic, k] - zp_w),
 *   g = o / (O/groups); a tap in the padding adds 0; int32 wrap-around.
 * out_kind Q8_I32: out = acc; Q8_F32: out = fround(acc * s_out).
 * Zero points (the op's input_zero_point / kernel_zero_point) run the
 * direct kernel, exact for any value.
 * workspace: device memory of at least q8_quantized_conv_workspace bytes
 * (may be 0: then NULL is accepted); calls that share a workspace must be
 * ordered (same stream). */
int q8_quantized_conv_workspace(int spatial_dims, const int64_t* x_shape, const int64_t* w_shape,
                                const int64_t* strides, const int64_t* pad_lo,
                                const int64_t* pad_hi, const int64_t* dilation, int64_t groups,
                                size_t* bytes);
int q8_quantized_conv(const int8_t* x, const int8_t* w, int spatial_dims, const int64_t* x_shape,
                      const int64_t* w_shape, const int64_t* strides, const int64_t* pad_lo,
                      const int64_t* pad_hi, const int64_t* dilation, int64_t groups,
                      int32_t zp_x, int32_t zp_w, int out_kind, double s_out, void* workspace,
                      size_t workspace_bytes, void* out, void* stream);
/* The same with the operand types: x_dtype / w_dtype Q8_I8 or Q8_U8 (the
 * lowering reads Int8Array or Uint8Array elements; the op admits mixed
 * types, ops/quantization.ts:176-178).  ui8 operands run the direct kernel. */
int q8_quantized_conv_ex(const void* x, int x_dtype, const void* w, int w_dtype, int spatial_dims,
                         const int64_t* x_shape, const int64_t* w_shape, const int64_t* strides,
                         const int64_t* pad_lo, const int64_t* pad_hi, const int64_t* dilation,
                         int64_t groups, int32_t zp_x, int32_t zp_w, int out_kind, double s_out,
                         void* workspace, size_t workspace_bytes, void* out, void* stream);

/* A conv weight prepacked once: the GEMM paths read the kernel tap-major,
 * w_taps[o][t * Cg + c] = w[o][c][t] (t the kernel position in row-major
 * order, Cg = C/groups), which q8_quantized_conv otherwise permutes on every
 * call.  The reference keeps its conv kernel as a constant buffer of the
 * compiled function (QuantizationPass quantizes it once,
 * quantization_pass.ts:286-360; ops/quantization.ts:156-190), so a weight
 * is constant across calls.  q8_conv_weight_taps writes the O * Cg *
 * prod(K) bytes for weights whose Cg is a multiple of 16 with 2..1024
 * kernel positions (Q8_ERR_UNSUPPORTED otherwise: those weights are used as
 * given); q8_quantized_conv_prepacked is q8_quantized_conv with that copy
 * (w stays an argument: paths that do not read the tap-major form use it),
 * bit for bit the same output.  16-byte aligned w and w_taps. */
int q8_conv_weight_taps(const int8_t* w, int spatial_dims, const int64_t* w_shape, int64_t groups,
                        int8_t* w_taps, void* stream);
int q8_quantized_conv_prepacked(const int8_t* x, const int8_t* w, const int8_t* w_taps, int spatial_dims,
                                const int64_t* x_shape, const int64_t* w_shape, const int64_t* strides,
                                const int64_t* pad_lo, const int64_t* pad_hi, const int64_t* dilation,
                                int64_t groups, int32_t zp_x, int32_t zp_w, int out_kind, double s_out,
                                void* workspace, size_t workspace_bytes, void* out, void* stream);

/* ---------------------------------------------------------------- fused */

/* h = fround(silu(g) * u) for the gated MLP (SiLU decomposition
 * src/compiler/passes/decompose/decomposition_pass.ts:197-203,224-230 and a
 * `mul`), followed by the per-token dynamic quantize of h (as
 * q8_quantize_rows with Q8_PER_TOKEN).  g, u: [M,K] fp32.  h_out may be
 * NULL (the fp32 h is then not written). */
int q8_silu_mul_quantize_rows(const float* g, const float* u, int64_t M, int64_t K,
                              float* h_out, int8_t* q, double* scales, void* stream);

/* As q8_silu_mul_quantize_rows, with g and u rows ldg and ldu floats apart
 * (>= K): g and u may be the two halves of one [M, 2K] output, so gate and
 * up come from a single GEMM over the concatenated weights.  h_out and q
 * stay [M, K] contiguous.  No counterpart in the reference (its gate and up
 * are two separate projections); each h element is the same. */
int q8_silu_mul_quantize_rows_ld(const float* g, int64_t ldg, const float* u, int64_t ldu,
                                 int64_t M, int64_t K, float* h_out, int8_t* q, double* scales,
                                 void* stream);

/* ------------------------------------------------------------ elementwise */

/* One elementwise loop nest -- a PrimFunc the reference lowers to a loop nest
 * with a single store, e.g. the per-channel tail convert -> broadcast ->
 * mul that QuantizationPass emits after quantized_dot
 * (quantization_pass.ts:431-456), the bias add, ReLU (max) or a `quantize`
 * fused into such a group (rules/fusion.ts:66-79) -- evaluated on the device
 * with the reference CPU backend's arithmetic (src/backend/cpu/codegen.ts:
 * 428-552): every value is an f64, an f32-typed MathOp or non-exact extern
 * is rounded once to binary32 (Math.fround), exact externs (max, min, abs,
 * floor, ceil, round, sign, sqrt, fmod) are not rounded, a cast to an
 * integer type is ToInt32 (`| 0`), and the store converts like a typed-array
 * store (Float32Array: RNE; Int32Array / Int8Array / Uint8Array: the low
 * 32 / 8 bits of ToInt32).
 *
 * The loop nest has `ndims` loops of the given extents (row-major, the last
 * fastest); loop index i_d.  Input j is read at element offset
 * in_coef[j][0..ndims-1] . i + in_coef[j][Q8_EW_MAX_DIMS] (broadcasts have
 * zero coefficients); the output is written at the row-major offset of i.
 * The program is straight-line code over Q8_EW_MAX_REGS f64 registers; the
 * value of register `result` is stored. */
#define Q8_F64 4                 /* element type of q8_ewise inputs / output */
#define Q8_EW_MAX_DIMS   6
#define Q8_EW_MAX_INPUTS 8
#define Q8_EW_MAX_CODE   96
#define Q8_EW_MAX_REGS   16
#define Q8_EW_MAX_CONST  32

/* opcodes: r[dst] = ... ; `rnd` = 1 rounds the result to binary32 */
#define Q8_EW_LOAD     0   /* input[aux] at its offset */
#define Q8_EW_CONST    1   /* konst[aux] */
#define Q8_EW_INDEX    2   /* (double) i_aux, a loop index */
#define Q8_EW_ADD      3   /* a + b */
#define Q8_EW_SUB      4   /* a - b */
#define Q8_EW_MUL      5   /* a * b */
#define Q8_EW_DIV      6   /* a / b */
#define Q8_EW_IDIV     7   /* Math.trunc(a / b) (int-typed '/') */
#define Q8_EW_MOD      8   /* ((a % b + b) % b) */
#define Q8_EW_FLOORDIV 9   /* Math.floor(a / b) */
#define Q8_EW_TMOD     10  /* a % b */
#define Q8_EW_TDIV     11  /* ((a / b) | 0) */
#define Q8_EW_NEG      12  /* -a */
#define Q8_EW_CMP      13  /* (a OP b) ? 1 : 0, OP = aux: 0 ==, 1 !=, 2 <, 3 <=, 4 >, 5 >= */
#define Q8_EW_SELECT   14  /* a ? b : c (a truthy: not 0, not NaN) */
#define Q8_EW_TOINT32  15  /* a | 0 */
#define Q8_EW_TOBOOL   16  /* a ? 1 : 0 */
#define Q8_EW_MAX      17  /* Math.max(a, b) */
#define Q8_EW_MIN      18  /* Math.min(a, b) */
#define Q8_EW_ABS      19
#define Q8_EW_FLOOR    20
#define Q8_EW_CEIL     21
#define Q8_EW_ROUND    22  /* Math.round */
#define Q8_EW_SIGN     23
#define Q8_EW_SQRT     24
#define Q8_EW_FMOD     25  /* ((a % b + b) % b) */
#define Q8_EW_EXP      26
#define Q8_EW_LOG      27
#define Q8_EW_TANH     28
#define Q8_EW_RSQRT    29  /* 1 / Math.sqrt(a) */
#define Q8_EW_POW      30
#define Q8_EW_NOPS     31

typedef struct {
  uint8_t op, dst, a, b, c, aux, rnd, pad;
} q8_ew_instr;

typedef struct {
  int32_t ndims;
  int32_t ninputs;
  int64_t extent[Q8_EW_MAX_DIMS];
  int32_t in_dtype[Q8_EW_MAX_INPUTS];     /* Q8_I8, Q8_U8, Q8_I32, Q8_F32, Q8_F64 */
  int64_t in_coef[Q8_EW_MAX_INPUTS][Q8_EW_MAX_DIMS + 1];
  int32_t out_dtype;
  int32_t ncode;
  int32_t result;
  int32_t nconst;
  q8_ew_instr code[Q8_EW_MAX_CODE];
  double konst[Q8_EW_MAX_CONST];
} q8_ew_prog;

/* Runs `prog` over its loop nest: inputs[j] is a device array of
 * in_numel[j] elements of prog->in_dtype[j], out a device array of
 * out_numel elements of prog->out_dtype (out_numel = product of the
 * extents).  Every input offset the nest can form is checked against
 * in_numel on the host before the launch.  Inputs may alias each other but
 * not the output. */
int q8_ewise(const q8_ew_prog* prog, const void* const* inputs, const int64_t* in_numel,
             void* out, int64_t out_numel, void* stream);

/* How q8_ewise runs a program, no counterpart in the reference (its CUDA
 * backend compiles every elementwise kernel with NVRTC, cuda_runtime.ts):
 * a call over at least 2^20 elements compiles the program with hiprtc once
 * per program and device (the same JS helper functions, the library's IEEE
 * flags) and launches the cached kernel; smaller calls, and any program
 * hiprtc cannot take, run on the interpreter.  mode >= 0 sets the choice
 * (0 by size, 1 always the interpreter, 2 always compiled); the call
 * returns the number of programs compiled and of compiled launches so far
 * (either pointer may be NULL).  For tests and diagnosis. */
int q8_debug_ewise_jit(int mode, int64_t* compiled, int64_t* launches);

/* Why the last program hiprtc could not take fell back to the interpreter:
 * the failing step (hiprtc compile, code object load ...), its error string
 * and the compiler log, copied into buf (cap bytes, truncated and
 * NUL-terminated; "" if no compile has failed); *len (may be NULL) gets the
 * message's full length.  No counterpart in the reference; for diagnosis. */
int q8_debug_ewise_jit_error(char* buf, size_t cap, size_t* len);

/* ------------------------------------------------------------ calibration */

/* An observer is a device buffer of q8_observer_state_bytes(num_bins) bytes
 * holding a ValueObserver (min / max / count) and, when enabled, its
 * HistogramCollector (src/compiler/analysis/calibration.ts:11-126).  The
 * caller allocates it (q8_alloc) and owns it; calls on one observer are
 * ordered by the stream they are made on. */
int q8_observer_state_bytes(int num_bins, size_t* bytes);

/* new ValueObserver() (calibration.ts:17-22), plus enableHistogram(num_bins)
 * (:36-38) when histogram != 0.  1 <= num_bins <= Q8_OBS_MAX_BINS. */
int q8_observer_reset(void* state, int num_bins, int histogram, void* stream);

/* ValueObserver.update(x) (calibration.ts:24-34) with HistogramCollector.update
 * (:58-80, _initRange :82-92, _expandAndRebucket :94-126) for n fp32 values
 * in device memory.  NaN values count but are not binned, as in the
 * reference.  Enqueued only: no host synchronisation. */
int q8_observer_update(void* state, const float* x, int64_t n, void* stream);

/* Synchronously reads an observer back.  summary[Q8_OBS_SUMMARY] =
 * {min, max, count, histogram, initialized, range_min, range_max,
 *  total_count, num_bins}; bins (may be NULL) receives num_bins counts.
 * min is -0.0 or +0.0 when the smallest values seen are zeros of both signs
 * (the reference keeps whichever came first). */
int q8_observer_read(const void* state, double* summary, double* bins, void* stream);

/* HistogramCollector.computePercentileThreshold(percentile)
 * (calibration.ts:130-141) on a read-back observer (summary and bins as
 * written by q8_observer_read).  Host only. */
int q8_hist_percentile(const double* summary, const double* bins, double percentile,
                       double* threshold);

/* HistogramCollector.computeEntropyThreshold(num_quant_bins)
 * (calibration.ts:143-187): the threshold whose num_quant_bins-level
 * requantisation of the histogram has the least KL divergence.  Host only. */
int q8_hist_entropy(const double* summary, const double* bins, int num_quant_bins,
                    double* threshold);

/* CalibrationResult.getQuantParams (calibration.ts:246-268) on a read-back
 * observer: mode Q8_CALIB_*, scheme Q8_SCHEME_*, unsigned_ = dtype ui8.
 * Percentile (0.999) / entropy (255 levels, 256 for ui8) thresholds apply
 * unless the scheme is per-tensor asymmetric; the range then goes through
 * QuantizationParams.fromRange (quantization_types.ts:248-263), whose
 * zero-point form serves every scheme but the symmetric one.
 * *has_params = 0 (and Q8_OK) when the observer saw no values (getRange ->
 * null).  Host only; bins may be NULL for Q8_CALIB_MINMAX. */
int q8_calib_params(const double* summary, const double* bins, int mode, int scheme,
                    int unsigned_, double* scale, double* zero_point, int* has_params);

#pragma GCC visibility pop
#ifdef __cplusplus
}
#endif
#endif /* Q8HIP_H */
