// q8_conv.hip -- quantized_conv for gfx950 (CDNA4).
//
// The reference op (src/compiler/ir/graph/ops/quantization.ts:156-190,
// lowered by rules/quantization.ts:44-62 through buildConvNest,
// src/compiler/passes/lowering/lowering_registry.ts:335-449) is an exact
// int32 convolution of int8 operands in NC(spatial) / OI(spatial) layout,
// with strides, [lo, hi] padding, dilation and groups; a tap whose input
// coordinate lies in the padding adds 0.
//
// Paths, all exact:
//   * GEMM form for contractions of 64 or more (Kc = Cg * prod(K)): the
//     [P, Kc] int8 matrix of a group's receptive fields (im2col) is built in
//     the caller's workspace and the int8 MFMA GEMM computes
//     out[n, g*Og : (g+1)*Og, :] = W_g [Og, Kc] x col^T -- the weight is the
//     A operand, so the [Og, P] result is already the NC(spatial) output
//     block and the dequant epilogue is fused as in q8_gemm.  With more than
//     16 output channels per group the images go in batches: the matrix of
//     nb images is [nb * P, Kc] and one GEMM computes [Og, nb * P], its
//     epilogue storing column n * P + p of the product at image n, position
//     p (column-blocked output), so a batch is one GEMM large enough to fill
//     the chip instead of nb small ones.  The matrix is built one of two ways:
//       - channels per group a multiple of 16: the group's input is first
//         transposed to a zero-padded channel-last frame, and the
//         contraction is taken tap-major (k = tap * Cg + c, the weight
//         permuted to match), so each row of the matrix is a run of
//         16-byte copies, one per tap; for a 1 x 1 kernel at stride 1 the
//         frame is the matrix and no copy is made.  Integer addition does
//         not depend on the order of the taps, so the sums are the same;
//       - otherwise a byte gather in the OI(spatial) order (ic-major, then
//         kernel positions), the contraction padded with zeros to a
//         multiple of 16 (the weight rows copied to that pitch).
//   * a direct kernel (one thread per output element) for short
//     contractions -- depthwise and other small-group convolutions, where a
//     GEMM per group would be launch-bound -- and for zero points and ui8
//     operands.
// Spatial ranks 1..3 share the code: unused trailing dimensions have size 1,
// stride 1, no padding and dilation 1.
#include "q8_device.h"
#include "q8_internal.h"

namespace q8 {

// im2col tile: I2C_TP output positions x I2C_TK contraction bytes of one
// image (contraction index k: ic-major, then kernel positions in row-major
// order -- the OI(spatial) weight's own order), zero past Kc.  Gather: the
// lanes of a wave take consecutive positions and one run of 32 contraction
// indices per wave, so each byte load of a wave reads neighbouring input
// bytes (with stride 1, consecutive bytes of a row); the tile is transposed
// through LDS so that the stores are 128-byte row segments of the matrix.
constexpr int I2C_TP = 64, I2C_TK = 128, I2C_PITCH = I2C_TK + 16;

__global__ __launch_bounds__(256) void k_im2col(const int8_t* __restrict__ x, ConvGeom G,
                                                int64_t n0, int64_t g, int8_t* __restrict__ col) {
  __shared__ __align__(16) uint32_t tile[I2C_TP * I2C_PITCH / 4];
  // blockIdx.y: image n0 + y of a batch, written at matrix rows y * P ..
  const int64_t n = n0 + blockIdx.y;
  col += (int64_t)blockIdx.y * G.Pn * G.Kc16;
  const int tk = (G.Kc16 + I2C_TK - 1) / I2C_TK;
  const int64_t pt = blockIdx.x / tk;
  const int k0 = (int)(blockIdx.x - pt * tk) * I2C_TK;
  const int64_t p0 = pt * I2C_TP;
  const int pl = threadIdx.x & 63;
  const int kq = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // the wave's 32 indices
  const int64_t p = p0 + pl;
  uint32_t w[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  int k = k0 + 32 * kq;
  if (p < G.Pn && k < G.Kc) {
    // output coordinates of p and the input coordinates of tap (0, 0, 0)
    const int o2 = (int)(p % G.P[2]);
    const int64_t t = p / G.P[2];
    const int o1 = (int)(t % G.P[1]);
    const int o0 = (int)(t / G.P[1]);
    const int b0 = (int)(o0 * G.st[0] - G.lo[0]);
    const int b1 = (int)(o1 * G.st[1] - G.lo[1]);
    const int b2 = (int)(o2 * G.st[2] - G.lo[2]);
    // contraction coordinates of the first byte, advanced with carries
    int ic = k / G.Kn;
    int r = k - ic * G.Kn;
    int k2 = r % G.K[2];
    r /= G.K[2];
    int k1 = r % G.K[1];
    int k0i = r / G.K[1];
    const int8_t* xg = x + (n * G.C + g * G.Cg) * G.Sn;
    // The contraction coordinates are the wave's own (uniform), advanced
    // with branch-free carries; a lane whose tap falls in the padding (or
    // past Kc) loads the plane's first byte and keeps 0.  The loop body is
    // one basic block, so its 32 loads issue back to back.
    uint32_t v[32];
#pragma unroll
    for (int b = 0; b < 32; ++b) {
      const int s0 = b0 + k0i * (int)G.dl[0];
      const int s1 = b1 + k1 * (int)G.dl[1];
      const int s2 = b2 + k2 * (int)G.dl[2];
      const bool kin = k + b < G.Kc;                       // uniform
      const bool in = kin && (unsigned)s0 < (unsigned)G.S[0] && (unsigned)s1 < (unsigned)G.S[1] &&
                      (unsigned)s2 < (unsigned)G.S[2];
      // offset in the plane, computed unconditionally (unsigned: no overflow
      // for a tap outside the image) and selected, so that no branch forms
      const uint32_t sp = ((uint32_t)s0 * (uint32_t)G.S[1] + (uint32_t)s1) * (uint32_t)G.S[2] + (uint32_t)s2;
      const int8_t* plane = xg + (int64_t)(kin ? ic : 0) * G.Sn;
      const uint32_t raw = (uint8_t)plane[in ? sp : 0u];   // in bounds either way
      v[b] = in ? raw : 0u;
      ++k2;
      const bool c2 = k2 == G.K[2];
      k2 = c2 ? 0 : k2;
      k1 += c2;
      const bool c1 = k1 == G.K[1];
      k1 = c1 ? 0 : k1;
      k0i += c1;
      const bool c0 = k0i == G.K[0];
      k0i = c0 ? 0 : k0i;
      ic += c0;
    }
#pragma unroll
    for (int b = 0; b < 32; ++b) w[b >> 2] |= v[b] << (8 * (b & 3));
  }
  uint32_t* trow = tile + (pl * I2C_PITCH + 32 * kq) / 4;
  reinterpret_cast<v4i*>(trow)[0] = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  reinterpret_cast<v4i*>(trow)[1] = v4i{(int)w[4], (int)w[5], (int)w[6], (int)w[7]};
  __syncthreads();
  // store: 8 lanes per 128-byte row segment, 32 rows per pass
  const int ch = threadIdx.x & 7;
#pragma unroll
  for (int pass = 0; pass < I2C_TP / 32; ++pass) {
    const int row = pass * 32 + (threadIdx.x >> 3);
    const int64_t prow = p0 + row;
    const int kk = k0 + 16 * ch;
    if (prow < G.Pn && kk < G.Kc16)
      *reinterpret_cast<v4i*>(col + prow * G.Kc16 + kk) =
          *reinterpret_cast<const v4i*>(tile + (row * I2C_PITCH + 16 * ch) / 4);
  }
}

// Launch grid of k_im2col for nb images: x = position tiles * contraction
// tiles, y = nb.  False if it does not fit a launch.
static bool im2col_grid(const ConvGeom& G, int64_t nb, dim3* grid) {
  const int64_t tiles = ((G.Pn + I2C_TP - 1) / I2C_TP) * ((G.Kc16 + I2C_TK - 1) / I2C_TK);
  if (tiles * 256 >= ((int64_t)1 << 32) || nb > 65535) return false;
  *grid = dim3((unsigned)tiles, (unsigned)nb);
  return true;
}

// Weight rows [O, Kc] -> [O, Kc16] with zero padding.
__global__ __launch_bounds__(256) void k_pad_rows(const int8_t* __restrict__ w, int64_t O, int64_t Kc,
                                                  int64_t Kc16, int8_t* __restrict__ wp) {
  const int64_t i = blockIdx.x * 256LL + threadIdx.x;
  if (i >= O * Kc16) return;
  const int64_t o = i / Kc16, k = i - o * Kc16;
  wp[i] = k < Kc ? w[o * Kc + k] : (int8_t)0;
}

// ---------------------------------------------------------------- channel-last path
// For Cg a multiple of 16 the contraction is taken tap-major, k = t * Cg + c
// (t: kernel position in row-major order, c: input channel of the group):
// the same products summed in another order, and int32 wrap-around addition
// does not depend on the order.  Each group's input goes once to a
// zero-padded channel-last frame xp[y][e][c], e over E0 x E1 x E2 with
// E_i = (P_i - 1) * st_i + (K_i - 1) * dl_i + 1 (input coordinate e_i - lo_i),
// so that the receptive field of output p at tap t is the Cg contiguous
// bytes xp[y][e(p) + off(t)][:] and im2col copies 16-byte chunks.  With a
// 1 x 1 kernel at stride 1 (E = P, off = 0) xp is the GEMM's B matrix itself.
struct ConvFrame {
  int E[3];
  int64_t Ep;   // E0 * E1 * E2
};

// xp[y][e][c] = x[n0 + y][g * Cg + c][e - lo] (0 outside the image), the nb
// images of a batch along blockIdx.y, 64-channel tiles along blockIdx.z.  A
// workgroup transposes 64 frame positions x 64 channels through LDS: in the
// gather each thread takes one position and 16 channels, the lanes of a
// wave consecutive positions, so each byte load of a wave reads
// neighbouring bytes of one channel plane; in the store the lanes take
// consecutive 16-byte chunks of the frame rows.
constexpr int FR_PITCH = 64 + 16;   // LDS row: 64 channel bytes + pad
__global__ __launch_bounds__(256) void k_conv_to_frame(const int8_t* __restrict__ x, ConvGeom G,
                                                       ConvFrame F, int64_t n0, int64_t g,
                                                       int8_t* __restrict__ xp) {
  __shared__ __align__(16) uint32_t tile[64 * FR_PITCH / 4];
  const int64_t y = blockIdx.y;
  const int64_t eb = blockIdx.x * 64LL;
  const int64_t e = eb + (threadIdx.x & 63);
  const int cs = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // the wave's 16-channel slice
  const int el = (int)(threadIdx.x & 63);
  bool in = false;
  uint32_t sp = 0u;
  if (e < F.Ep) {
    const int e2 = (int)(e % F.E[2]);
    const int64_t q = e / F.E[2];
    const int e1 = (int)(q % F.E[1]);
    const int e0 = (int)(q / F.E[1]);
    const int s0 = e0 - (int)G.lo[0], s1 = e1 - (int)G.lo[1], s2 = e2 - (int)G.lo[2];
    in = (unsigned)s0 < (unsigned)G.S[0] && (unsigned)s1 < (unsigned)G.S[1] &&
         (unsigned)s2 < (unsigned)G.S[2];
    // a position in the padding (or past the frame) reads the plane's
    // first byte and keeps 0
    sp = in ? ((uint32_t)s0 * (uint32_t)G.S[1] + (uint32_t)s1) * (uint32_t)G.S[2] + (uint32_t)s2 : 0u;
  }
  const int8_t* src = x + ((n0 + y) * G.C + g * G.Cg) * G.Sn + sp;
  for (int64_t ct = 64LL * blockIdx.z; ct < G.Cg; ct += 64LL * gridDim.z) {   // uniform
    const int64_t c = ct + 16 * cs;
    uint32_t w4[4] = {0u, 0u, 0u, 0u};
    if (c < G.Cg) {
      const int8_t* sc = src + c * G.Sn;
      uint32_t v[16];
#pragma unroll
      for (int b = 0; b < 16; ++b) v[b] = (uint8_t)sc[(int64_t)b * G.Sn];
#pragma unroll
      for (int b = 0; b < 16; ++b) w4[b >> 2] |= (in ? v[b] : 0u) << (8 * (b & 3));
    }
    reinterpret_cast<v4i*>(tile + (el * FR_PITCH + 16 * cs) / 4)[0] =
        v4i{(int)w4[0], (int)w4[1], (int)w4[2], (int)w4[3]};
    __syncthreads();
    // store: chunk ch of row r; 4 chunks per row of this channel tile
    const int cw = G.Cg - ct < 64 ? (int)((G.Cg - ct) >> 4) : 4;   // chunks in this tile
    for (int i = threadIdx.x; i < 64 * cw; i += 256) {
      const int r = i / cw, ch = i - r * cw;
      if (eb + r < F.Ep)
        *reinterpret_cast<v4i*>(xp + (y * F.Ep + eb + r) * G.Cg + ct + 16 * ch) =
            *reinterpret_cast<const v4i*>(tile + (r * FR_PITCH + 16 * ch) / 4);
    }
    __syncthreads();
  }
}

// wt[o][t * Cg + c] = w[o][c * Kn + t]: the OI(spatial) weight with its
// contraction in tap-major order.  A slice is 16 channels of one output
// channel o (slice s = o * (Cg / 16) + c / 16); its 16 * Kn weight bytes are
// contiguous, and so are those of consecutive slices.  A workgroup stages
// `ns` consecutive slices in LDS with 16-byte loads, then writes their
// ns * Kn 16-byte chunks wt[o][t * Cg + c0 .. + 16], tap-major so that
// neighbouring lanes write neighbouring chunks.  ns * Kn <= WT_CHUNKS.
constexpr int WT_CHUNKS = 1024;
__global__ __launch_bounds__(256) void k_conv_weight_taps(const int8_t* __restrict__ w, int64_t nslices,
                                                          int Cg, int Kn, int ns,
                                                          int8_t* __restrict__ wt) {
  __shared__ __align__(16) uint8_t buf[16 * WT_CHUNKS];
  const int64_t Kc = (int64_t)Cg * Kn;
  const int slices = Cg >> 4;
  const int64_t s0 = (int64_t)blockIdx.x * ns;
  const int n = (int)(nslices - s0 < ns ? nslices - s0 : ns);      // slices of this workgroup
  const v4i* src = reinterpret_cast<const v4i*>(w + s0 * 16 * Kn);   // 16-byte aligned
  for (int i = threadIdx.x; i < n * Kn; i += 256) reinterpret_cast<v4i*>(buf)[i] = src[i];
  __syncthreads();
  for (int i = threadIdx.x; i < n * Kn; i += 256) {
    const int t = i / n, sl = i - t * n;
    uint32_t w4[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int b = 0; b < 16; ++b) w4[b >> 2] |= (uint32_t)buf[(sl * 16 + b) * Kn + t] << (8 * (b & 3));
    const int64_t s = s0 + sl;
    const int64_t o = s / slices;
    const int c0 = (int)(s - o * slices) * 16;
    *reinterpret_cast<v4i*>(wt + o * Kc + (int64_t)t * Cg + c0) =
        v4i{(int)w4[0], (int)w4[1], (int)w4[2], (int)w4[3]};
  }
}

// col[y * Pn + p][t * Cg + c] = xp[y][e(p) + off(t)][c] with the frame
// position of output p, e(p) = row-major index of (o_i * st_i), and the
// offset of tap t, off(t) = row-major index of (k_i * dl_i), both over E.
// A thread copies one 16-byte channel chunk of output p for a group of four
// consecutive taps at a time (four loads in flight); the groups are spread
// over blockIdx.z.  Tap coordinates are uniform.
__global__ __launch_bounds__(256) void k_im2col_taps(const int8_t* __restrict__ xp, ConvGeom G,
                                                     ConvFrame F, int8_t* __restrict__ col) {
  const int64_t y = blockIdx.y;
  const int cpr = G.Cg >> 4;
  const int64_t idx = blockIdx.x * 256LL + threadIdx.x;
  if (idx >= G.Pn * cpr) return;
  const int64_t p = idx / cpr;
  const int c = (int)(idx - p * cpr) * 16;
  const int o2 = (int)(p % G.P[2]);
  const int64_t q = p / G.P[2];
  const int o1 = (int)(q % G.P[1]);
  const int o0 = (int)(q / G.P[1]);
  const int64_t ep = ((int64_t)o0 * G.st[0] * F.E[1] + (int64_t)o1 * G.st[1]) * F.E[2] +
                     (int64_t)o2 * G.st[2];
  const int64_t Cg = G.Cg;
  const int8_t* src = xp + (y * F.Ep + ep) * Cg + c;
  int8_t* dst = col + (y * G.Pn + p) * G.Kc + c;
  for (int t0 = 4 * blockIdx.z; t0 < G.Kn; t0 += 4 * gridDim.z) {
    int k2 = t0 % G.K[2];
    const int r = t0 / G.K[2];
    int k1 = r % G.K[1];
    int k0 = r / G.K[1];
    int64_t o4[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // a tap past Kn repeats tap t0: the same bytes, stored again at t0
      o4[j] = t0 + j < G.Kn ? (((int64_t)k0 * G.dl[0] * F.E[1] + (int64_t)k1 * G.dl[1]) * F.E[2] +
                               (int64_t)k2 * G.dl[2])
                            : o4[0];
      const bool c2 = ++k2 == G.K[2];
      k2 = c2 ? 0 : k2;
      k1 += c2;
      const bool c1 = k1 == G.K[1];
      k1 = c1 ? 0 : k1;
      k0 += c1;
    }
    v4i a[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = *reinterpret_cast<const v4i*>(src + o4[j] * Cg);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<v4i*>(dst + (int64_t)(t0 + j < G.Kn ? t0 + j : t0) * Cg) = a[j];
  }
}

// Direct form: one thread per output element, taps in the reference's
// order (ic, then kernel positions), int32 wrap-around sum of
// (x - zpx) * (w - zpw) over the taps inside the image (a padded tap adds
// 0), operands read as i8 or ui8.
__global__ __launch_bounds__(256) void k_conv_direct(const int8_t* __restrict__ x,
                                                     const int8_t* __restrict__ w, ConvGeom G,
                                                     GemmEpi e, void* __restrict__ out) {
  const int64_t idx = blockIdx.x * 256LL + threadIdx.x;
  const int64_t total = G.N * G.O * G.Pn;
  if (idx >= total) return;
  const int64_t p = idx % G.Pn;
  const int64_t no = idx / G.Pn;
  const int64_t o = no % G.O, n = no / G.O;
  const int64_t g = o / G.Og;
  const int o2 = (int)(p % G.P[2]);
  const int64_t t = p / G.P[2];
  const int o1 = (int)(t % G.P[1]);
  const int o0 = (int)(t / G.P[1]);
  const int8_t* xg = x + (n * G.C + g * G.Cg) * G.Sn;
  const int8_t* wo = w + o * (int64_t)G.Kc;
  uint32_t acc = 0;
  for (int ic = 0; ic < G.Cg; ++ic) {
    const int8_t* xc = xg + (int64_t)ic * G.Sn;
    const int8_t* wc = wo + (int64_t)ic * G.Kn;
    for (int k0 = 0; k0 < G.K[0]; ++k0) {
      const int64_t s0 = (int64_t)o0 * G.st[0] + (int64_t)k0 * G.dl[0] - G.lo[0];
      if (s0 < 0 || s0 >= G.S[0]) continue;
      for (int k1 = 0; k1 < G.K[1]; ++k1) {
        const int64_t s1 = (int64_t)o1 * G.st[1] + (int64_t)k1 * G.dl[1] - G.lo[1];
        if (s1 < 0 || s1 >= G.S[1]) continue;
        for (int k2 = 0; k2 < G.K[2]; ++k2) {
          const int64_t s2 = (int64_t)o2 * G.st[2] + (int64_t)k2 * G.dl[2] - G.lo[2];
          if (s2 < 0 || s2 >= G.S[2]) continue;
          const int64_t xi = (s0 * G.S[1] + s1) * G.S[2] + s2;
          const int64_t wi = (k0 * G.K[1] + k1) * G.K[2] + k2;
          const int xv = G.x_u8 ? (int)reinterpret_cast<const uint8_t*>(xc)[xi] : (int)xc[xi];
          const int wv = G.w_u8 ? (int)reinterpret_cast<const uint8_t*>(wc)[wi] : (int)wc[wi];
          acc += (uint32_t)((xv - G.zpx) * (wv - G.zpw));
        }
      }
    }
  }
  if (e.out_i32) static_cast<int32_t*>(out)[idx] = (int32_t)acc;
  else static_cast<float*>(out)[idx] = (float)((double)(int32_t)acc * e.s_out);
}

// k_im2col computes input coordinates and offsets within one channel plane
// in 32 bits: every coordinate lies in [-lo, (P - 1) * st + (K - 1) * dl].
bool conv_uses_gemm(const ConvGeom& G) {
  if (G.Kc < 64 || G.Sn >= ((int64_t)1 << 31)) return false;
  for (int i = 0; i < 3; ++i)
    if ((int64_t)(G.P[i] - 1) * G.st[i] + (int64_t)(G.K[i] - 1) * G.dl[i] >= ((int64_t)1 << 31)) return false;
  return true;
}

bool conv_direct(const ConvGeom& G) {
  return !conv_uses_gemm(G) || G.zpx != 0 || G.zpw != 0 || G.x_u8 || G.w_u8;
}

constexpr size_t CONV_BATCH_BYTES = (size_t)128 << 20;   // workspace per batch of images
static size_t round256(size_t b) { return (b + 255) & ~(size_t)255; }

// Images per batch: as many as fit CONV_BATCH_BYTES of per-image workspace
// (`per`), within the launch limits; 1 with 16 or fewer output channels per
// group, which go through the GEMV kernel one image at a time.
static int64_t conv_batch_of(const ConvGeom& G, size_t per) {
  if (G.Og <= 16) return 1;
  int64_t nb = per ? (int64_t)(CONV_BATCH_BYTES / per) : 1;
  nb = nb > G.N ? G.N : nb;
  nb = nb > 65535 ? 65535 : nb;                                 // grid.y of the per-image launches
  const int64_t cap = ((int64_t)1 << 31) / (G.Pn > 0 ? G.Pn : 1) - 1;   // GEMM N = nb * P in an int
  nb = nb > cap ? cap : nb;
  return nb < 1 ? 1 : nb;
}

// The channel-last path: Cg a multiple of 16, at most WT_CHUNKS kernel
// positions, frame and matrix offsets of one image within 31 bits.
static bool conv_frame_of(const ConvGeom& G, ConvFrame* F) {
  if (G.Cg % 16 != 0 || G.Kn > WT_CHUNKS) return false;
  int64_t ep = 1;
  for (int i = 0; i < 3; ++i) {
    const int64_t E = (int64_t)(G.P[i] - 1) * G.st[i] + (int64_t)(G.K[i] - 1) * G.dl[i] + 1;
    if (E > ((int64_t)1 << 31) / ep) return false;
    F->E[i] = (int)E;
    ep *= E;
  }
  F->Ep = ep;
  return ep * G.Cg < ((int64_t)1 << 31) && G.Pn * G.Kc < ((int64_t)1 << 31);
}

static bool conv_pointwise(const ConvGeom& G) {
  return G.Kn == 1 && G.st[0] == 1 && G.st[1] == 1 && G.st[2] == 1;
}

// Implicit GEMM (launch_gemm_conv: the GEMM reads the frame itself, no
// im2col matrix): channels per group a multiple of 64, a contraction of at
// most 16384, more than 16 output channels per group (the GEMM, not the
// GEMV); a pointwise conv needs no im2col in any case.
static bool conv_implicit(const ConvGeom& G) {
  return !conv_pointwise(G) && G.Cg % 64 == 0 && G.Kc <= 16384 && G.Og > 16;
}

// channel-last workspace: [col: nb * Pn * Kc, unless pointwise or implicit] [frame:
// nb * Ep * Cg] [tap-major weight: O * Kc, unless 1 x 1] [split-K partial
// sums of the implicit GEMM], each rounded up to 256 bytes
struct ClLayout {
  int64_t nb;
  size_t col, frame, wt, part;   // part: split-K partial sums of the implicit GEMM
};
static ClLayout cl_layout(const ConvGeom& G, const ConvFrame& F) {
  const bool no_col = conv_pointwise(G) || conv_implicit(G);
  const size_t col1 = no_col ? 0 : (size_t)G.Pn * (size_t)G.Kc;
  const size_t fr1 = (size_t)F.Ep * (size_t)G.Cg;
  ClLayout L;
  L.nb = conv_batch_of(G, col1 + fr1);
  L.col = round256((size_t)L.nb * col1);
  L.frame = round256((size_t)L.nb * fr1);
  L.wt = G.Kn == 1 ? 0 : round256((size_t)G.O * (size_t)G.Kc);   // 1 x 1: the weight as given
  L.part = 0;
  if (conv_implicit(G)) {
    const ConvGemmPlan pl = conv_gemm_plan(G.Og, L.nb * G.Pn, G.Kc, (size_t)1 << 30);
    if (pl.splits > 1) L.part = round256((size_t)pl.splits * (size_t)G.Og * (size_t)(L.nb * G.Pn) * 4);
  }
  return L;
}

size_t conv_workspace_bytes(const ConvGeom& G) {
  if (!conv_uses_gemm(G)) return 0;
  // the im2col form: batched matrices, then padded weight rows
  size_t b = round256((size_t)conv_batch_of(G, (size_t)G.Pn * (size_t)G.Kc16) * (size_t)G.Pn *
                      (size_t)G.Kc16);
  if (G.Kc16 != G.Kc) b += (size_t)G.O * (size_t)G.Kc16;
  ConvFrame F;
  if (conv_frame_of(G, &F)) {   // also enough for the im2col form it falls back to
    const ClLayout L = cl_layout(G, F);
    const size_t cl = L.col + L.frame + L.wt + L.part;
    b = cl > b ? cl : b;
  }
  return b;
}

static hipError_t launch_conv_channel_last(const int8_t* x, const int8_t* w, const int8_t* w_taps,
                                           const ConvGeom& G, const ConvFrame& F, const GemmEpi& e,
                                           void* workspace, void* out, hipStream_t st) {
  const ClLayout L = cl_layout(G, F);
  const bool pw = conv_pointwise(G);
  int8_t* col = static_cast<int8_t*>(workspace);
  int8_t* xp = col + L.col;
  // a 1 x 1 kernel's weight is its own tap-major form; a prepacked one
  // (q8_conv_weight_taps) is used as given
  int8_t* wt = G.Kn == 1 ? const_cast<int8_t*>(w) : w_taps ? const_cast<int8_t*>(w_taps) : xp + L.frame;
  int32_t* part = reinterpret_cast<int32_t*>(xp + L.frame + L.wt);
  const int64_t nsl = G.O * (G.Cg >> 4);                   // weight slices
  const int wns = G.Kn >= 256 ? WT_CHUNKS / G.Kn : 256 / G.Kn;   // slices per workgroup
  const int64_t wblk = (nsl + wns - 1) / wns;
  const int64_t xch = G.Pn * (G.Cg >> 4);
  const int64_t ctiles = (G.Cg + 63) / 64, tgroups = (G.Kn + 3) / 4;
  if (wblk >= ((int64_t)1 << 24) || (F.Ep + 63) / 64 >= ((int64_t)1 << 24) ||
      (xch + 255) / 256 >= ((int64_t)1 << 24))
    return hipErrorInvalidValue;
  const unsigned fz = (unsigned)(ctiles < 65535 ? ctiles : 65535);   // strided loops cover the rest
  const unsigned tz = (unsigned)(tgroups < 65535 ? tgroups : 65535);
  hipError_t err = hipSuccess;
  if (G.Kn > 1 && !w_taps) {
    hipLaunchKernelGGL(k_conv_weight_taps, dim3((unsigned)wblk), dim3(256), 0, st, w, nsl, G.Cg, G.Kn,
                       wns, wt);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  const size_t osz = e.out_i32 ? sizeof(int32_t) : sizeof(float);
  GemmEpi eb = e;
  eb.col_blk = G.Pn;
  eb.blk_stride = G.O * G.Pn;
  eb.ld_out = G.Pn;
  const bool impl = conv_implicit(G);
  if (impl) {
    GemmEpi::ConvB& c = eb.cb;
    c.Pn = (uint32_t)G.Pn;
    c.P1 = (uint32_t)G.P[1];
    c.P2 = (uint32_t)G.P[2];
    c.st0 = (uint32_t)G.st[0];
    c.st1 = (uint32_t)G.st[1];
    c.st2 = (uint32_t)G.st[2];
    c.E1 = (uint32_t)F.E[1];
    c.E2 = (uint32_t)F.E[2];
    c.Ep = (uint32_t)F.Ep;
    c.Cg = (uint32_t)G.Cg;
    c.K1 = (uint32_t)G.K[1];
    c.K2 = (uint32_t)G.K[2];
    c.Kn = (uint32_t)G.Kn;
    c.dl0 = (uint32_t)G.dl[0];
    c.dl1 = (uint32_t)G.dl[1];
    c.dl2 = (uint32_t)G.dl[2];
  }
  for (int64_t n0 = 0; n0 < G.N; n0 += L.nb) {
    const int64_t nb = G.N - n0 < L.nb ? G.N - n0 : L.nb;
    for (int64_t g = 0; g < G.groups; ++g) {
      hipLaunchKernelGGL(k_conv_to_frame, dim3((unsigned)((F.Ep + 63) / 64), (unsigned)nb, fz),
                         dim3(256), 0, st, x, G, F, n0, g, xp);
      err = hipGetLastError();
      if (err != hipSuccess) return err;
      const int8_t* A = wt + g * G.Og * G.Kc;
      void* o = static_cast<char*>(out) + (size_t)((n0 * G.O + g * G.Og) * G.Pn) * osz;
      if (impl) {
        GemmEpi ei = eb;
        ei.cb.frame_bytes = (uint32_t)(nb * F.Ep * G.Cg);
        const ConvGemmPlan pl = conv_gemm_plan(G.Og, nb * G.Pn, G.Kc, L.part);
        err = launch_gemm_conv(A, xp, G.Og, nb * G.Pn, G.Kc, ei, pl, part, o, st);
        if (err != hipSuccess) return err;
        continue;
      }
      const int8_t* B = xp;
      if (!pw) {
        hipLaunchKernelGGL(k_im2col_taps, dim3((unsigned)((xch + 255) / 256), (unsigned)nb, tz),
                           dim3(256), 0, st, xp, G, F, col);
        err = hipGetLastError();
        if (err != hipSuccess) return err;
        B = col;
      }
      if (nb > 1) err = launch_gemm(A, B, G.Og, nb * G.Pn, G.Kc, eb, o, st);
      else if (G.Og <= 16) err = launch_gemv(A, B, G.Og, G.Pn, G.Kc, e, o, st);
      else err = launch_gemm(A, B, G.Og, G.Pn, G.Kc, e, o, st);
      if (err != hipSuccess) return err;
    }
  }
  return hipSuccess;
}

bool conv_taps_used(const ConvGeom& G) { return G.Cg % 16 == 0 && G.Kn > 1 && G.Kn <= WT_CHUNKS; }

hipError_t launch_conv_weight_taps(const int8_t* w, const ConvGeom& G, int8_t* w_taps, hipStream_t st) {
  if (!conv_taps_used(G) || G.O == 0) return hipErrorInvalidValue;
  const int64_t nsl = G.O * (G.Cg >> 4);
  const int wns = G.Kn >= 256 ? WT_CHUNKS / G.Kn : 256 / G.Kn;
  const int64_t wblk = (nsl + wns - 1) / wns;
  if (wblk >= ((int64_t)1 << 24)) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_conv_weight_taps, dim3((unsigned)wblk), dim3(256), 0, st, w, nsl, G.Cg, G.Kn, wns, w_taps);
  return hipGetLastError();
}

hipError_t launch_conv(const int8_t* x, const int8_t* w, const int8_t* w_taps, const ConvGeom& G,
                       const GemmEpi& e, void* workspace, void* out, hipStream_t st) {
  if (G.N * G.O * G.Pn == 0) return hipSuccess;
  if (conv_direct(G)) {
    const int64_t total = G.N * G.O * G.Pn;
    hipLaunchKernelGGL(k_conv_direct, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x,
                       w, G, e, out);
    return hipGetLastError();
  }
  ConvFrame F;
  if (conv_frame_of(G, &F) && ((reinterpret_cast<uintptr_t>(workspace) | reinterpret_cast<uintptr_t>(w)) & 15) == 0)
    return launch_conv_channel_last(x, w, w_taps, G, F, e, workspace, out, st);
  int8_t* col = static_cast<int8_t*>(workspace);
  const int64_t NB = conv_batch_of(G, (size_t)G.Pn * (size_t)G.Kc16);
  const size_t col_bytes = ((size_t)NB * (size_t)G.Pn * (size_t)G.Kc16 + 255) & ~(size_t)255;
  const int8_t* wmat = w;
  if (G.Kc16 != G.Kc) {
    int8_t* wp = col + col_bytes;
    const int64_t n = G.O * G.Kc16;
    hipLaunchKernelGGL(k_pad_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, G.O,
                       (int64_t)G.Kc, (int64_t)G.Kc16, wp);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    wmat = wp;
  }
  const size_t osz = e.out_i32 ? sizeof(int32_t) : sizeof(float);
  // batched form: the GEMM's MFMA path needs 16-byte-aligned operands (the
  // weight rows and the workspace); otherwise one image at a time
  const bool aligned = ((reinterpret_cast<uintptr_t>(wmat) | reinterpret_cast<uintptr_t>(col)) & 15) == 0;
  if (NB > 1 && aligned && (int64_t)G.Kc16 * 256 < ((int64_t)1 << 31)) {
    GemmEpi eb = e;
    eb.col_blk = G.Pn;
    eb.blk_stride = G.O * G.Pn;
    eb.ld_out = G.Pn;
    for (int64_t n0 = 0; n0 < G.N; n0 += NB) {
      const int64_t nb = G.N - n0 < NB ? G.N - n0 : NB;
      for (int64_t g = 0; g < G.groups; ++g) {
        dim3 grid;
        if (!im2col_grid(G, nb, &grid)) return hipErrorInvalidValue;
        hipLaunchKernelGGL(k_im2col, grid, dim3(256), 0, st, x, G, n0, g, col);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        const int8_t* A = wmat + g * G.Og * G.Kc16;
        void* o = static_cast<char*>(out) + (size_t)((n0 * G.O + g * G.Og) * G.Pn) * osz;
        err = launch_gemm(A, col, G.Og, nb * G.Pn, G.Kc16, eb, o, st);
        if (err != hipSuccess) return err;
      }
    }
    return hipSuccess;
  }
  for (int64_t n = 0; n < G.N; ++n)
    for (int64_t g = 0; g < G.groups; ++g) {
      dim3 grid;
      if (!im2col_grid(G, 1, &grid)) return hipErrorInvalidValue;
      hipLaunchKernelGGL(k_im2col, grid, dim3(256), 0, st, x, G, n, g, col);
      hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
      const int8_t* A = wmat + g * G.Og * G.Kc16;
      void* o = static_cast<char*>(out) + (size_t)((n * G.O + g * G.Og) * G.Pn) * osz;
      err = G.Og <= 16 ? launch_gemv(A, col, G.Og, G.Pn, G.Kc16, e, o, st)
                       : launch_gemm(A, col, G.Og, G.Pn, G.Kc16, e, o, st);
      if (err != hipSuccess) return err;
    }
  return hipSuccess;
}

}  // namespace q8
