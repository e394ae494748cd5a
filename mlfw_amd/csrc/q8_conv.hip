// q8_conv.hip -- quantized_conv for gfx950 (CDNA4).
//
// The reference op (src/compiler/ir/graph/ops/quantization.ts:156-190,
// lowered by rules/quantization.ts:44-62 through buildConvNest,
// src/compiler/passes/lowering/lowering_registry.ts:335-449) is an exact
// int32 convolution of int8 operands in NC(spatial) / OI(spatial) layout,
// with strides, [lo, hi] padding, dilation and groups; a tap whose input
// coordinate lies in the padding adds 0.
//
// Two paths, both exact:
//   * implicit-GEMM form for contractions of 64 or more (Cg * prod(K)):
//     an im2col pass writes the [P, Kc16] int8 matrix of a group's receptive
//     fields (contraction padded with zeros to a multiple of 16) into the
//     caller's workspace, and the int8 MFMA GEMM computes
//     out[n, g*Og : (g+1)*Og, :] = W_g [Og, Kc16] x col^T -- the weight is
//     the A operand, so the [Og, P] result is already the NC(spatial)
//     output block and the dequant epilogue is fused as in q8_gemm.  With
//     more than 16 output channels per group the images go in batches: one
//     im2col launch fills [nb * P, Kc16] and one GEMM computes [Og, nb * P],
//     its epilogue storing column n * P + p of the product at image n,
//     position p (column-blocked output), so a batch of images is one
//     launch of a GEMM large enough to fill the chip instead of nb small
//     ones.  An OI(spatial) weight is [O, Kc] row-major, i.e. the GEMM's
//     A layout; it is copied to a 16-byte-aligned row pitch only when Kc is
//     not a multiple of 16.
//   * a direct kernel (one thread per output element) for short
//     contractions -- depthwise and other small-group convolutions, where a
//     GEMM per group would be launch-bound.
// Spatial ranks 1..3 share the code: unused trailing dimensions have size 1,
// stride 1, no padding and dilation 1.
#include "q8_device.h"
#include "q8_internal.h"

namespace q8 {

// 16 bytes of the im2col matrix per thread: receptive field of output
// position p, contraction indices 16c .. 16c+15 (ic-major, then kernel
// positions in row-major order -- the OI(spatial) weight's own order).
__global__ __launch_bounds__(256) void k_im2col(const int8_t* __restrict__ x, ConvGeom G,
                                                int64_t n0, int64_t g, int8_t* __restrict__ col) {
  // blockIdx.y: image n0 + y of a batch, written at matrix rows y * P ..
  const int64_t n = n0 + blockIdx.y;
  col += (int64_t)blockIdx.y * G.Pn * G.Kc16;
  const int64_t nch = G.Kc16 >> 4;
  const int64_t idx = blockIdx.x * 256LL + threadIdx.x;
  if (idx >= G.Pn * nch) return;
  const int64_t p = idx / nch;
  const int c = (int)(idx - p * nch);
  // output coordinates of p
  const int o2 = (int)(p % G.P[2]);
  const int64_t t = p / G.P[2];
  const int o1 = (int)(t % G.P[1]);
  const int o0 = (int)(t / G.P[1]);
  // contraction coordinates of the first byte, advanced with carries
  int k = 16 * c;
  int ic = k / G.Kn;
  int r = k - ic * G.Kn;
  int k2 = r % G.K[2];
  r /= G.K[2];
  int k1 = r % G.K[1];
  int k0 = r / G.K[1];
  const int8_t* xg = x + (n * G.C + g * G.Cg) * G.Sn;
  uint32_t w4[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int b = 0; b < 16; ++b, ++k) {
    if (k < G.Kc) {
      const int64_t s0 = (int64_t)o0 * G.st[0] + (int64_t)k0 * G.dl[0] - G.lo[0];
      const int64_t s1 = (int64_t)o1 * G.st[1] + (int64_t)k1 * G.dl[1] - G.lo[1];
      const int64_t s2 = (int64_t)o2 * G.st[2] + (int64_t)k2 * G.dl[2] - G.lo[2];
      if (s0 >= 0 && s0 < G.S[0] && s1 >= 0 && s1 < G.S[1] && s2 >= 0 && s2 < G.S[2]) {
        const uint8_t v = (uint8_t)xg[(int64_t)ic * G.Sn + (s0 * G.S[1] + s1) * G.S[2] + s2];
        w4[b >> 2] |= (uint32_t)v << (8 * (b & 3));
      }
      if (++k2 == G.K[2]) {
        k2 = 0;
        if (++k1 == G.K[1]) {
          k1 = 0;
          if (++k0 == G.K[0]) {
            k0 = 0;
            ++ic;
          }
        }
      }
    }
  }
  const v4i out = {(int)w4[0], (int)w4[1], (int)w4[2], (int)w4[3]};
  reinterpret_cast<v4i*>(col + p * G.Kc16)[c] = out;
}

// Weight rows [O, Kc] -> [O, Kc16] with zero padding.
__global__ __launch_bounds__(256) void k_pad_rows(const int8_t* __restrict__ w, int64_t O, int64_t Kc,
                                                  int64_t Kc16, int8_t* __restrict__ wp) {
  const int64_t i = blockIdx.x * 256LL + threadIdx.x;
  if (i >= O * Kc16) return;
  const int64_t o = i / Kc16, k = i - o * Kc16;
  wp[i] = k < Kc ? w[o * Kc + k] : (int8_t)0;
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

bool conv_uses_gemm(const ConvGeom& G) { return G.Kc >= 64; }

bool conv_direct(const ConvGeom& G) {
  return !conv_uses_gemm(G) || G.zpx != 0 || G.zpw != 0 || G.x_u8 || G.w_u8;
}

// Images per im2col batch: all of them, up to CONV_BATCH_BYTES of im2col
// matrix; 1 with 16 or fewer output channels per group, which go through
// the GEMV kernel one image at a time.
constexpr size_t CONV_BATCH_BYTES = (size_t)128 << 20;
static int64_t conv_batch(const ConvGeom& G) {
  if (G.Og <= 16) return 1;
  const size_t per = (size_t)G.Pn * (size_t)G.Kc16;
  int64_t nb = per ? (int64_t)(CONV_BATCH_BYTES / per) : 1;
  nb = nb > G.N ? G.N : nb;
  nb = nb > 65535 ? 65535 : nb;                                 // grid.y of the im2col launch
  const int64_t cap = ((int64_t)1 << 31) / (G.Pn > 0 ? G.Pn : 1) - 1;   // GEMM N = nb * P in an int
  nb = nb > cap ? cap : nb;
  return nb < 1 ? 1 : nb;
}

size_t conv_workspace_bytes(const ConvGeom& G) {
  if (!conv_uses_gemm(G)) return 0;
  size_t b = (size_t)conv_batch(G) * (size_t)G.Pn * (size_t)G.Kc16;   // im2col matrices
  b = (b + 255) & ~(size_t)255;
  if (G.Kc16 != G.Kc) b += (size_t)G.O * (size_t)G.Kc16;  // padded weight rows
  return b;
}

hipError_t launch_conv(const int8_t* x, const int8_t* w, const ConvGeom& G, const GemmEpi& e,
                       void* workspace, void* out, hipStream_t st) {
  if (G.N * G.O * G.Pn == 0) return hipSuccess;
  if (conv_direct(G)) {
    const int64_t total = G.N * G.O * G.Pn;
    hipLaunchKernelGGL(k_conv_direct, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x,
                       w, G, e, out);
    return hipGetLastError();
  }
  int8_t* col = static_cast<int8_t*>(workspace);
  const int64_t NB = conv_batch(G);
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
  const int64_t cells = G.Pn * (G.Kc16 >> 4);
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
        hipLaunchKernelGGL(k_im2col, dim3((unsigned)((cells + 255) / 256), (unsigned)nb), dim3(256), 0, st,
                           x, G, n0, g, col);
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
      hipLaunchKernelGGL(k_im2col, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, st, x, G,
                         n, g, col);
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
