"""GPU parity of quantized_conv (q8_quantized_conv) against the CPU oracle.

int32 accumulators and fp32 dequantized outputs are compared bit for bit.
The cases cover both device paths (direct kernel for contractions shorter
than 64, im2col + MFMA GEMM otherwise, with and without a contraction that
is a multiple of 16), the GEMV and the GEMM kernels behind the latter
(<= 16 and > 16 output channels per group), groups / depthwise, strides,
asymmetric padding, dilation, batch > 1 (batches of images in one GEMM
whose epilogue scatters columns to images, with 16-byte and with
per-element stores; one image at a time for the GEMV), spatial ranks 1 to
3, and the three GEMM forms of the contraction: the byte-gather im2col
(channels per group not a multiple of 16), the channel-last frame with a
tap-major im2col (1 x 1 kernels use the frame itself), and the implicit
GEMM reading the frame (channels per group a multiple of 64), with and
without a split of K; zero
points and ui8 operands; then the whole pipeline QuantizationPass builds
for a conv (quantize input, quantize kernel, quantized_conv, dequantize).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from mlfw_amd import ops as O
    from mlfw_amd import _lib
    _lib.call("q8_init", 0)
    return O


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def same_bits(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    av = a.view(np.uint8).reshape(-1, a.itemsize)
    bv = b.view(np.uint8).reshape(-1, b.itemsize)
    bad = np.nonzero(np.any(av != bv, axis=1))[0]
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{bad.size} of {a.size} differ; first at flat {i}: "
                             f"{a.reshape(-1)[i]!r} vs {b.reshape(-1)[i]!r}")


CASES = [
    # x shape, w shape, strides, padding, dilation, groups      path
    ((1, 3, 8, 8), (16, 3, 3, 3), [1, 1], [[0, 0], [0, 0]], [1, 1], 1),      # direct (Kc 27)
    ((1, 3, 8, 8), (16, 3, 3, 3), [2, 2], [[1, 1], [1, 1]], [1, 1], 1),      # direct
    ((2, 32, 9, 7), (8, 8, 3, 2), [2, 1], [[1, 2], [0, 1]], [2, 1], 4),      # direct (Kc 48), groups
    ((1, 64, 10), (64, 1, 3), [1], [[1, 1]], [2], 64),                       # depthwise 1-D
    ((2, 64, 12, 12), (32, 64, 3, 3), [1, 1], [[1, 1], [1, 1]], [1, 1], 1),  # GEMM (Kc 576)
    ((1, 20, 11, 13), (48, 10, 3, 3), [1, 2], [[0, 2], [1, 0]], [1, 1], 2),  # GEMM, Kc 90 -> 96, groups
    ((3, 16, 7, 9), (8, 16, 2, 3), [1, 1], [[1, 0], [0, 0]], [2, 1], 1),     # GEMV (Og 8), Kc 96
    ((1, 8, 6, 5, 7), (24, 8, 2, 3, 2), [1, 2, 1], [[1, 0], [0, 1], [1, 1]], [1, 1, 2], 1),  # 3-D
    ((1, 256, 14, 14), (300, 256, 1, 1), [1, 1], [[0, 0], [0, 0]], [1, 1], 1),  # 1x1, tile edges
    # batched im2col + column-blocked GEMM (N > 1, Og > 16)
    ((3, 20, 12, 12), (48, 10, 3, 3), [1, 1], [[1, 1], [1, 1]], [1, 1], 2),  # groups, Kc 90 -> 96
    ((5, 256, 14, 14), (300, 256, 1, 1), [1, 1], [[0, 0], [0, 0]], [1, 1], 1),  # P 196, edges
    ((4, 32, 6, 10), (40, 32, 3, 3), [1, 1], [[1, 1], [1, 1]], [1, 1], 1),   # P 60, tile straddles
    ((2, 64, 11, 11), (32, 64, 3, 3), [1, 1], [[0, 0], [0, 0]], [1, 1], 1),  # P 81: element stores
    ((3, 512, 7, 7), (64, 512, 3, 3), [1, 1], [[1, 1], [1, 1]], [1, 1], 1),  # P 49, Kc 4608
    # channel-last frame (Cg % 16 == 0) beyond the cases above
    ((2, 32, 9, 11), (48, 16, 3, 2), [2, 1], [[1, 2], [0, 1]], [1, 2], 2),   # groups, stride, dilation
    ((2, 16, 5, 6, 7), (32, 16, 2, 3, 2), [1, 2, 1], [[1, 0], [0, 1], [1, 1]], [1, 1, 2], 1),  # 3-D
    ((3, 64, 9, 9), (40, 64, 1, 1), [2, 2], [[0, 0], [0, 0]], [1, 1], 1),    # 1x1 at stride 2
    ((2, 48, 6, 6), (24, 48, 1, 1), [1, 1], [[1, 1], [0, 2]], [1, 1], 1),    # 1x1 padded: frame is B
    # implicit GEMM split over K (few tiles, long contraction)
    ((2, 64, 9, 9), (48, 64, 5, 5), [1, 1], [[2, 2], [2, 2]], [1, 1], 1),    # 3 splits, K % 128 = 64
    ((2, 256, 6, 6), (96, 128, 3, 3), [1, 1], [[1, 1], [1, 1]], [1, 1], 2),  # 2 splits, groups
]


@pytest.mark.parametrize("case", CASES)
def test_quantized_conv_int32(ops, oracle, case):
    xs, ws, st, pd, dl, g = case
    rng = np.random.default_rng(sum(xs) + 13 * g)
    x = rng.integers(-128, 128, xs).astype(np.int8)
    w = rng.integers(-128, 128, ws).astype(np.int8)
    print(f"conv case x{xs} w{ws} s{st} p{pd} d{dl} g{g}", flush=True)
    got = ops.quantized_conv(dev(x), dev(w), st, pd, dl, g)
    same_bits(host(got), oracle.quantized_conv(x, w, st, pd, dl, g))


@pytest.mark.parametrize("case", CASES)
def test_quantized_conv_prepacked_weight(ops, oracle, case):
    """A constant weight prepacked once (q8_conv_weight_taps: tap-major,
    w_taps[o][t * Cg + c] = w[o][c][t]) gives the same bits as the per-call
    permutation, on every path that reads it; weights without a tap-major
    form (Cg % 16 != 0, one kernel position) report None."""
    xs, ws, st, pd, dl, g = case
    rng = np.random.default_rng(sum(xs) + 17 * g)
    x = rng.integers(-128, 128, xs).astype(np.int8)
    w = rng.integers(-128, 128, ws).astype(np.int8)
    wt = ops.conv_weight_taps(dev(w), g)
    kn = int(np.prod(ws[2:]))
    if ws[1] % 16 != 0 or kn < 2:
        assert wt is None
        return
    O, Cg = ws[0], ws[1]
    same_bits(host(wt), w.reshape(O, Cg, kn).transpose(0, 2, 1).reshape(-1))
    for s_out in (None, 1e-4):
        got = ops.quantized_conv(dev(x), dev(w), st, pd, dl, g, s_out=s_out, w_taps=wt)
        acc = oracle.quantized_conv(x, w, st, pd, dl, g)
        want = acc if s_out is None else oracle.dequantize(acc.reshape(-1), s_out).reshape(acc.shape)
        same_bits(host(got), want)


@pytest.mark.parametrize("case", CASES[:2] + CASES[4:6] + CASES[9:])
def test_quantized_conv_dequant_epilogue(ops, oracle, case):
    xs, ws, st, pd, dl, g = case
    rng = np.random.default_rng(sum(ws))
    x = rng.integers(-128, 128, xs).astype(np.int8)
    w = rng.integers(-128, 128, ws).astype(np.int8)
    s_out = (2.5 / 127) * (0.07 / 127)
    got = ops.quantized_conv(dev(x), dev(w), st, pd, dl, g, s_out=s_out)
    acc = oracle.quantized_conv(x, w, st, pd, dl, g)
    want = oracle.dequantize(acc.reshape(-1), s_out).reshape(acc.shape)
    same_bits(host(got), want)


@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[4], CASES[7]])
@pytest.mark.parametrize("x_u8,w_u8", [(False, False), (True, False), (True, True)])
def test_quantized_conv_zero_points_and_ui8(ops, oracle, case, x_u8, w_u8):
    """input_zero_point / kernel_zero_point and ui8 operands (the direct
    kernel), int32 bit for bit; a padded tap adds 0."""
    xs, ws, st, pd, dl, g = case
    rng = np.random.default_rng(len(xs) * 13 + g + 2 * x_u8 + w_u8)
    x = rng.integers(0, 256, xs).astype(np.uint8)
    w = rng.integers(0, 256, ws).astype(np.uint8)
    x = x if x_u8 else x.view(np.int8)
    w = w if w_u8 else w.view(np.int8)
    for zpx, zpw in ((0, 0), (128, 0), (3, -2), (128, 128)):
        print(f"conv zp {xs} {ws} x_u8={x_u8} w_u8={w_u8} zp=({zpx},{zpw})", flush=True)
        want = oracle.quantized_conv(x, w, st, pd, dl, g, zpx, zpw)
        got = ops.quantized_conv(dev(x), dev(w), st, pd, dl, g, zpx=zpx, zpw=zpw)
        same_bits(host(got), want)


def test_conv_pipeline_of_the_quantization_pass(ops, oracle):
    """quantize(input), quantize(kernel), quantized_conv, dequantize -- the op
    sequence pass.test.js:428-441 pins -- on fp32 data, both quantizes with the
    compiled op's arithmetic (quant_math.ts:16-27) and calibrated per-tensor
    symmetric scales, output scale input_scale * kernel_scale in f64."""
    r = oracle.Rng(41)
    x = r.normal((2, 64, 10, 10))
    w = r.normal((32, 64, 3, 3), 0.0, 0.05)
    sx = oracle.scale_per_tensor(x)
    sw = oracle.scale_per_tensor(w)
    xq = oracle.quantize(x.reshape(-1), sx).reshape(x.shape)
    wq = oracle.quantize(w.reshape(-1), sw).reshape(w.shape)
    s_out = sx * sw
    acc = oracle.quantized_conv(xq, wq, [1, 1], [[1, 1], [1, 1]], [1, 1], 1)
    want = oracle.dequantize(acc.reshape(-1), s_out).reshape(acc.shape)
    xq_d = ops.quantize(dev(x), sx)
    wq_d = ops.quantize(dev(w), sw)
    same_bits(host(xq_d), xq)
    same_bits(host(wq_d), wq)
    got = ops.quantized_conv(xq_d, wq_d, [1, 1], [[1, 1], [1, 1]], [1, 1], 1, s_out=s_out)
    same_bits(host(got), want)


def test_conv_workspace_is_reused(ops, oracle):
    """A caller-owned workspace serves consecutive calls on one stream."""
    rng = np.random.default_rng(3)
    x = rng.integers(-128, 128, (1, 64, 9, 9)).astype(np.int8)
    w = rng.integers(-128, 128, (40, 64, 3, 3)).astype(np.int8)
    ws = torch.empty(1 << 20, dtype=torch.int8, device=DEV)
    a = ops.quantized_conv(dev(x), dev(w), [1, 1], [[0, 0], [0, 0]], workspace=ws)
    b = ops.quantized_conv(dev(x[:, :, :5, :5].copy()), dev(w), [1, 1], [[0, 0], [0, 0]], workspace=ws)
    same_bits(host(a), oracle.quantized_conv(x, w, [1, 1], [[0, 0], [0, 0]]))
    same_bits(host(b), oracle.quantized_conv(x[:, :, :5, :5].copy(), w, [1, 1], [[0, 0], [0, 0]]))
