"""Seeded shape fuzz of the int8 GEMM against the oracle.

Random M, N, K (K tails that are not multiples of 16 included, so both the
MFMA kernel and the generic fallback run), per-token or per-tensor
activation scales, per-channel or per-tensor weight scales, and every
output form of the GEMM: raw int32 (quantized_dot, M1 of
rules/quantization.ts:23-42), the fp32 row x column epilogue with or
without bias and ReLU / SiLU (quantization_pass.ts:431-456), and the
static int8 requant of that value (quant_math.ts:16-27).  The shapes span
the tile choices of the launch (256x256 / 256x192 / 256x128 / 128x128 /
64x64) with partial tiles on both edges.  Bit for bit; each case prints
its seed and shape first."""
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


def same_bits(a, b, what):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    ne = a.view(np.uint8).reshape(-1, a.itemsize) != b.view(np.uint8).reshape(-1, b.itemsize)
    ne = np.any(ne, axis=1)
    if a.dtype.kind == "f":
        ne &= ~(np.isnan(a.reshape(-1)) & np.isnan(b.reshape(-1)))
    bad = np.nonzero(ne)[0]
    assert bad.size == 0, f"{what}: {bad.size} of {a.size} differ; first at {bad[0]}: " \
                          f"{a.reshape(-1)[bad[0]]!r} vs {b.reshape(-1)[bad[0]]!r}"


def shape_of(seed):
    rng = np.random.default_rng(1000 + seed)
    big = seed % 3 == 0
    M = int(rng.integers(1, 1100 if big else 300))
    N = int(rng.integers(1, 1500 if big else 400))
    K = int(rng.integers(1, 40)) * 16 * (2 if big else 1)
    if seed % 5 == 1:
        K += int(rng.integers(1, 16))          # a tail: the generic kernel
    return rng, M, N, K


@pytest.mark.parametrize("seed", range(24))
def test_gemm_fuzz(ops, oracle, seed):
    rng, M, N, K = shape_of(seed)
    form = ["i32", "f32", "f32_bias_relu", "f32_bias_silu", "q8"][seed % 5]
    per_token = seed % 2 == 0
    per_channel = seed % 4 != 3
    print(f"gemm fuzz seed={seed} M={M} N={N} K={K} form={form} per_token={per_token} "
          f"per_channel={per_channel}", flush=True)
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    B = rng.integers(-128, 128, (N, K)).astype(np.int8)
    acc = oracle.quantized_dot(A, B, b_layout=1)
    if form == "i32":
        same_bits(host(ops.quantized_dot(dev(A), dev(B))), acc, f"seed {seed} int32")
        return
    sA = rng.uniform(1e-3, 0.05, M if per_token else 1)
    sB = rng.uniform(1e-4, 0.02, N if per_channel else 1)
    bias = rng.uniform(-1, 1, N).astype(np.float32) if "bias" in form else None
    act = "relu" if "relu" in form else "silu" if "silu" in form else "none"
    sA_full = sA if per_token else np.full(M, sA[0])
    sB_full = sB if per_channel else np.full(N, sB[0])
    y = oracle.epilogue(acc, "rowcol", sA_full, sB_full, bias=bias, act=act)
    b_dev = None if bias is None else dev(bias)
    if form == "q8":
        s_next = float(np.abs(y).max() / 127.0) or 1.0
        got = ops.qlinear_requant(dev(A), dev(sA), dev(B), dev(sB), s_next, bias=b_dev, act=act)
        same_bits(host(got), oracle.quantize(y.reshape(-1), s_next).reshape(M, N), f"seed {seed} int8 requant")
    else:
        got = ops.qlinear(dev(A), dev(sA), dev(B), dev(sB), bias=b_dev, act=act)
        same_bits(host(got), y, f"seed {seed} fp32 {act}")
