"""GPU parity of quantized_dot with zero points and ui8 operands
(q8_quantized_dot) against the oracle's restatement of the reference's
lowering (rules/quantization.ts:23-42), int32 bit for bit.

Covers i8 x i8, ui8 x i8, i8 x ui8 and ui8 x ui8, zero points on either
side (the 128 of an affine ui8 scheme, negative, asymmetric pairs), the
GEMM (M > 16), GEMV (M <= 16) and generic (K % 16 != 0) kernels, and a
case whose exact sum leaves the int32 range (ToInt32 wrap).
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


SHAPES = [(300, 264, 256), (5, 1000, 4096), (1, 77, 48), (40, 36, 40), (17, 130, 96), (3, 5, 7)]
KINDS = [(False, False), (True, False), (False, True), (True, True)]
ZPS = [(0, 0), (128, 0), (0, 128), (128, 128), (-3, 7), (255, -128)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("a_u8,b_u8", KINDS)
def test_quantized_dot_zero_points(ops, oracle, M, N, K, a_u8, b_u8):
    rng = np.random.default_rng(M * 31 + N + K + 2 * a_u8 + b_u8)
    A = rng.integers(0, 256, (M, K)).astype(np.uint8)
    B = rng.integers(0, 256, (N, K)).astype(np.uint8)
    A = A if a_u8 else A.view(np.int8)
    B = B if b_u8 else B.view(np.int8)
    dA, dB = dev(A), dev(B)
    for zpA, zpB in ZPS:
        print(f"quantized_dot M={M} N={N} K={K} a_u8={a_u8} b_u8={b_u8} zp=({zpA},{zpB})", flush=True)
        want = oracle.quantized_dot(A, B, 1, zpA, zpB)
        got = host(ops.quantized_dot(dA, dB, zpA, zpB))
        np.testing.assert_array_equal(got, want)


def test_quantized_dot_int32_wrap(ops, oracle):
    """sum (255 - 0) * (255 - 0) over K = 2^16 exceeds 2^31: stored ToInt32."""
    K = 1 << 16
    A = np.full((20, K), 255, np.uint8)
    B = np.full((3, K), 255, np.uint8)
    B[1] = 0
    want = oracle.quantized_dot(A, B, 1, 0, 0)
    exact = 255 * 255 * K
    assert exact >= 1 << 31 and want[0, 0] == ((exact + (1 << 31)) % (1 << 32)) - (1 << 31)
    np.testing.assert_array_equal(host(ops.quantized_dot(dev(A), dev(B))), want)
    np.testing.assert_array_equal(host(ops.quantized_dot(dev(A), dev(B), 3, 250)),
                                  oracle.quantized_dot(A, B, 1, 3, 250))
