"""Zero-size calls on the GPU: every op with an empty dimension does what the
reference's loops do over zero iterations (src/backend/cpu/codegen.ts
loop nests; quantized_dot zero-initializes its accumulator before the K
loop, rules/quantization.ts:23-42).  Compared with the oracle on the same
inputs: rows of zero length quantize with the observer's empty-range
scale, a contraction over K = 0 gives int32 zeros and the epilogue of a
zero accumulator (bias and activation included), and calls with no rows
or no columns write nothing and succeed."""
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
    assert a.tobytes() == b.tobytes(), what


@pytest.mark.parametrize("M,K", [(0, 64), (0, 0), (3, 0)])
def test_quantize_per_token_empty(ops, oracle, M, K):
    x = np.zeros((M, K), np.float32)
    q, s = ops.quantize_per_token(dev(x))
    same_bits(host(s), oracle.scales_per_token(x), f"scales M={M} K={K}")
    assert tuple(q.shape) == (M, K)


@pytest.mark.parametrize("M,K", [(0, 64), (4, 0)])
def test_dequantize_empty(ops, oracle, M, K):
    q = np.zeros((M, K), np.int8)
    s = np.full(M, 0.25)
    y = ops.dequantize(dev(q), dev(s))
    same_bits(host(y), oracle.dequantize_rows(q, s), f"dequantize M={M} K={K}")


@pytest.mark.parametrize("M,N,K", [(0, 8, 64), (8, 0, 64), (5, 7, 0), (0, 0, 0)])
def test_quantized_dot_empty(ops, oracle, M, N, K):
    A, B = np.zeros((M, K), np.int8), np.zeros((N, K), np.int8)
    acc = ops.quantized_dot(dev(A), dev(B))
    same_bits(host(acc), oracle.quantized_dot(A, B, b_layout=1), f"quantized_dot {M}x{N}x{K}")


@pytest.mark.parametrize("act", ["none", "relu", "silu"])
def test_qlinear_over_k_zero(ops, oracle, act):
    """K = 0: acc = 0, so y = act(fround(0 * sv) + b) -- the bias through the
    activation, signed zeros included."""
    M, N = 3, 6
    A, B = np.zeros((M, 0), np.int8), np.zeros((N, 0), np.int8)
    sA, sB = np.array([0.5, 0.25, 2.0]), np.linspace(0.1, 0.6, N)
    b = np.array([-1.5, -0.0, 0.0, 0.75, 3.0, -2.0], np.float32)
    y = ops.qlinear(dev(A), dev(sA), dev(B), dev(sB), bias=dev(b), act=act)
    want = oracle.epilogue(np.zeros((M, N), np.int32), "rowcol", sA, sB, bias=b, act=act)
    same_bits(host(y), want, f"qlinear K=0 {act}")


def test_ewise_over_no_elements(ops):
    """A loop nest with an extent of 0 runs no iteration on either route."""
    from mlfw_amd import _lib
    prog = ops.ew_program((0, 16), [(torch.float32, (16, 1))],
                          [("load", 0, 0, 0, 0, 0, 0), ("const", 1, 0, 0, 0, 0, 0), ("mul", 2, 0, 1, 0, 0, 1)],
                          2, torch.float32, konst=(0.5,))
    x = torch.empty((0, 16), dtype=torch.float32, device=DEV)
    out = torch.empty((0, 16), dtype=torch.float32, device=DEV)
    for mode in (1, 2):
        _lib.call("q8_debug_ewise_jit", mode, None, None)
        try:
            ops.ewise(prog, [x], out)
            torch.cuda.synchronize()
        finally:
            _lib.call("q8_debug_ewise_jit", 0, None, None)
