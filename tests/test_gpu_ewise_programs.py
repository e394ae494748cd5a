"""q8_ewise on the three elementwise PrimFuncs bench.py times
(configs.ewise_programs): the per-channel dequant with bias, ReLU fused
with quantize, and a dequantize feeding an add, over [M, N] with ragged
shapes.  Expected values follow the reference CPU codegen's JS for the same
loop bodies (src/backend/cpu/codegen.ts:428-552): every value an f64, an
f32-typed mul / add / div rounded once to binary32 (Math.fround), max and
round exact, the Int8Array store of `| 0`; the quantize is the oracle's R1.
Compared bit for bit."""
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


def same_bits(a, b, what=""):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    ne = np.any(a.view(np.uint8).reshape(-1, a.itemsize) != b.view(np.uint8).reshape(-1, b.itemsize), axis=1)
    bad = np.nonzero(ne)[0]
    assert bad.size == 0, f"{what}: {bad.size} of {a.size} differ; first at {bad[0]}: {a.reshape(-1)[bad[0]]!r} vs {b.reshape(-1)[bad[0]]!r}"


def f32(x):
    return np.asarray(x, np.float64).astype(np.float32)


@pytest.mark.parametrize("M,N", [(4096, 4096), (37, 1001), (1, 5), (300, 4099)])
def test_ewise_programs_match_js_semantics(ops, oracle, M, N):
    from mlfw_amd import configs as C
    rng = np.random.default_rng(M * 7 + N)
    progs = C.ewise_programs(M, N, s_q=0.05, s_dq=0.01)
    # per-channel dequant with bias
    prog, _, _, _ = progs["dequant_bias"]
    acc = rng.integers(-2 ** 31, 2 ** 31, (M, N), dtype=np.int64).astype(np.int32)
    acc[0, : min(N, 4)] = [2 ** 31 - 1, -2 ** 31, 0, 1 << 24][: min(N, 4)]
    sv = rng.uniform(1e-6, 1e-3, N).astype(np.float32)
    b = rng.uniform(-1, 1, N).astype(np.float32)
    out = torch.empty((M, N), dtype=torch.float32, device=DEV)
    ops.ewise(prog, [dev(acc), dev(sv), dev(b)], out)
    want = f32(f32(acc.astype(np.float64) * sv.astype(np.float64)[None, :]).astype(np.float64)
               + b.astype(np.float64)[None, :])
    same_bits(host(out), want, "dequant_bias")
    # ReLU + quantize, with NaN, +-inf, -0 and exact ties
    prog, _, _, _ = progs["relu_quantize"]
    x = (rng.standard_normal((M, N)) * 4).astype(np.float32)
    flat = x.reshape(-1)
    edge = np.array([np.nan, np.inf, -np.inf, -0.0, 0.025, 0.075, 6.375, 6.35, 1e30], np.float32)
    flat[: min(flat.size, edge.size)] = edge[: min(flat.size, edge.size)]
    out8 = torch.empty((M, N), dtype=torch.int8, device=DEV)
    ops.ewise(prog, [dev(x)], out8)
    relu = np.where(np.isnan(x), np.float32(np.nan), np.maximum(x, np.float32(0)))
    same_bits(host(out8), oracle.quantize(relu.reshape(-1), 0.05).reshape(M, N), "relu_quantize")
    # dequantize feeding an add
    prog, _, _, _ = progs["dequant_add"]
    q = rng.integers(-128, 128, (M, N)).astype(np.int8)
    y = rng.standard_normal((M, N)).astype(np.float32)
    ops.ewise(prog, [dev(q), dev(y)], out)
    want = f32(f32(q.astype(np.float64) * 0.01).astype(np.float64) + y.astype(np.float64))
    same_bits(host(out), want, "dequant_add")
