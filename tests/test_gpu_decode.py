"""GPU parity of the one-call dynamic int8 linear (q8_qlinear_dynamic).

Expected values are the oracle's composition -- per-token (or per-tensor)
S-abs scales and R1 codes of x, exact int32 quantized_dot, the E-rowcol
epilogue with bias and activation -- compared bit for bit, together with
the codes and scales the call writes.  Shapes cover the fused one-token
kernel (M = 1, K <= 4096, K % 16 == 0: partial row blocks, K = 16, K = 48)
and the two-kernel route (M > 1 up to 16 tokens, K % 16 != 0, K > 4096);
rows carry NaN, +-inf, all-zero rows and exact half-way ties.  Each case is
also compared with the two separate calls (quantize_per_token +
qlinear) on the device.
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


def same_bits(a, b, what=""):
    """Bit equality, except that any NaN equals any NaN: the reference's
    values are JS numbers, and a NaN stored into a Float32Array may take
    any NaN encoding (ECMA-262 NumericToRawBytes), so sign and payload of a
    NaN are not part of its result (here: acc * inf through SiLU)."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    ne = np.any(a.view(np.uint8).reshape(-1, a.itemsize) != b.view(np.uint8).reshape(-1, b.itemsize), axis=1)
    if a.dtype.kind == "f":
        ne &= ~(np.isnan(a.reshape(-1)) & np.isnan(b.reshape(-1)))
    bad = np.nonzero(ne)[0]
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} of {a.size} differ; first at flat {i}: "
                             f"{a.reshape(-1)[i]!r} vs {b.reshape(-1)[i]!r}")


def expected(oracle, x, Wq, sW, bias, act, per_tensor):
    M, K = x.shape
    if per_tensor:
        s = oracle.scale_per_tensor(x)
        sx = np.array([s])
        xq = oracle.quantize(x.reshape(-1), s).reshape(M, K)
    else:
        sx = oracle.scales_per_token(x)
        xq = oracle.quantize_rows(x, sx)
    acc = oracle.quantized_dot(xq, Wq, b_layout=1)
    sA = np.full(M, sx[0]) if per_tensor else sx
    y = oracle.epilogue(acc, "rowcol", sA, sW, bias=bias, act=act)
    return y, xq, sx


def edge_rows(x):
    M, K = x.shape
    x[0, 5 % K] = np.nan
    if M > 1:
        x[1, :] = 0.0
    if M > 2:
        x[2, 7 % K] = np.inf
        x[2, 3 % K] = -np.inf
    if M > 3 and K >= 6:
        x[3, :6] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5]     # s = 1: x / s lands on ties
        x[3, 6:] = np.clip(x[3, 6:], -100, 100)
    return x


CASES = [(1, 4096, 4096), (2, 4096, 4096), (3, 4096, 4096), (4, 4096, 4096), (1, 1000, 4096),
         (4, 1001, 4096), (2, 77, 16), (1, 77, 16), (1, 33, 48), (3, 33, 48), (4, 11008, 4096),
         (1, 11008, 4096), (1, 19, 4000), (2, 19, 4000), (1, 64, 8192), (4, 64, 8192),
         (6, 300, 512), (1, 5, 4096), (1, 1001, 1024),
         # up to 16 tokens: the MFMA GEMV routes (balanced row ranges with
         # partial blocks at K = 4096, K < 4096, K > 4096)
         (8, 4096, 4096), (16, 4096, 4096), (16, 11008, 4096), (13, 1001, 1024), (16, 19, 4000),
         (5, 77, 16), (9, 33, 48), (16, 64, 8192)]


@pytest.mark.parametrize("M,N,K", CASES)
@pytest.mark.parametrize("bias,act", [(False, "none"), (True, "silu"), (True, "relu")])
def test_qlinear_dynamic_matches_oracle(ops, oracle, M, N, K, bias, act):
    r = oracle.Rng(M * 131 + N + K)
    x = edge_rows(r.normal((M, K)))
    W = r.normal((N, K), 0.0, 0.02)
    from oracle import configs as OC
    Wq, sW = OC.pack_pc(W, 0)
    b = r.uniform((N,), -0.1, 0.1) if bias else None
    print(f"qlinear_dynamic M={M} N={N} K={K} bias={bias} {act}", flush=True)
    want, want_q, want_s = expected(oracle, x, Wq, sW, b, act, False)
    y, xq, sx = ops.qlinear_dynamic(dev(x), dev(Wq), dev(sW), bias=None if b is None else dev(b), act=act)
    same_bits(host(sx), want_s, "scales")
    same_bits(host(xq), want_q, "codes")
    same_bits(host(y), want, "y")
    # the two separate calls on the device
    xq2, sx2 = ops.quantize_per_token(dev(x))
    y2 = ops.qlinear(xq2, sx2, dev(Wq), dev(sW), bias=None if b is None else dev(b), act=act)
    same_bits(host(y), host(y2), "vs quantize_per_token + qlinear")


def one_token_rows(K):
    """Single rows for the fused one-token kernel: every scale corner case."""
    rows = {}
    rows["zeros"] = np.zeros((1, K), np.float32)                   # scale 1e-10
    rows["all_nan"] = np.full((1, K), np.nan, np.float32)         # scale inf
    r = np.linspace(-3, 3, K, dtype=np.float32)[None, :]
    r[0, 1] = np.inf
    rows["inf"] = r
    t = np.clip(np.linspace(-100, 100, K, dtype=np.float32), -100, 100)[None, :]
    t[0, :6] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.5]                  # s = 1: ties
    rows["ties"] = t
    o = np.sin(np.arange(K, dtype=np.float32))[None, :]
    o[0, 3] = 5e4                                                  # outlier
    rows["outlier"] = o
    d = np.full((1, K), 1e-41, np.float32)                         # subnormal row
    rows["subnormal"] = d
    return rows


@pytest.mark.parametrize("K", [4096, 48, 1024])
def test_qlinear_dynamic_one_token_edge_rows(ops, oracle, K):
    r = oracle.Rng(K)
    W = r.normal((300, K), 0.0, 0.02)
    from oracle import configs as OC
    Wq, sW = OC.pack_pc(W, 0)
    b = r.uniform((300,), -0.1, 0.1)
    for name, x in one_token_rows(K).items():
        print(f"qlinear_dynamic one token K={K} {name}", flush=True)
        want, want_q, want_s = expected(oracle, x, Wq, sW, b, "relu", False)
        y, xq, sx = ops.qlinear_dynamic(dev(x), dev(Wq), dev(sW), bias=dev(b), act="relu")
        same_bits(host(sx), want_s, f"{name} scale")
        same_bits(host(xq), want_q, f"{name} codes")
        same_bits(host(y), want, f"{name} y")


@pytest.mark.parametrize("M,N,K", [(1, 256, 4096), (1, 513, 1024), (4, 513, 1024), (3, 40, 4000),
                                   (16, 11008, 4096), (11, 300, 2048)])
def test_qlinear_dynamic_per_tensor(ops, oracle, M, N, K):
    r = oracle.Rng(M + N + K + 7)
    x = r.normal((M, K))
    x[0, 1] = np.nan
    W = r.normal((N, K), 0.0, 0.02)
    from oracle import configs as OC
    Wq, sW = OC.pack_pc(W, 0)
    print(f"qlinear_dynamic per-tensor M={M} N={N} K={K}", flush=True)
    want, want_q, want_s = expected(oracle, x, Wq, sW, None, "none", True)
    y, xq, sx = ops.qlinear_dynamic(dev(x), dev(Wq), dev(sW), per_tensor=True)
    same_bits(host(sx), want_s, "scale")
    same_bits(host(xq), want_q, "codes")
    same_bits(host(y), want, "y")


def test_qlinear_dynamic_per_tensor_weight_scale(ops, oracle):
    """A per-tensor weight scale ([1]) in the fused kernel."""
    r = oracle.Rng(5)
    x = r.normal((1, 512))
    W = r.normal((70, 512), 0.0, 0.02)
    sWt = oracle.scale_per_tensor(W)
    Wq = oracle.quantize(W.reshape(-1), sWt).reshape(W.shape)
    want, _, _ = expected(oracle, x, Wq, np.full(70, sWt), None, "none", False)
    y, _, _ = ops.qlinear_dynamic(dev(x), dev(Wq), dev(np.array([sWt])))
    same_bits(host(y), want, "y")


def test_qlinear_dynamic_c5_decode(ops, oracle):
    """C5's decode GEMVs (seed 4, K = 4096, N = 4096 / 11008, M = 1 / 4) as
    the one-call op, against the oracle's composition on the same inputs."""
    from oracle import configs as OC
    inp = OC.c5_inputs(with_quant_tensor=False)
    for N in (4096, 11008):
        Wq, sW = OC.pack_pc(inp["W"][N], 0)
        for M in (1, 4):
            x = inp["x"][M]
            print(f"C5 decode M={M} N={N}", flush=True)
            y, _, _ = ops.qlinear_dynamic(dev(x), dev(Wq), dev(sW))
            same_bits(host(y), OC.qlinear_rows(x, Wq, sW), f"C5 M={M} N={N}")
