"""GPU parity of every primitive of the int8 path against the CPU oracle.

All comparisons are bit-exact (int8 codes, int32 accumulators, f64 scales and
fp32 outputs compared as bit patterns), except the Box-Muller fill, whose
log/cos/sin come from different libms (see test_fill_normal_matches_oracle).
Inputs come from the oracle's seeded generator and are uploaded, so both
sides see identical bits.
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


def edge_rows(oracle, K=4096):
    """Rows that exercise the rounding and the scale corner cases."""
    rng = oracle.Rng(123)
    rows = []
    base = rng.normal((K,))
    rows.append(base)                                   # plain
    r = base.copy(); r[7] = 50.0; rows.append(r)        # outlier
    rows.append(np.zeros(K, np.float32))                # all zero -> scale 1e-10
    r = np.full(K, np.nan, np.float32); rows.append(r)  # all NaN -> scale inf
    r = base.copy(); r[::97] = np.nan; rows.append(r)   # some NaN
    r = base.copy(); r[3] = np.inf; rows.append(r)      # +inf -> scale inf
    r = base.copy(); r[5] = -np.inf; r[6] = np.inf; rows.append(r)
    r = base.copy(); r[:10] = -0.0; rows.append(r)      # negative zeros
    r = (base * 1e-30).astype(np.float32); rows.append(r)   # subnormal-ish range
    r = (base * 1e30).astype(np.float32); rows.append(r)
    # exact ties: x / s = k + 0.5 for s = 1 (absmax 127)
    t = np.arange(-127, 128, 1, dtype=np.float32) * 0.5
    r = np.resize(t, K).astype(np.float32); r[0] = 127.0; rows.append(r)
    # values one ulp around ties for s = 127/127 = 1
    t = np.float32(2.5)
    r = np.resize(np.array([np.nextafter(t, np.float32(3)), t, np.nextafter(t, np.float32(2)),
                            -t, np.nextafter(-t, np.float32(0))], np.float32), K)
    r[0] = 127.0
    rows.append(r.astype(np.float32))
    return np.stack(rows).astype(np.float32)


# ------------------------------------------------------------------ quantize
@pytest.mark.parametrize("shape", [(1, 1), (3, 5), (7, 4096), (33, 1000), (16, 11008),
                                   (2, 12289), (5, 0)])
def test_quantize_per_token_random(ops, oracle, shape):
    x = oracle.Rng(1).normal(shape)
    if x.size:
        x.reshape(-1)[:: max(1, x.size // 17)] *= 40.0
    q, s = ops.quantize_per_token(dev(x))
    s_ref = oracle.scales_per_token(x)
    same_bits(host(s), s_ref)
    same_bits(host(q), oracle.quantize_rows(x, s_ref))


def test_quantize_per_token_edges(ops, oracle):
    x = edge_rows(oracle)
    q, s = ops.quantize_per_token(dev(x))
    s_ref = oracle.scales_per_token(x)
    same_bits(host(s), s_ref)
    same_bits(host(q), oracle.quantize_rows(x, s_ref))


def test_quantize_per_token_unaligned(ops, oracle):
    # K % 4 != 0 and a misaligned view take the scalar kernel
    x = oracle.Rng(5).normal((9, 1023))
    q, s = ops.quantize_per_token(dev(x))
    s_ref = oracle.scales_per_token(x)
    same_bits(host(s), s_ref)
    same_bits(host(q), oracle.quantize_rows(x, s_ref))


@pytest.mark.parametrize("n", [0, 1, 4095, 1 << 20])
def test_quantize_per_tensor(ops, oracle, n):
    x = oracle.Rng(2).normal((n,))
    if n > 10:
        x[7] = -33.0
        x[9] = np.nan
    q, s = ops.quantize_per_tensor(dev(x))
    s_ref = oracle.scale_per_tensor(x)
    same_bits(host(s), np.array([s_ref]))
    same_bits(host(q), oracle.quantize(x, s_ref))


@pytest.mark.parametrize("fill", ["zeros", "nans", "nan_and_zero", "inf"])
def test_quantize_per_tensor_degenerate(ops, oracle, fill):
    # all zeros -> 1e-10, only NaNs -> +inf (an observer that saw no value),
    # an infinity -> +inf; the key's start value and the final mapping
    x = np.zeros(5000, np.float32)
    if fill == "nans":
        x[:] = np.nan
    elif fill == "nan_and_zero":
        x[::2] = np.nan
    elif fill == "inf":
        x = oracle.Rng(4).normal((5000,))
        x[77] = -np.inf
    q, s = ops.quantize_per_tensor(dev(x))
    s_ref = oracle.scale_per_tensor(x)
    same_bits(host(s), np.array([s_ref]))
    same_bits(host(q), oracle.quantize(x, s_ref))


def test_quantize_per_tensor_concurrent_streams(ops, oracle):
    # Per-tensor reductions keep their key in the call's own scales output,
    # so calls on different streams with different outputs never interfere.
    # Each stream's tensor has its own absmax; all calls are enqueued before
    # any is waited for, several rounds in a row.
    n = 1 << 20
    xs = []
    for i in range(4):
        x = oracle.Rng(40 + i).normal((n,))
        x[1000 * i + 3] = 10.0 * (i + 2)
        xs.append(x)
    streams = [torch.cuda.Stream() for _ in xs]
    xd = [dev(x) for x in xs]
    torch.cuda.synchronize()
    outs = [(torch.empty(n, dtype=torch.int8, device=DEV),
             torch.empty(1, dtype=torch.float64, device=DEV)) for _ in xs]
    for _ in range(5):
        for st, x, (q, s) in zip(streams, xd, outs):
            with torch.cuda.stream(st):
                ops.quantize_per_tensor(x, q, s)
        torch.cuda.synchronize()
        for x, (q, s) in zip(xs, outs):
            s_ref = oracle.scale_per_tensor(x)
            same_bits(host(s), np.array([s_ref]))
            same_bits(host(q), oracle.quantize(x, s_ref))


def test_pack_weight_per_tensor_concurrent_streams(ops, oracle):
    Ws = [oracle.Rng(60 + i).normal((256, 512), 0.0, 0.5 + i) for i in range(3)]
    streams = [torch.cuda.Stream() for _ in Ws]
    Wd = [dev(W) for W in Ws]
    torch.cuda.synchronize()
    res = []
    for st, W in zip(streams, Wd):
        with torch.cuda.stream(st):
            res.append(ops.pack_weight(W, axis=0, granularity="per_tensor"))
    torch.cuda.synchronize()
    for W, (Wq, s) in zip(Ws, res):
        s_ref = oracle.scale_const_array(W)
        same_bits(host(s), np.array([s_ref]))
        same_bits(host(Wq), oracle.weight_quantize_per_tensor(W, s_ref, -127, 127))


@pytest.mark.parametrize("ldx", [8, 12])
def test_quantize_per_token_many_rows(ops, oracle, ldx):
    # More rows than the 2^20 row workers of one launch: the pipelined loop
    # (two register sets, the prefetch of row + G, the early exit), with
    # contiguous and row-strided rows.
    M, K = (1 << 20) + 3, 8
    x = oracle.Rng(77).normal((M, ldx))
    x[::4099, 1] = 9.0
    x[5::7001, :K] = 0.0
    xd = dev(x)
    q, s = ops.quantize_per_token(xd[:, :K] if ldx != K else xd)
    xc = np.ascontiguousarray(x[:, :K])
    s_ref = oracle.scales_per_token(xc)
    same_bits(host(s), s_ref)
    same_bits(host(q), oracle.quantize_rows(xc, s_ref))


@pytest.mark.parametrize("scale,zp,tgt", [(6 / 127, 0.0, "i8"), (0.0123, 0.0, "i8"),
                                          (6 / 255, -128.0, "i8"), (1 / 255, 0.0, "ui8"),
                                          (6 / 255, 3.0, "ui8"), (1e-10, 0.0, "i8"),
                                          (1e30, 0.0, "i8"), (1.0, 0.0, "i8")])
def test_quantize_static(ops, oracle, scale, zp, tgt):
    x = oracle.Rng(3).normal((4099,), 0.0, 3.0)
    x[:6] = [3.5, -2.1, 5.9, 1.234, -5.9, 0.001]       # pass.test.js:451 data
    x[6:12] = [np.nan, np.inf, -np.inf, -0.0, 0.5, -0.5]
    q = ops.quantize(dev(x), scale, zp, tgt)
    same_bits(host(q), oracle.quantize(x, scale, zp, tgt == "ui8"))


def test_quantize_static_rejects_nonpositive_scale(ops):
    from mlfw_amd._lib import Q8Error
    with pytest.raises(Q8Error):
        ops.quantize(torch.zeros(4, device=DEV), 0.0)
    with pytest.raises(Q8Error):
        ops.quantize(torch.zeros(4, device=DEV), -1.0)



def test_caller_outputs_are_checked(ops):
    """Caller-supplied output tensors of the wrong dtype, size or device are
    refused before any launch (the kernels write M*N elements)."""
    A = torch.zeros((32, 64), dtype=torch.int8, device=DEV)
    B = torch.zeros((48, 64), dtype=torch.int8, device=DEV)
    sA = torch.ones(32, dtype=torch.float64, device=DEV)
    sB = torch.ones(48, dtype=torch.float64, device=DEV)
    with pytest.raises(ValueError):
        ops.qlinear(A, sA, B, sB, out=torch.empty((32, 47), dtype=torch.float32, device=DEV))
    with pytest.raises(TypeError):
        ops.quantized_dot(A, B, out=torch.empty((32, 48), dtype=torch.float32, device=DEV))
    with pytest.raises(ValueError):
        ops.quantized_dot(A, B, out=torch.empty((32, 48), dtype=torch.int32))
    x = torch.zeros((8, 64), dtype=torch.float32, device=DEV)
    with pytest.raises(ValueError):
        ops.quantize_per_token(x, scales=torch.empty(7, dtype=torch.float64, device=DEV))
    assert ops.quantized_dot(A, B, out=torch.empty((32, 48), dtype=torch.int32, device=DEV)).shape == (32, 48)


@pytest.mark.parametrize("off,n", [(0, 0), (3, 1), (1, 15), (0, 4096), (5, 100003)])
def test_memset_fill_kernel(ops, off, n):
    """q8_memset writes exactly [off, off + n) (unaligned heads and tails)."""
    from mlfw_amd import _lib
    import ctypes as C
    buf = torch.full((n + 64,), 7, dtype=torch.uint8, device=DEV)
    _lib.call("q8_memset", C.c_void_p(buf.data_ptr() + off), 0xAB, n, ops._stream())
    want = np.full(n + 64, 7, np.uint8)
    want[off:off + n] = 0xAB
    np.testing.assert_array_equal(host(buf), want)


def test_memset_in_a_graph(ops):
    """q8_memset captured in a HIP graph (with a quantize after it) gives the
    right bytes on every replay, with eager writes to the buffer between."""
    from mlfw_amd import _lib
    import ctypes as C
    buf = torch.zeros(5000, dtype=torch.uint8, device=DEV)
    x = torch.linspace(-3, 3, 8 * 64, device=DEV).reshape(8, 64)
    q = torch.empty((8, 64), dtype=torch.int8, device=DEV)
    s = torch.empty(8, dtype=torch.float64, device=DEV)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            _lib.call("q8_memset", C.c_void_p(buf.data_ptr() + 1), 0x5A, 4099, ops._stream())
            ops.quantize_per_token(x, q, s)
    q_eager, s_eager = ops.quantize_per_token(x)
    for rep in range(3):
        buf.fill_(rep)
        q.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        b = host(buf)
        assert b[0] == rep and b[4100] == rep and (b[1:4100] == 0x5A).all(), rep
        np.testing.assert_array_equal(host(q), host(q_eager))
        np.testing.assert_array_equal(host(s), host(s_eager))

# ------------------------------------------------------------------ dequantize
def test_dequantize_rows_i8(ops, oracle):
    x = edge_rows(oracle, 1024)
    s = oracle.scales_per_token(x)
    q = oracle.quantize_rows(x, s)
    y = ops.dequantize(dev(q), dev(s))
    same_bits(host(y), oracle.dequantize_rows(q, s))


@pytest.mark.parametrize("dt,zp", [(np.int8, 0.0), (np.int8, 5.0), (np.uint8, 128.0),
                                   (np.int32, 0.0), (np.int32, -7.0)])
def test_dequantize_per_tensor(ops, oracle, dt, zp):
    rng = np.random.default_rng(0)
    if dt == np.int32:
        q = rng.integers(-2 ** 31, 2 ** 31, size=(37, 64), dtype=np.int64).astype(np.int32)
    else:
        info = np.iinfo(dt)
        q = rng.integers(info.min, info.max + 1, size=(37, 64)).astype(dt)
    for s in (6 / 127, 0.0012345678901234, 3.0e-7 * 7.77):
        y = ops.dequantize(dev(q), s, zp)
        same_bits(host(y), oracle.dequantize(q, s, zp))


@pytest.mark.parametrize("dt,zp", [(np.int8, 0.0), (np.uint8, 128.0), (np.int32, -7.0)])
@pytest.mark.parametrize("K", [4096, 4100, 11008])
def test_dequantize_long_rows(ops, oracle, dt, zp, K):
    """Rows of 4096 elements and more take the 512-thread form (two
    4-element groups per lane); 4100 and 11008 leave a partial last pass."""
    rng = np.random.default_rng(K)
    if dt == np.int32:
        q = rng.integers(-2 ** 31, 2 ** 31, size=(3, K), dtype=np.int64).astype(np.int32)
    else:
        info = np.iinfo(dt)
        q = rng.integers(info.min, info.max + 1, size=(3, K)).astype(dt)
    s = 0.0012345678901234
    same_bits(host(ops.dequantize(dev(q), s, zp)), oracle.dequantize(q, s, zp))
    if dt == np.int8:
        rows = oracle.Rng(K).uniform((3,), 0.001, 0.1).astype(np.float64)
        same_bits(host(ops.dequantize(dev(q), dev(rows))), oracle.dequantize_rows(q, rows))


def test_dequantize_scalar_path(ops, oracle):
    q = np.random.default_rng(1).integers(-128, 128, size=(5, 13)).astype(np.int8)
    s = oracle.Rng(9).uniform((5,), 0.001, 0.1).astype(np.float64)
    y = ops.dequantize(dev(q), dev(s))
    same_bits(host(y), oracle.dequantize_rows(q, s))


# ------------------------------------------------------------------ weights
@pytest.mark.parametrize("shape,axis", [((64, 128), 0), ((128, 64), 1), ((4096, 4096), 1),
                                        ((10, 128), 0), ((97, 130), 1), ((3, 0), 0)])
def test_pack_weight_per_channel(ops, oracle, shape, axis):
    W = oracle.Rng(7).normal(shape, 0.0, 0.02)
    if W.size > 20:
        W.reshape(-1)[5] = np.nan
        W.reshape(-1)[11] = 0.3
    if shape == (10, 128):
        W[2, :] = 0.25                         # constant channel: +-0.5 expansion
        W[3, :] = 0.0
        W[4, 7] = np.inf
    Wq, s = ops.pack_weight(dev(W), axis=axis)
    s_ref = oracle.scales_per_channel(W, axis)
    q_ref = oracle.weight_quantize_per_channel(W, axis, s_ref)
    same_bits(host(s), s_ref)
    same_bits(host(Wq), q_ref if axis == 0 else q_ref.T.copy())


def test_pack_weight_per_tensor(ops, oracle):
    W = oracle.Rng(8).normal((96, 200), 0.0, 1.0)
    Wq, s = ops.pack_weight(dev(W), axis=0, granularity="per_tensor")
    s_ref = oracle.scale_const_array(W)
    same_bits(host(s), np.array([s_ref]))
    same_bits(host(Wq), oracle.weight_quantize_per_tensor(W, s_ref, -127, 127))


# ------------------------------------------------------------------ matmul
def rand_i8(rng, shape):
    return rng.integers(-128, 128, size=shape).astype(np.int8)


@pytest.mark.parametrize("M,N,K", [(32, 64, 128), (17, 33, 48), (256, 256, 784),
                                   (64, 10, 128), (300, 260, 1040), (128, 128, 4096),
                                   (20, 30, 7)])
def test_quantized_dot_small(ops, oracle, M, N, K):
    rng = np.random.default_rng(M * 7 + N)
    A, B = rand_i8(rng, (M, K)), rand_i8(rng, (N, K))
    acc = ops.quantized_dot(dev(A), dev(B))
    same_bits(host(acc), oracle.quantized_dot(A, B, b_layout=1))


def test_generic_gemm_route_is_counted(ops, oracle):
    """K % 16 != 0 takes the generic kernel (exact) and is counted; an
    MFMA-shaped call is not."""
    rng = np.random.default_rng(41)
    before = ops.generic_gemm_launches()
    A = rng.integers(-128, 128, (40, 40)).astype(np.int8)
    B = rng.integers(-128, 128, (24, 40)).astype(np.int8)
    same_bits(host(ops.quantized_dot(dev(A), dev(B))), oracle.quantized_dot(A, B, b_layout=1))
    assert ops.generic_gemm_launches() == before + 1
    A = rng.integers(-128, 128, (40, 64)).astype(np.int8)
    B = rng.integers(-128, 128, (24, 64)).astype(np.int8)
    same_bits(host(ops.quantized_dot(dev(A), dev(B))), oracle.quantized_dot(A, B, b_layout=1))
    assert ops.generic_gemm_launches() == before + 1


@pytest.mark.parametrize("M,N,K", [(1024, 1024, 4096), (2048, 4096, 4096), (768, 1280, 11008),
                                   (4096, 4096, 4096), (4001, 3100, 2048), (4001, 3099, 2064),
                                   (1000, 1001, 4112), (513, 4095, 272), (2048, 12288, 4096),
                                   (100, 3000, 16), (3000, 100, 32),
                                   # 256 x 192 tiles (whole rounds at N = 6144 / 12288), partial in M and N
                                   (1000, 12100, 4096), (2048, 6144, 4096)])
def test_quantized_dot_large_exact(ops, M, N, K):
    """Large shapes: integer products and sums are exact in f64 (|acc| < 2^53),
    so an f64 matmul of the same int8 values is an exact closed-form check."""
    g = torch.Generator(device=DEV).manual_seed(M + N + K)
    A = torch.randint(-128, 128, (M, K), dtype=torch.int8, device=DEV, generator=g)
    B = torch.randint(-128, 128, (N, K), dtype=torch.int8, device=DEV, generator=g)
    acc = ops.quantized_dot(A, B)
    ref = (A.double() @ B.double().t().contiguous())
    torch.cuda.synchronize()
    assert torch.equal(acc.double(), ref)


def test_quantized_dot_wraps_like_int32(ops, oracle):
    # |acc| up to K * 128 * 128 = 2^31 at K = 2^17: the JS accumulator is exact
    # and the Int32Array store wraps; the GPU's int32 accumulation wraps the same.
    K = 1 << 17
    A = np.full((2, K), -128, np.int8)
    B = np.full((2, K), -128, np.int8)
    B[1, :] = 127
    acc = ops.quantized_dot(dev(A), dev(B))
    same_bits(host(acc), oracle.quantized_dot(A, B, b_layout=1))


@pytest.mark.parametrize("act", [None, "relu", "silu"])
@pytest.mark.parametrize("M,N,K", [(64, 96, 256), (300, 130, 512), (4, 200, 4096),
                                   (257, 131, 144), (1030, 2050, 1024), (33, 4099, 784)])
def test_qlinear_rowcol_epilogue(ops, oracle, M, N, K, act):
    rng = oracle.Rng(M + N)
    x = rng.normal((M, K))
    W = rng.normal((N, K), 0.0, 0.02)
    bias = rng.uniform((N,), -0.1, 0.1)
    sx = oracle.scales_per_token(x)
    xq = oracle.quantize_rows(x, sx)
    sw = oracle.scales_per_channel(W, 0)
    Wq = oracle.weight_quantize_per_channel(W, 0, sw)
    y = ops.qlinear(dev(xq), dev(sx), dev(Wq), dev(sw), bias=dev(bias), act=act)
    acc = oracle.quantized_dot(xq, Wq, b_layout=1)
    ref = oracle.epilogue(acc, "rowcol", sx, sw, bias=bias, act=act or "none")
    same_bits(host(y), ref)


def test_qlinear_pertensor_scales(ops, oracle):
    rng = oracle.Rng(44)
    x = rng.normal((40, 128))
    W = rng.normal((64, 128), 0.0, 0.02)
    sx = np.array([oracle.scale_per_tensor(x)])
    xq = oracle.quantize(x, sx[0])
    sw = oracle.scales_per_channel(W, 0)
    Wq = oracle.weight_quantize_per_channel(W, 0, sw)
    y = ops.qlinear(dev(xq), dev(sx), dev(Wq), dev(sw))
    acc = oracle.quantized_dot(xq, Wq, b_layout=1)
    same_bits(host(y), oracle.epilogue(acc, "rowcol", sx[0], sw))


@pytest.mark.parametrize("M,N,K", [(2000, 3000, 1024), (4096, 4096, 4096), (515, 517, 528),
                                   (1000, 12100, 1024), (2048, 6144, 4096)])   # the last two: 256 x 192 tiles
def test_qlinear_large_rowcol_exact(ops, oracle, M, N, K):
    """Full-size epilogue check: accumulators from an exact f64 matmul of the
    same int8 values, then the oracle epilogue on every element."""
    g = torch.Generator(device=DEV).manual_seed(M * 3 + N)
    A = torch.randint(-128, 128, (M, K), dtype=torch.int8, device=DEV, generator=g)
    B = torch.randint(-128, 128, (N, K), dtype=torch.int8, device=DEV, generator=g)
    sA = torch.rand(M, dtype=torch.float64, device=DEV, generator=g) * 1e-2 + 1e-4
    sB = torch.rand(N, dtype=torch.float64, device=DEV, generator=g) * 1e-3 + 1e-5
    bias = torch.rand(N, dtype=torch.float32, device=DEV, generator=g) - 0.5
    y = ops.qlinear(A, sA, B, sB, bias=bias)
    acc = (A.double() @ B.double().t().contiguous()).to(torch.int32)
    ref = oracle.epilogue(host(acc), "rowcol", host(sA), host(sB), bias=host(bias))
    same_bits(host(y), ref)


@pytest.mark.parametrize("M,N,K", [(300, 260, 4096), (8, 300, 4096), (2, 77, 8192), (1024, 6144, 4096)])
def test_qlinear_large_accumulators(ops, oracle, M, N, K):
    """Saturated rows and columns (|acc| up to K * 128 * 128 = 2^26 at
    K = 4096, beyond 2^24 where an int32 stops being exactly a binary32):
    the epilogue's f64 path, in strips that also hold small accumulators,
    on the MFMA GEMM (M > 16) and the GEMV kernels."""
    g = torch.Generator(device=DEV).manual_seed(M + N + K)
    A = torch.randint(-128, 128, (M, K), dtype=torch.int8, device=DEV, generator=g)
    B = torch.randint(-128, 128, (N, K), dtype=torch.int8, device=DEV, generator=g)
    A[0, :] = 127
    A[M - 1, :] = -128
    B[:5, :] = 127
    B[5:9, :] = -128
    B[N - 1, : K // 2] = -128
    sA = torch.rand(M, dtype=torch.float64, device=DEV, generator=g) * 1e-2 + 1e-4
    sB = torch.rand(N, dtype=torch.float64, device=DEV, generator=g) * 1e-3 + 1e-5
    bias = torch.rand(N, dtype=torch.float32, device=DEV, generator=g) - 0.5
    for act in (None, "silu"):
        y = ops.qlinear(A, sA, B, sB, bias=bias, act=act)
        acc = (A.double() @ B.double().t().contiguous()).to(torch.int32)
        a = host(acc)
        assert np.abs(a).max() > (1 << 24)
        ref = oracle.epilogue(a, "rowcol", host(sA), host(sB), bias=host(bias), act=act or "none")
        same_bits(host(y), ref)


def test_qlinear_pt_epilogue(ops, oracle):
    rng = np.random.default_rng(3)
    A, B = rand_i8(rng, (48, 256)), rand_i8(rng, (72, 256))
    s_out = (5 / 127) * (6 / 127)
    y = ops.qlinear_pt(dev(A), dev(B), s_out)
    acc = oracle.quantized_dot(A, B, b_layout=1)
    same_bits(host(y), oracle.epilogue(acc, "pt", s_out=s_out))


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 9, 13, 15, 16])
@pytest.mark.parametrize("N,K", [(4096, 4096), (1000, 4096), (77, 8192 + 512), (11008, 4096),
                                 (5, 16), (33, 16400)])
def test_gemv(ops, oracle, M, N, K):
    rng = oracle.Rng(M * 31 + N)
    x = rng.normal((M, K))
    W = rng.normal((N, K), 0.0, 0.02)
    sx = oracle.scales_per_token(x)
    xq = oracle.quantize_rows(x, sx)
    sw = oracle.scales_per_channel(W, 0)
    Wq = oracle.weight_quantize_per_channel(W, 0, sw)
    y = ops.qlinear(dev(xq), dev(sx), dev(Wq), dev(sw))
    acc = oracle.quantized_dot(xq, Wq, b_layout=1)
    same_bits(host(y), oracle.epilogue(acc, "rowcol", sx, sw))
    acc_gpu = ops.quantized_dot(dev(xq), dev(Wq))
    same_bits(host(acc_gpu), acc)


@pytest.mark.parametrize("M", [9, 16])
def test_gemv_sixteen_wave_route(ops, oracle, M):
    """More row blocks than two per CU and more than 8 tokens: one 16-wave
    workgroup per CU walks the row blocks; N not a multiple of 16, K = 11008
    in three passes of 4096 (the last one partial), bias and SiLU."""
    N, K = 9001, 11008
    rng = oracle.Rng(M * 7 + 11)
    x = rng.normal((M, K))
    W = rng.normal((N, K), 0.0, 0.02)
    bias = rng.uniform((N,), -0.1, 0.1)
    sx = oracle.scales_per_token(x)
    xq = oracle.quantize_rows(x, sx)
    sw = oracle.scales_per_channel(W, 0)
    Wq = oracle.weight_quantize_per_channel(W, 0, sw)
    acc = oracle.quantized_dot(xq, Wq, b_layout=1)
    y = ops.qlinear(dev(xq), dev(sx), dev(Wq), dev(sw), bias=dev(bias), act="silu")
    same_bits(host(y), oracle.epilogue(acc, "rowcol", sx, sw, bias=bias, act="silu"))
    same_bits(host(ops.quantized_dot(dev(xq), dev(Wq))), acc)


# ------------------------------------------------------------------ fused / inputs
@pytest.mark.parametrize("M,K", [(4, 11008), (3, 1000), (2, 64), (2, 8192), (3, 6000), (2, 12288)])
def test_silu_mul_quantize(ops, oracle, M, K):
    rng = oracle.Rng(K)
    g = rng.normal((M, K), 0.0, 3.0)
    u = rng.normal((M, K))
    g.reshape(-1)[:4] = [0.0, -0.0, 88.0, -104.0]
    h_out = torch.empty((M, K), dtype=torch.float32, device=DEV)
    q, s = ops.silu_mul_quantize(dev(g), dev(u), h_out)
    h = oracle.silu_mul(g, u)
    same_bits(host(h_out), h)
    s_ref = oracle.scales_per_token(h)
    same_bits(host(s), s_ref)
    same_bits(host(q), oracle.quantize_rows(h, s_ref))



@pytest.mark.parametrize("M,K,pad", [(4, 11008, 11008), (3, 1000, 1000), (2, 64, 4), (3, 6000, 2), (2, 30, 3)])
def test_silu_mul_quantize_strided(ops, oracle, M, K, pad):
    """g and u as row-strided views: the two halves of one [M, 2K] output
    (pad = K) or of a wider buffer; odd strides take the scalar kernel."""
    rng = oracle.Rng(K + pad)
    g = rng.normal((M, K), 0.0, 3.0)
    u = rng.normal((M, K))
    buf = np.zeros((M, 2 * K + pad), np.float32)
    buf[:, :K] = g
    buf[:, K + pad:] = u
    d = dev(buf)
    gv, uv = d[:, :K], d[:, K + pad:]
    assert not gv.is_contiguous() and gv.stride(0) == 2 * K + pad
    h_out = torch.empty((M, K), dtype=torch.float32, device=DEV)
    q, s = ops.silu_mul_quantize(gv, uv, h_out)
    h = oracle.silu_mul(g, u)
    same_bits(host(h_out), h)
    s_ref = oracle.scales_per_token(h)
    same_bits(host(s), s_ref)
    same_bits(host(q), oracle.quantize_rows(h, s_ref))

@pytest.mark.parametrize("M,K,off,tail", [(5, 4096, 8192, 0), (3, 1000, 3, 1), (7, 64, 4, 0),
                                          (2, 30, 1, 2), (4, 20000, 4, 4)])
def test_quantize_per_token_strided(ops, oracle, M, K, off, tail):
    """x as a column slice of a wider buffer (the V third of a fused qkv
    output is off = 2K of a [M, 3K] row); odd strides take the scalar kernel.
    A zero row and a row with one large outlier are included."""
    rng = oracle.Rng(K + off)
    x = rng.normal((M, K))
    x[0] = 0.0
    x[-1, K // 2] = 5000.0
    buf = rng.normal((M, off + K + tail))
    buf[:, off:off + K] = x
    d = dev(buf)
    v = d[:, off:off + K]
    assert not v.is_contiguous() and v.stride(0) == off + K + tail
    q, s = ops.quantize_per_token(v)
    s_ref = oracle.scales_per_token(x)
    same_bits(host(s), s_ref)
    same_bits(host(q), oracle.quantize_rows(x, s_ref))
    q2, s2 = ops.quantize_per_token(v.contiguous())
    same_bits(host(q), host(q2))
    with pytest.raises(ValueError):
        ops.quantize_per_token(d.t()[:K])                 # column stride != 1


def test_fill_uniform_matches_oracle(ops, oracle):
    r = oracle.Rng(11)
    ref = r.uniform((10001,), -0.1, 0.1)
    t = torch.empty(10001, dtype=torch.float32, device=DEV)
    ops.fill_uniform(t, 11, 0, -0.1, 0.1)
    same_bits(host(t), ref)


def test_fill_normal_matches_oracle(ops, oracle):
    """mulberry32 draws are integer-exact; Box-Muller uses log/cos/sin, which
    the device libm and glibc may round differently in the last f64 bit.
    After the f32 rounding nearly every value is identical; the rest differ
    by one f32 ulp."""
    r = oracle.Rng(5)
    _ = r.normal((1001,))                 # consume 1002 draws: offset test
    ref = r.normal((200001,), 0.0, 0.02)
    t = torch.empty(200001, dtype=torch.float32, device=DEV)
    ops.fill_normal(t, 5, 1002, 0.0, 0.02)
    got = host(t)
    diff = np.abs(got.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert diff.max() <= 1
    assert (diff != 0).mean() < 1e-3
