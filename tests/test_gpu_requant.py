"""GPU parity of the fused requant epilogue (q8_gemm_requant) against the oracle.

The expected int8 codes are the oracle's epilogue (E-rowcol / E-pt, bias,
activation) followed by the oracle's compiled quantize with the static
scale -- the two ops QuantizationPass's calibrated chain runs one after the
other -- compared bit for bit.  Shapes exercise the MFMA GEMM (interior and
edge tiles, N not a multiple of 4), both GEMV kernels and the generic
kernel (K not a multiple of 16); scales exercise ties, clamping and the
exact (non-fast-path) branch.  The C2 test runs the 3-layer MLP with every
requant fused and checks it against the dynamic per-tensor C2 output, with
the static scales calibrated on the same batch.
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
    bad = np.nonzero(a.view(np.uint8).reshape(-1, a.itemsize) != b.view(np.uint8).reshape(-1, b.itemsize))[0]
    if bad.size:
        i = np.unique(bad)[0]
        raise AssertionError(f"{np.unique(bad).size} of {a.size} differ; first at flat {i}: "
                             f"{a.reshape(-1)[i]!r} vs {b.reshape(-1)[i]!r}")


SHAPES = [(300, 264, 256), (257, 131, 64), (512, 512, 1024), (5, 1000, 4096), (1, 77, 256), (40, 36, 40)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("mode", ["rowcol", "pt"])
@pytest.mark.parametrize("bias,act", [(False, "none"), (True, "relu"), (True, "silu")])
def test_requant_matches_epilogue_then_quantize(ops, oracle, M, N, K, mode, bias, act):
    rng = np.random.default_rng(M * 7 + N + K + len(act))
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    B = rng.integers(-128, 128, (N, K)).astype(np.int8)
    sA = rng.random(M) * 1e-2 + 1e-4
    sB = rng.random(N) * 1e-3 + 1e-5
    s_out = 3.1e-5
    b = (rng.random(N).astype(np.float32) - 0.5) if bias else None
    acc = oracle.quantized_dot(A, B, b_layout=1)
    if mode == "rowcol":
        y = oracle.epilogue(acc, "rowcol", sA, sB, bias=b, act=act)
    else:
        y = oracle.epilogue(acc, "pt", s_out=s_out, bias=b, act=act)
    for s_next in (float(np.max(np.abs(y))) / 127 or 1e-3, float(np.max(np.abs(y))) / 300, 1e-200):
        print(f"requant M={M} N={N} K={K} {mode} bias={bias} {act} s_next={s_next:g}", flush=True)
        want = oracle.quantize(y.reshape(-1), s_next).reshape(M, N)
        bt = None if b is None else dev(b)
        if mode == "rowcol":
            got = ops.qlinear_requant(dev(A), dev(sA), dev(B), dev(sB), s_next, bias=bt, act=act)
        else:
            got = ops.qlinear_requant(dev(A), None, dev(B), None, s_next, bias=bt, act=act, s_out=s_out)
        same_bits(host(got), want)


@pytest.mark.parametrize("M,N,K", [(300, 260, 4096), (1030, 520, 4096)])
@pytest.mark.parametrize("bias,act", [(False, "none"), (True, "relu"), (True, "silu")])
def test_requant_large_accumulators(ops, oracle, M, N, K, bias, act):
    """Saturated rows and columns (|acc| up to 2^26, past 2^24 where the
    binary32 multiply of the epilogue stops being exact): the f64 path of the
    static-requant epilogue, in quads that also hold small accumulators, on
    the 128 x 128 and 256 x 256 tiles."""
    rng = np.random.default_rng(M + N + len(act))
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    B = rng.integers(-128, 128, (N, K)).astype(np.int8)
    A[0, :] = 127
    A[M - 1, :] = -128
    B[:5, :] = 127
    B[N - 1, : K // 2] = -128
    sA = rng.random(M) * 1e-4 + 1e-6
    sB = rng.random(N) * 1e-3 + 1e-5
    b = (rng.random(N).astype(np.float32) - 0.5) if bias else None
    acc = (A.astype(np.float64) @ B.T.astype(np.float64)).astype(np.int32)
    assert np.abs(acc).max() > (1 << 24)
    y = oracle.epilogue(acc, "rowcol", sA, sB, bias=b, act=act)
    s_next = float(np.max(np.abs(y))) / 127
    got = ops.qlinear_requant(dev(A), dev(sA), dev(B), dev(sB), s_next, bias=None if b is None else dev(b),
                              act=None if act == "none" else act)
    same_bits(host(got), oracle.quantize(y.reshape(-1), s_next).reshape(M, N))


def test_c2_with_fused_static_requant_equals_dynamic_c2(ops, oracle):
    """C2 (784 -> 256 -> 128 -> 10, ReLU, per-tensor requant between layers)
    run with the requant of layers 1 and 2 fused into the GEMM epilogue.
    The static scales come from a calibration pass over the same batch
    (absmax / 127 of each layer's fp32 output), so the fused network must
    reproduce the dynamic per-tensor C2 exactly."""
    from oracle import configs as OC
    inp, y_ref = OC.c2()
    x = inp["x"]
    packed = [OC.pack_pc(W, 0) for W in inp["W"]]
    # calibration (oracle): per-tensor scale of each layer's input
    scales = []
    h = x
    for i, (Wq, sW) in enumerate(packed):
        s = oracle.scale_per_tensor(h)
        scales.append(s)
        hq = oracle.quantize(h.reshape(-1), s).reshape(h.shape)
        acc = oracle.quantized_dot(hq, Wq, b_layout=1)
        h = oracle.epilogue(acc, "rowcol", np.array([s]), sW, act="relu" if i < 2 else "none")
    same_bits(h, y_ref)
    # device: quantize the input once, then two fused GEMMs and the last fp32 one
    hq = ops.quantize(dev(x), scales[0])
    for i in range(2):
        Wq, sW = packed[i]
        hq = ops.qlinear_requant(hq, dev(np.array([scales[i]])), dev(Wq), dev(sW), scales[i + 1],
                                 act="relu")
    Wq, sW = packed[2]
    y = ops.qlinear(hq, dev(np.array([scales[2]])), dev(Wq), dev(sW))
    same_bits(host(y), y_ref)


# ------------------------------------------------------------ dynamic per-row requant
DYN_SHAPES = [(2048, 4096, 4096),   # C4's O projection: 128 co-resident tiles, fused route
              (300, 520, 1024),     # edge tiles in both dimensions, N % 4 == 0
              (257, 131, 64),       # N not a multiple of 4 (scalar stores)
              (12, 900, 4096),      # GEMV route (fp32 in the workspace, then quantize_rows)
              (4096, 8192, 256),    # 512 tiles: more than fit the chip, fallback route
              (64, 96, 40)]         # K not a multiple of 16


@pytest.mark.parametrize("M,N,K", DYN_SHAPES)
@pytest.mark.parametrize("bias,act", [(False, "none"), (True, "relu"), (True, "silu")])
def test_requant_dynamic_matches_epilogue_then_quantize_rows(ops, oracle, M, N, K, bias, act):
    if M * N * K > 2048 * 4096 * 4096 // 4 and (bias, act) != (False, "none"):
        pytest.skip("the full-size shape runs once, without bias")
    rng = np.random.default_rng(M + 3 * N + 7 * K + len(act))
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    B = rng.integers(-128, 128, (N, K)).astype(np.int8)
    sA = (rng.random(M) * 0.01 + 1e-4).astype(np.float64)
    sB = (rng.random(N) * 1e-3 + 1e-5).astype(np.float64)
    b = (rng.standard_normal(N) * 0.5).astype(np.float32) if bias else None
    # a row of saturating accumulators (|acc| > 2^24: the f64 epilogue path)
    A[1, :] = 127
    B[3, :] = 127
    q, s = ops.qlinear_requant_dynamic(dev(A), dev(sA), dev(B), dev(sB),
                                       bias=dev(b) if bias else None, act=None if act == "none" else act)
    if M * N * K > 1 << 30:
        # exact: |acc| <= 4096 * 128 * 128 < 2^53
        acc = (A.astype(np.float64) @ B.T.astype(np.float64)).astype(np.int32)
    else:
        acc = oracle.quantized_dot(A, B, b_layout=1)
    y = oracle.epilogue(acc, "rowcol", sA, sB, bias=b, act=act)
    s_ref = oracle.scales_per_token(y)
    same_bits(host(s), s_ref)
    same_bits(host(q), oracle.quantize_rows(y, s_ref))


def test_requant_dynamic_routes_and_status(ops):
    from mlfw_amd import _lib
    import ctypes as C
    nb, fused = ops.requant_dynamic_workspace(2048, 4096, 4096)
    assert fused and nb < 64 * 1024, (nb, fused)
    nb, fused = ops.requant_dynamic_workspace(4096, 8192, 256)
    assert not fused and nb >= 4096 * 8192 * 4
    nb, fused = ops.requant_dynamic_workspace(12, 900, 4096)
    assert not fused
    # the fused route's bounded wait did not run out
    M, N, K = 1024, 2048, 512
    rng = np.random.default_rng(5)
    A = dev(rng.integers(-128, 128, (M, K)).astype(np.int8))
    B = dev(rng.integers(-128, 128, (N, K)).astype(np.int8))
    sA = dev(np.full(M, 1e-3))
    sB = dev(np.full(N, 1e-3))
    nb, fused = ops.requant_dynamic_workspace(M, N, K)
    assert fused
    ws = torch.empty(nb, dtype=torch.int8, device=DEV)
    for _ in range(3):
        ops.qlinear_requant_dynamic(A, sA, B, sB, workspace=ws)
    flag = C.c_int(-1)
    _lib.call("q8_gemm_requant_dynamic_status", C.c_void_p(ws.data_ptr()), M, C.byref(flag),
              C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert flag.value == 0


def test_requant_dynamic_reports_a_timed_out_wait(ops):
    """The host-forced timeout (an arrival target the grid never reaches,
    a short bound): every workgroup's wait ends, the status word reports it,
    and the next ordinary call clears it and is exact again."""
    from mlfw_amd import _lib
    import ctypes as C
    M, N, K = 512, 1024, 256
    rng = np.random.default_rng(9)
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    B = rng.integers(-128, 128, (N, K)).astype(np.int8)
    sA, sB = np.full(M, 1e-3), np.full(N, 2e-3)
    nb, fused = ops.requant_dynamic_workspace(M, N, K)
    assert fused
    ws = torch.empty(nb, dtype=torch.int8, device=DEV)
    st = C.c_void_p(torch.cuda.current_stream().cuda_stream)

    def status():
        flag = C.c_int(-1)
        _lib.call("q8_gemm_requant_dynamic_status", C.c_void_p(ws.data_ptr()), M, C.byref(flag), st)
        return flag.value

    _lib.call("q8_debug_dq_force_timeout", 1)
    try:
        ops.qlinear_requant_dynamic(dev(A), dev(sA), dev(B), dev(sB), workspace=ws)
        assert status() == 1
        with pytest.raises(RuntimeError, match="wait ran out"):
            ops.qlinear_requant_dynamic(dev(A), dev(sA), dev(B), dev(sB), workspace=ws, check=True)
    finally:
        _lib.call("q8_debug_dq_force_timeout", 0)
    q, s = ops.qlinear_requant_dynamic(dev(A), dev(sA), dev(B), dev(sB), workspace=ws, check=True)
    assert status() == 0
    y = ops.qlinear(dev(A), dev(sA), dev(B), dev(sB))
    q_ref, s_ref = ops.quantize_per_token(y)
    same_bits(host(s), host(s_ref))
    same_bits(host(q), host(q_ref))
