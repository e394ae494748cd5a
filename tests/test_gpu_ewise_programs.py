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


def jit_counts():
    import ctypes as C
    from mlfw_amd import _lib
    compiled, launches = C.c_int64(0), C.c_int64(0)
    _lib.call("q8_debug_ewise_jit", -1, C.byref(compiled), C.byref(launches))
    return compiled.value, launches.value


def set_jit(mode):
    from mlfw_amd import _lib
    _lib.call("q8_debug_ewise_jit", mode, None, None)


def test_large_programs_run_compiled(ops, oracle):
    """Calls of 2^20 elements and more run the hiprtc-compiled kernel (the
    4096 x 4096 case above checks its values); here: that route is taken,
    and gives the interpreter's bits."""
    from mlfw_amd import configs as C
    set_jit(0)
    M = N = 1024
    prog, _, _, _ = C.ewise_programs(M, N)["relu_quantize"]
    x = torch.randn((M, N), device=DEV)
    c0, l0 = jit_counts()
    a = torch.empty((M, N), dtype=torch.int8, device=DEV)
    ops.ewise(prog, [x], a)
    torch.cuda.synchronize()
    c1, l1 = jit_counts()
    assert l1 == l0 + 1, f"a 2^20-element call should launch the compiled kernel: {ops.ewise_jit_error()!r}"
    set_jit(1)
    try:
        b = torch.empty_like(a)
        ops.ewise(prog, [x], b)
        torch.cuda.synchronize()
        assert jit_counts()[1] == l1
    finally:
        set_jit(0)
    same_bits(host(a), host(b), "compiled vs interpreted")


def test_program_first_seen_under_graph_capture(ops):
    """A program first called while its stream is captured into a HIP graph
    is not compiled there (the capture records the interpreter); the next
    eager call compiles it.  Every replay, with eager work between them,
    gives the compiled kernel's bits."""
    from mlfw_amd import configs as C
    set_jit(0)
    M = N = 1024
    prog, _, _, _ = C.ewise_programs(M, N, s_q=0.0371)["relu_quantize"]    # a scale no other test uses
    x = torch.randn((M, N), device=DEV)
    c0, l0 = jit_counts()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    out_g = torch.empty((M, N), dtype=torch.int8, device=DEV)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        ops.ewise(prog, [x], out_g)
    torch.cuda.synchronize()
    assert jit_counts() == (c0, l0), "no compile and no compiled launch while capturing"
    out_e = torch.empty_like(out_g)
    ops.ewise(prog, [x], out_e)
    torch.cuda.synchronize()
    c1, l1 = jit_counts()
    assert (c1, l1) == (c0 + 1, l0 + 1), ops.ewise_jit_error()
    for r in range(3):
        out_g.zero_()
        g.replay()
        torch.cuda.synchronize()
        same_bits(host(out_g), host(out_e), f"replay {r} (interpreter) vs eager (compiled)")
        ops.ewise(prog, [x], out_e)       # eager work between the replays
        torch.cuda.synchronize()


ALL_OPS = ["add", "sub", "mul", "div", "idiv", "mod", "floordiv", "tmod", "tdiv", "neg", "cmp", "select",
           "toint32", "tobool", "max", "min", "abs", "floor", "ceil", "round", "sign", "sqrt", "fmod", "exp",
           "log", "tanh", "rsqrt", "pow", "index", "const"]


def same_or_both_nan(a, b, what):
    a = np.ascontiguousarray(a).reshape(-1)
    b = np.ascontiguousarray(b).reshape(-1)
    ne = a.view(np.uint8).reshape(-1, a.itemsize) != b.view(np.uint8).reshape(-1, b.itemsize)
    ne = np.any(ne, axis=1)
    if a.dtype.kind == "f":
        ne &= ~(np.isnan(a) & np.isnan(b))
    bad = np.nonzero(ne)[0]
    assert bad.size == 0, f"{what}: {bad.size} differ; first {bad[0]}: {a[bad[0]]!r} vs {b[bad[0]]!r}"


@pytest.mark.parametrize("seed", range(16))
def test_random_programs_compiled_equal_interpreted(ops, seed):
    """Random programs over every opcode, input and output dtype, broadcast
    and strided inputs, three loops: the compiled kernel and the interpreter
    give the same bits (NaNs of float outputs compared as NaN: their
    payload is not part of the reference's result)."""
    rng = np.random.default_rng(seed)
    dts = [torch.int8, torch.uint8, torch.int32, torch.float32, torch.float64]
    # even seeds: the last extent a multiple of 4 (the four-elements-per-lane kernels)
    last = int(rng.integers(1, 18)) * 4 if seed % 2 == 0 else int(rng.integers(1, 70))
    E = (int(rng.integers(1, 9)), int(rng.integers(1, 40)), last)
    n_in = int(rng.integers(1, 5))
    inputs, tensors = [], []
    for j in range(n_in):
        dt = dts[int(rng.integers(0, len(dts)))]
        if j and rng.integers(0, 4) == 0:
            # the last two loops transposed in memory: read element by element
            coefs = [E[1] * E[2], 1, E[1]]
            numel = E[0] * E[1] * E[2]
        else:
            # contiguous, or broadcast over a random subset of the loops
            mask = [bool(rng.integers(0, 2)) if j else True for _ in range(3)]
            shape = [E[d] if mask[d] else 1 for d in range(3)]
            coefs, st = [0, 0, 0], 1
            for d in (2, 1, 0):
                if mask[d]:
                    coefs[d] = st
                st *= shape[d]
            numel = int(np.prod(shape))
        if dt.is_floating_point:
            v = rng.standard_normal(numel) * rng.choice([1.0, 1e3, 1e-3])
            v[rng.integers(0, numel, max(1, numel // 16))] = rng.choice(
                [np.nan, np.inf, -np.inf, 0.0, -0.0, 0.5, -2.5, 1e300 if dt == torch.float64 else 3e38])
            t = torch.tensor(v, dtype=dt, device=DEV)
        else:
            lo, hi = {torch.int8: (-128, 128), torch.uint8: (0, 256), torch.int32: (-2 ** 31, 2 ** 31)}[dt]
            t = torch.tensor(rng.integers(lo, hi, numel, dtype=np.int64), dtype=dt, device=DEV)
        inputs.append((dt, coefs + [0]))
        tensors.append(t)
    code, live = [], []
    for j in range(n_in):
        code.append(("load", j, 0, 0, 0, j, int(rng.integers(0, 2))))
        live.append(j)
    konst = [0.0, 1.0, -0.0, 0.5, 3.0, -7.25, 1e-30, 2.0 ** 40, np.nan, np.inf]
    for _ in range(int(rng.integers(4, 30))):
        op = ALL_OPS[int(rng.integers(0, len(ALL_OPS)))]
        dst = int(rng.integers(0, 16))
        a, b, c = (int(rng.choice(live)) for _ in range(3))
        aux = 0
        if op == "cmp":
            aux = int(rng.integers(0, 6))
        elif op == "index":
            aux = int(rng.integers(0, 3))
        elif op == "const":
            aux = int(rng.integers(0, len(konst)))
        code.append((op, dst, a, b, c, aux, int(rng.integers(0, 2))))
        if dst not in live:
            live.append(dst)
    out_dt = dts[int(rng.integers(0, len(dts)))]
    prog = ops.ew_program(E, inputs, code, code[-1][1], out_dt, konst=konst)
    outs = []
    try:
        for mode in (1, 2):
            set_jit(mode)
            o = torch.empty(E, dtype=out_dt, device=DEV)
            ops.ewise(prog, tensors, o)
            outs.append(host(o))
    finally:
        set_jit(0)
    same_or_both_nan(outs[1], outs[0], f"seed {seed}")
