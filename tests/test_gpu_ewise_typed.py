"""q8_ewise's compiled programs against its interpreter on every binary32
input, for the instruction forms the compiled kernels evaluate in binary32
or through a reciprocal instead of in f64.

The interpreter evaluates every instruction in f64 and rounds a `rnd`
instruction's value once to binary32: the reference CPU backend's JS
(src/backend/cpu/codegen.ts:428-552; Math.fround around f32-typed
arithmetic).  The compiled kernels hold binary32-exact values as float and
run max / min / abs / neg / floor / ceil / round / sign / compare / ToInt32
and the rounded + - * / of two binary32 operands in binary32, and a rounded
division by a constant that is not binary32 as a product with the
constant's reciprocal, checked against the binary32 rounding midpoints (the
true division where the check fails).  Each program below runs over all
2^32 bit patterns of x as a [2^32] f32 input (in chunks), once on each
route, and the outputs must be equal bit for bit (any NaN equal to any NaN
in f32 outputs: the reference's values are JS numbers, whose NaN has no
payload).  The divisors cover a decimal scale (0.05, the bench program's),
values whose reciprocal is inexact both ways, a power of two, a binary32
divisor (the binary32 division), and divisors that push quotients out of
the binary32 range (overflow to infinity, underflow to subnormals and
zero)."""
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
CHUNK = 1 << 26


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from mlfw_amd import ops as O
    from mlfw_amd import _lib
    _lib.call("q8_init", 0)
    return O


def set_route(mode):
    from mlfw_amd import _lib
    _lib.call("q8_debug_ewise_jit", mode, None, None)


def f32(v):
    return float(torch.tensor(v, dtype=torch.float32).item())


def compare_all_inputs(ops, code, konst, out_dtype, what):
    """Runs `code` (register 0 = x, the loaded input) over every binary32 x
    on both routes and compares the outputs."""
    prog = ops.ew_program((CHUNK,), [(torch.float32, (1,))], [("load", 0, 0, 0, 0, 0, 0)] + code,
                          code[-1][1], out_dtype, konst=konst)
    base = torch.arange(CHUNK, dtype=torch.int64, device=DEV)
    a = torch.empty(CHUNK, dtype=out_dtype, device=DEV)
    b = torch.empty(CHUNK, dtype=out_dtype, device=DEV)
    ndiff = 0
    first = None
    try:
        for c in range((1 << 32) // CHUNK):
            u = base + c * CHUNK
            x = torch.where(u >= 1 << 31, u - (1 << 32), u).to(torch.int32).view(torch.float32)
            set_route(1)
            ops.ewise(prog, [x], a)
            set_route(2)
            ops.ewise(prog, [x], b)
            if out_dtype == torch.float32:
                ne = (a.view(torch.int32) != b.view(torch.int32)) & ~(torch.isnan(a) & torch.isnan(b))
            else:
                ne = a != b
            k = int(ne.sum().item())
            if k and first is None:
                i = int(torch.nonzero(ne)[0].item())
                first = (hex(int(x.view(torch.int32)[i].item()) & 0xFFFFFFFF), a[i].item(), b[i].item())
            ndiff += k
    finally:
        set_route(0)
    assert ndiff == 0, f"{what}: {ndiff} of 2^32 inputs differ; first (x bits, interpreted, compiled): {first}"


@pytest.mark.parametrize("c", [0.05, 0.1, 1.0 / 3.0, 0.007, 1e-3, 2.5e-3, 0.125, 7.0, -0.3, 1e-30, 3e36])
def test_rounded_division_by_a_constant(ops, c):
    """fround(x / c): the reciprocal route (c not binary32) or the binary32
    division (c = 0.125, 7)."""
    print(f"fround(x / {c!r}) over every binary32 x", flush=True)
    compare_all_inputs(ops, [("const", 1, 0, 0, 0, 0, 0), ("div", 2, 0, 1, 0, 0, 1)], (c,), torch.float32,
                       f"fround(x / {c!r})")


@pytest.mark.parametrize("op,k", [("add", 0.75), ("add", f32(1e-40)), ("sub", -3.0), ("mul", f32(0.1)),
                                  ("mul", f32(3e-39)), ("div", f32(0.1))])
def test_rounded_binary32_arithmetic(ops, op, k):
    """fround(x op k) for binary32 k: the binary32 operation (subnormal
    constants and results included)."""
    print(f"fround(x {op} {k!r}) over every binary32 x", flush=True)
    compare_all_inputs(ops, [("const", 1, 0, 0, 0, 0, 0), (op, 2, 0, 1, 0, 0, 1)], (k,), torch.float32,
                       f"fround(x {op} {k!r})")


def test_rounded_square(ops):
    print("fround(x * x) over every binary32 x", flush=True)
    compare_all_inputs(ops, [("mul", 1, 0, 0, 0, 0, 1)], (), torch.float32, "fround(x * x)")


def test_relu_quantize_program(ops):
    """bench.py's ReLU fused with quantize, (min(max(Math.round(
    Math.fround(max(x, 0) / 0.05)), -128), 127) | 0), int8 out."""
    print("relu_quantize over every binary32 x", flush=True)
    code = [("const", 1, 0, 0, 0, 0, 0), ("max", 2, 0, 1, 0, 0, 0), ("const", 3, 0, 0, 0, 1, 0),
            ("div", 4, 2, 3, 0, 0, 1), ("round", 5, 4, 0, 0, 0, 0), ("const", 6, 0, 0, 0, 2, 0),
            ("max", 7, 5, 6, 0, 0, 0), ("const", 8, 0, 0, 0, 3, 0), ("min", 9, 7, 8, 0, 0, 0),
            ("toint32", 10, 9, 0, 0, 0, 0)]
    compare_all_inputs(ops, code, (0.0, 0.05, -128.0, 127.0), torch.int8, "relu_quantize")


QUANT_CHAIN = [("const", 1, 0, 0, 0, 0, 0), ("div", 2, 0, 1, 0, 0, 1), ("round", 3, 2, 0, 0, 0, 0),
               ("const", 4, 0, 0, 0, 1, 0), ("max", 5, 3, 4, 0, 0, 0), ("const", 6, 0, 0, 0, 2, 0),
               ("min", 7, 5, 6, 0, 0, 0), ("toint32", 8, 7, 0, 0, 0, 0)]


@pytest.mark.parametrize("s", [1e-3, 0.1, 1.0 / 3.0, 7.0, 2.0 ** -100, 2.0 ** 100, 6e-31])
def test_quantize_chain(ops, s):
    """QuantizationPass's int8 quantize, (min(max(Math.round(Math.fround(x /
    s)), -128), 127) | 0): the compiled kernels run the chain as the
    library's quantize fast path (binary32 product with 1/s, exact f64 steps
    near rounding ties) for s in [2^-100, 2^100] -- both ends included --
    and as the separate steps for s outside it (6e-31)."""
    print(f"quantize chain s={s!r} over every binary32 x", flush=True)
    compare_all_inputs(ops, QUANT_CHAIN, (s, -128.0, 127.0), torch.int8, f"quantize s={s!r}")


def test_quantize_chain_not_fused(ops):
    """Chains the fusion must leave alone, on every binary32 x: the rounded
    quotient read again after the chain (added to the code), and a clamp to
    [0, 255] (a u8 range, not the int8 one)."""
    print("quantize chain variants over every binary32 x", flush=True)
    reused = QUANT_CHAIN[:-1] + [("toint32", 8, 7, 0, 0, 0, 0), ("add", 9, 8, 2, 0, 0, 0)]
    compare_all_inputs(ops, reused, (0.05, -128.0, 127.0), torch.int32, "quantize + quotient")
    compare_all_inputs(ops, QUANT_CHAIN, (0.05, 0.0, 255.0), torch.uint8, "quantize to [0, 255]")


@pytest.mark.parametrize("op", ["round", "floor", "ceil", "sign", "abs", "neg"])
def test_exact_unary_ops(ops, op):
    """Exact unary ops on binary32 values, stored as f32 (-0 and NaN kept)."""
    print(f"{op}(x) over every binary32 x", flush=True)
    compare_all_inputs(ops, [(op, 1, 0, 0, 0, 0, 0)], (), torch.float32, f"{op}(x)")


@pytest.mark.parametrize("out", ["i32", "u8"])
def test_toint32_of_binary32(ops, out):
    """ToInt32 of every binary32 value (NaN, infinities, |x| >= 2^31 wrap
    mod 2^32), stored as Int32Array or Uint8Array."""
    print(f"x | 0 -> {out} over every binary32 x", flush=True)
    dt = torch.int32 if out == "i32" else torch.uint8
    compare_all_inputs(ops, [("toint32", 1, 0, 0, 0, 0, 0)], (), dt, f"x | 0 ({out})")


@pytest.mark.parametrize("op,k", [("max", 0.0), ("max", -0.0), ("min", 0.0), ("min", -1.5)])
def test_max_min_with_signed_zero(ops, op, k):
    """Math.max / Math.min against +-0 and a negative constant (NaN wins,
    +0 above -0)."""
    print(f"{op}(x, {k!r}) over every binary32 x", flush=True)
    compare_all_inputs(ops, [("const", 1, 0, 0, 0, 0, 0), (op, 2, 0, 1, 0, 0, 0)], (k,), torch.float32,
                       f"{op}(x, {k!r})")
