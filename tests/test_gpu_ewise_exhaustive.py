"""q8_ewise's exp / log / tanh externs against the reference's own engine on
every one of the 2^32 binary32 inputs.

The reference's CPU backend emits an f32-typed exp, log or tanh extern as
Math.fround(Math.<fn>(x)) (src/backend/cpu/codegen.ts:534; the expected
string 'Math.fround(Math.exp(x))' of codegen-internals.test.js), and V8
computes Math.exp / log / tanh in f64 with its own approximations, which
ECMA-262 does not fix.  tests/golden/ewise_v8_hashes.json holds, per chunk
of 2^24 consecutive bit patterns, two hashes of those outputs as V8 (Node
v12.22.9) gives them (tests/golden/ewise_v8_hashes.js, run by
make_ewise_v8_hashes.py).  Here the device evaluates the same inputs
through the C ABI: q8_ewise with the one-instruction program a JS
PrimFunc `out[i] = exp(in[i])` translates to (LOAD, then EXP / LOG / TANH
rounded to binary32), and the same hashes are taken on the device.  Equal
hashes on all 256 chunks: the device's bits equal V8's (any NaN counted as
one NaN) for every input, on both of q8_ewise's routes (the interpreter and
the hiprtc-compiled program)."""
import ctypes as C
import json
import os

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
M32 = 0xFFFFFFFF
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "ewise_v8_hashes.json")

# include/q8hip.h: the q8_ew_prog layout and opcodes
MAX_DIMS, MAX_INPUTS, MAX_CODE, MAX_CONST = 6, 8, 96, 32
EW_LOAD, EW_EXP, EW_LOG, EW_TANH = 0, 26, 27, 28
Q8_F32 = 3


class Instr(C.Structure):
    _fields_ = [(n, C.c_uint8) for n in ("op", "dst", "a", "b", "c", "aux", "rnd", "pad")]


class Prog(C.Structure):
    _fields_ = [("ndims", C.c_int32), ("ninputs", C.c_int32), ("extent", C.c_int64 * MAX_DIMS),
                ("in_dtype", C.c_int32 * MAX_INPUTS), ("in_coef", (C.c_int64 * (MAX_DIMS + 1)) * MAX_INPUTS),
                ("out_dtype", C.c_int32), ("ncode", C.c_int32), ("result", C.c_int32), ("nconst", C.c_int32),
                ("code", Instr * MAX_CODE), ("konst", C.c_double * MAX_CONST)]


def unary_prog(op, n):
    """out[i] = fround(fn(in[i])) over a flat [n] f32 array."""
    p = Prog()
    p.ndims, p.ninputs = 1, 1
    p.extent[0] = n
    p.in_dtype[0] = Q8_F32
    p.in_coef[0][0] = 1
    p.out_dtype = Q8_F32
    p.code[0] = Instr(EW_LOAD, 0, 0, 0, 0, 0, 0, 0)
    p.code[1] = Instr(op, 1, 0, 0, 0, 0, 1, 0)
    p.ncode, p.result = 2, 1
    return p


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from mlfw_amd import _lib
    _lib.call("q8_init", 0)
    return _lib


def chunk_hash(h, w):
    """s1 = sum mix(v_i) * (2i + 1), s2 = sum mix(v_i), both mod 2^32, v_i the
    bits of h with NaN as 0x7fc00000 (ewise_v8_hashes.js)."""
    v = h.reshape(-1).view(torch.int32).to(torch.int64) & M32
    v = torch.where(torch.isnan(h.reshape(-1)), torch.full_like(v, 0x7FC00000), v)
    v = v ^ (v >> 16)
    v = (v * 0x7FEB352D) & M32
    v = v ^ (v >> 15)
    s1 = int(((v * w) & M32).sum().item()) & M32
    s2 = int(v.sum().item()) & M32
    return [s1, s2]


@pytest.mark.parametrize("route", [1, 2], ids=["interpreted", "compiled"])
@pytest.mark.parametrize("name,op", [("exp", EW_EXP), ("log", EW_LOG), ("tanh", EW_TANH)])
def test_ewise_extern_bits_equal_v8_on_every_input(lib, name, op, route):
    with open(GOLDEN) as f:
        golden = json.load(f)[name]
    assert len(golden) == 256
    n = 1 << 24
    prog = unary_prog(op, n)
    w = 2 * torch.arange(n, dtype=torch.int64, device=DEV) + 1
    bits = torch.arange(n, dtype=torch.int64, device=DEV)
    out = torch.empty(n, dtype=torch.float32, device=DEV)
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    lib.call("q8_debug_ewise_jit", route, None, None)      # q8_ewise's interpreter, or the compiled program
    bad = []
    try:
        chunks(lib, prog, bits, out, w, golden, n, stream, bad, name)
    finally:
        lib.call("q8_debug_ewise_jit", 0, None, None)
    assert not bad, f"{name}: {len(bad)} of 256 chunks differ from V8: {bad[:16]}"


def chunks(lib, prog, bits, out, w, golden, n, stream, bad, name):
    for c in range(256):
        x = ((bits + c * n) & M32)
        x = torch.where(x >= 1 << 31, x - (1 << 32), x).to(torch.int32).view(torch.float32)
        ins = (C.c_void_p * 1)(x.data_ptr())
        nums = (C.c_int64 * 1)(n)
        lib.call("q8_ewise", C.c_void_p(C.addressof(prog)), C.cast(ins, C.c_void_p), C.cast(nums, C.c_void_p),
                 C.c_void_p(out.data_ptr()), n, stream)
        if chunk_hash(out, w) != golden[c]:
            bad.append(c)
        if c % 64 == 63:
            print(f"{name} exhaustive: chunks 0..{c} done, {len(bad)} differ", flush=True)
