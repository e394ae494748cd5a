"""The device SiLU (every GEMM / GEMV epilogue with act = SiLU and the
SiLU-up requant use the same function) against the reference's own SiLU on
every one of the 2^32 binary32 inputs.

The reference evaluates SiLU as decomposition_pass.ts:197-230 lowered by
its CPU backend: x * (1 / (1 + exp(-x))) with Math.fround at every f32 op
and Math.exp in f64.  tests/golden/silu_v8_hashes.json holds, per chunk of
2^24 consecutive bit patterns, two hashes of that function's output bits
as computed by V8 (tests/golden/silu_v8_hashes.js, run by
make_silu_v8_hashes.py).  Here the device evaluates the same inputs through
the C ABI -- q8_silu_mul_quantize_rows with u = 1, whose h output is
fround(silu(g) * 1) = silu(g) -- and the same hashes are taken on the device.
Equal hashes on all 256 chunks: the device's bits equal V8's (any NaN
counted as one NaN) for every input."""
import json
import os

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
M32 = 0xFFFFFFFF
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "silu_v8_hashes.json")


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from mlfw_amd import ops as O
    from mlfw_amd import _lib
    _lib.call("q8_init", 0)
    return O


def chunk_hash(h, w):
    """s1 = sum mix(v_i) * (2i + 1), s2 = sum mix(v_i), both mod 2^32 (the
    definitions of silu_v8_hashes.js), v_i the bits of h with NaN as
    0x7fc00000."""
    v = h.reshape(-1).view(torch.int32).to(torch.int64) & M32
    v = torch.where(torch.isnan(h.reshape(-1)), torch.full_like(v, 0x7FC00000), v)
    v = v ^ (v >> 16)
    v = (v * 0x7FEB352D) & M32
    v = v ^ (v >> 15)
    s1 = int(((v * w) & M32).sum().item()) & M32
    s2 = int(v.sum().item()) & M32
    return [s1, s2]


def test_silu_bits_equal_v8_on_every_input(ops):
    with open(GOLDEN) as f:
        golden = json.load(f)["hashes"]
    assert len(golden) == 256
    n = 1 << 24
    w = 2 * torch.arange(n, dtype=torch.int64, device=DEV) + 1
    u = torch.ones((4096, 4096), dtype=torch.float32, device=DEV)
    h = torch.empty((4096, 4096), dtype=torch.float32, device=DEV)
    bits = torch.arange(n, dtype=torch.int64, device=DEV)
    bad = []
    for c in range(256):
        g = ((bits + c * n) & M32).to(torch.int64)
        g = torch.where(g >= 1 << 31, g - (1 << 32), g).to(torch.int32).view(torch.float32).reshape(4096, 4096)
        ops.silu_mul_quantize(g, u, h)
        if chunk_hash(h, w) != golden[c]:
            bad.append(c)
        if c % 64 == 63:
            print(f"silu exhaustive: chunks 0..{c} done, {len(bad)} differ", flush=True)
    assert not bad, f"{len(bad)} of 256 chunks differ from V8: {bad[:16]}"
