"""The device's compiled quantize R1 (q8_quantize_static: the f32 fast path
with the exact f64 fallback near ties, the same functions the per-token
quantize, the SiLU-up requant and the requant epilogues use) against V8's
evaluation of the reference's expression
    (Math.min(Math.max(Math.round(Math.fround(x / S)), -128), 127) | 0)
on every one of the 2^32 binary32 inputs, for each scale of
tests/golden/quant_v8_hashes.json (typical absmax / 127 scales, an inexact
decimal, a power of two with exact ties, small scales, and two outside the
fast path's range, which take the exact path).  Per chunk of 2^24 inputs
the device output's hashes must equal V8's (quant_v8_hashes.js)."""
import json
import os

import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
M32 = 0xFFFFFFFF
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_v8_hashes.json")

with open(GOLDEN) as _f:
    _DOC = json.load(_f)


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from mlfw_amd import ops as O
    from mlfw_amd import _lib
    _lib.call("q8_init", 0)
    return O


@pytest.mark.parametrize("scale", _DOC["scales"])
def test_quantize_bits_equal_v8_on_every_input(ops, scale):
    golden = _DOC["hashes"][scale]
    s = float(scale)
    n = 1 << 24
    w = 2 * torch.arange(n, dtype=torch.int64, device=DEV) + 1
    bits = torch.arange(n, dtype=torch.int64, device=DEV)
    mix = torch.arange(256, dtype=torch.int64, device=DEV)
    mix = mix ^ (mix >> 16)
    mix = (mix * 0x7FEB352D) & M32
    mix = mix ^ (mix >> 15)
    bad = []
    for c in range(256):
        g = (bits + c * n) & M32
        x = torch.where(g >= 1 << 31, g - (1 << 32), g).to(torch.int32).view(torch.float32)
        q = ops.quantize(x, s)
        m = mix[q.view(torch.uint8).to(torch.int64)]
        h = [int(((m * w) & M32).sum().item()) & M32, int(m.sum().item()) & M32]
        if h != golden[c]:
            bad.append(c)
    print(f"quantize exhaustive S={scale}: {len(bad)} of 256 chunks differ", flush=True)
    assert not bad, f"S={scale}: {len(bad)} chunks differ from V8: {bad[:16]}"
