"""Seeded geometry fuzz of quantized_conv against the oracle
(ops/quantization.ts:156-190, the conv loop nest of
lowering_registry.ts:335-449).

Random 1-D to 3-D geometries: batch, channels per group (3: the direct
kernel; 16 and 48: the channel-last frame with an im2col matrix; 64 and
128: the implicit GEMM, split over K when the contraction is long and the
tiles few), groups, output channels per group (the GEMV below 17, the GEMM
above), kernel sizes, strides, dilations and asymmetric padding (padding
larger than the kernel reach included), int32 out or the fused dequant
fround(acc * s_out), and the prepacked tap-major weight on the routes that
take it.  Bit for bit; each case prints its seed and geometry first."""
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


def geometry(seed):
    rng = np.random.default_rng(500 + seed)
    nd = int(rng.integers(1, 4))
    groups = int(rng.choice([1, 1, 2, 3]))
    cg = int(rng.choice([3, 16, 48, 64, 128]))
    og = int(rng.choice([4, 12, 20, 48, 96]))
    n = int(rng.integers(1, 4))
    sizes = {1: (5, 40), 2: (3, 14), 3: (2, 7)}[nd]
    ks, st, dl, pd, sp = [], [], [], [], []
    for _ in range(nd):
        k = int(rng.integers(1, 4 if nd == 3 else 6))
        s = int(rng.integers(1, 3))
        d = int(rng.integers(1, 3))
        lo, hi = int(rng.integers(0, 3)), int(rng.integers(0, 3))
        reach = d * (k - 1) + 1
        size = max(int(rng.integers(*sizes)), reach - lo - hi)     # at least one output position
        ks.append(k); st.append(s); dl.append(d); pd.append([lo, hi]); sp.append(size)
    xs = (n, groups * cg, *sp)
    ws = (groups * og, cg, *ks)
    return rng, xs, ws, st, pd, dl, groups


@pytest.mark.parametrize("seed", range(32))
def test_conv_fuzz(ops, oracle, seed):
    rng, xs, ws, st, pd, dl, g = geometry(seed)
    out_f32 = seed % 2 == 1
    print(f"conv fuzz seed={seed} x{xs} w{ws} s{st} p{pd} d{dl} g{g} f32={out_f32}", flush=True)
    x = rng.integers(-128, 128, xs).astype(np.int8)
    w = rng.integers(-128, 128, ws).astype(np.int8)
    want = oracle.quantized_conv(x, w, st, pd, dl, g)
    s_out = 1.7e-4 if out_f32 else None
    if out_f32:
        want = (want.astype(np.float64) * s_out).astype(np.float32)
    got = ops.quantized_conv(dev(x), dev(w), st, pd, dl, g, s_out=s_out)
    gb = host(got)
    assert gb.shape == want.shape, (gb.shape, want.shape)
    assert gb.tobytes() == want.tobytes(), f"seed {seed}: {np.count_nonzero(gb != want)} of {want.size} differ"
    if g == 1 and ws[1] % 16 == 0 and np.prod(ws[2:]) > 1:
        wt = ops.conv_weight_taps(dev(w))
        got2 = ops.quantized_conv(dev(x), dev(w), st, pd, dl, g, s_out=s_out, w_taps=wt)
        assert host(got2).tobytes() == want.tobytes(), f"seed {seed}: prepacked weight"
