"""q8_gemm_glu: gate and up linears with SiLU(gate) * up fused into one GEMM.

The reference runs the two per-channel linears (quantization_pass.ts:390-459),
the SiLU decomposition (decomposition_pass.ts:197-230) and the product as
separate ops.  Every h here is compared bit for bit with the oracle's
epilogue of each half's exact int32 accumulators followed by the oracle's
silu_mul, on the MFMA route (both tile shapes, partial tiles in M and in F,
the f64 path for |acc| > 2^24, biases), the decode route (M <= 16: GEMV into
the workspace, then the pairing kernel) and the generic route (K % 16 != 0).
The interleaved weight is compared with a numpy interleave of the two packs.
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
    av = a.view(np.uint8).reshape(-1, a.itemsize)
    bv = b.view(np.uint8).reshape(-1, b.itemsize)
    bad = np.nonzero(np.any(av != bv, axis=1))[0]
    assert bad.size == 0, (f"{what}: {bad.size} of {a.size} differ; first at {bad[0]}: "
                           f"{a.reshape(-1)[bad[0]]!r} vs {b.reshape(-1)[bad[0]]!r}")


def interleave_rows(g, u):
    """numpy form of the GLU weight layout: groups of 32 gate rows, then the
    same 32 up rows."""
    F = g.shape[0]
    out = np.empty((2 * F,) + g.shape[1:], g.dtype)
    for j in range(F // 32):
        out[64 * j:64 * j + 32] = g[32 * j:32 * j + 32]
        out[64 * j + 32:64 * j + 64] = u[32 * j:32 * j + 32]
    return out


def exact_acc(Aq, Bq):
    return (Aq.astype(np.float64) @ Bq.astype(np.float64).T).astype(np.int32)


def glu_ref(oracle, Aq, sA, Wg, sg, Wu, su, bg=None, bu=None):
    g = oracle.epilogue(exact_acc(Aq, Wg), "rowcol", sA, sg, bias=bg)
    u = oracle.epilogue(exact_acc(Aq, Wu), "rowcol", sA, su, bias=bu)
    return oracle.silu_mul(g, u)


# (M, F, K): 256 x 256 tiles with partial tiles in M and F; 128 x 128 tiles
# (partial); one full 256-row block; decode sizes; K not a multiple of 16
SHAPES = [(4000, 2016, 256), (300, 1056, 512), (4096, 2048, 128), (16, 1024, 4096), (5, 96, 4096),
          (1, 32, 64), (64, 64, 40), (33, 160, 16)]


@pytest.mark.parametrize("M,F,K", SHAPES)
@pytest.mark.parametrize("per_token,with_bias", [(True, False), (False, True)])
def test_glu_matches_two_linears_and_silu_mul(ops, oracle, M, F, K, per_token, with_bias):
    rng = np.random.default_rng(M * 131 + F * 7 + K + 2 * per_token + with_bias)
    Aq = rng.integers(-128, 128, (M, K)).astype(np.int8)
    Wg = rng.integers(-127, 128, (F, K)).astype(np.int8)
    Wu = rng.integers(-127, 128, (F, K)).astype(np.int8)
    # scales that put g around the SiLU's curved region
    sA = rng.uniform(0.5, 2.0, M if per_token else 1) * (4.0 / (128.0 * np.sqrt(K) * 100))
    sg = rng.uniform(0.5, 2.0, F) * 0.9
    su = rng.uniform(0.5, 2.0, F) * 1.1
    bg = rng.uniform(-0.5, 0.5, F).astype(np.float32) if with_bias else None
    bu = rng.uniform(-0.5, 0.5, F).astype(np.float32) if with_bias else None
    packed = ops.glu_interleave((dev(Wg), dev(sg)), (dev(Wu), dev(su)),
                                *((dev(bg), dev(bu)) if with_bias else ()))
    same_bits(host(packed[0]), interleave_rows(Wg, Wu), "interleaved codes")
    same_bits(host(packed[1]), interleave_rows(sg, su), "interleaved scales")
    if with_bias:
        same_bits(host(packed[2]), interleave_rows(bg, bu), "interleaved biases")
    W, s = packed[0], packed[1]
    b = packed[2] if with_bias else None
    h = ops.qlinear_glu(dev(Aq), dev(sA), W, s, bias=b)
    ref = glu_ref(oracle, Aq, sA if per_token else sA[0], Wg, sg, Wu, su, bg, bu)
    same_bits(host(h), ref, f"h M={M} F={F} K={K}")


def test_glu_exact_path_for_large_accumulators(ops, oracle):
    """|acc| > 2^24 (K = 4096 of saturated codes) takes the f64 product of
    the epilogue; mixed with ordinary rows in the same strips."""
    M, F, K = 512, 256, 4096
    rng = np.random.default_rng(5)
    Aq = rng.integers(-128, 128, (M, K)).astype(np.int8)
    Aq[::7] = 127
    Wg = rng.integers(-127, 128, (F, K)).astype(np.int8)
    Wu = rng.integers(-127, 128, (F, K)).astype(np.int8)
    Wg[::5] = 127
    Wu[::3] = -127
    sA = rng.uniform(1e-9, 4e-9, M)
    sg, su = rng.uniform(0.5, 2.0, F), rng.uniform(0.5, 2.0, F)
    assert np.abs(exact_acc(Aq, Wg)).max() > 2 ** 24
    W, s = ops.glu_interleave((dev(Wg), dev(sg)), (dev(Wu), dev(su)))
    h = ops.qlinear_glu(dev(Aq), dev(sA), W, s)
    same_bits(host(h), glu_ref(oracle, Aq, sA, Wg, sg, Wu, su), "h with |acc| > 2^24")


def test_glu_rejects_bad_arguments(ops):
    W = torch.zeros((96, 64), dtype=torch.int8, device=DEV)      # 2F = 96: F = 48, not a multiple of 32
    s = torch.ones(96, dtype=torch.float64, device=DEV)
    A = torch.zeros((4, 64), dtype=torch.int8, device=DEV)
    with pytest.raises(ValueError):
        ops.qlinear_glu(A, torch.ones(1, dtype=torch.float64, device=DEV), W, s)
    Wg = torch.zeros((48, 64), dtype=torch.int8, device=DEV)
    sg = torch.ones(48, dtype=torch.float64, device=DEV)
    from mlfw_amd import _lib
    with pytest.raises(_lib.Q8Error, match="multiple of 32"):
        ops.glu_interleave((Wg, sg), (Wg, sg))
