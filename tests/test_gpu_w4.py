"""GPU parity of the 4-bit per-group path (q8_pack_weight_int4, q8_gemv_w4).

Packing is compared with the oracle's fromConstantArrayPerGroup /
quantizeArrayPerGroup restatement (codes and f64 scales bit for bit, NaN and
zero groups included); the W4A8 GEMV with the oracle's definition of it
(exact per-group sums, f64 sum over groups in order), bit for bit, on the
MFMA kernel (2 <= M <= 16, K <= 4096), the dot4 kernel (M <= 4,
power-of-two groups) and the generic one.
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
    assert bad.size == 0, f"{np.unique(bad).size} of {a.size} differ"


def ref_pack(oracle, W, g):
    from mlfw_amd.checkpoint import pack_int4
    s = oracle.scales_per_group(W.reshape(-1), g, num_bits=4)
    q = oracle.weight_quantize_per_group(W.reshape(-1), g, s, lo=-8, hi=7).reshape(W.shape)
    return pack_int4(q), s


# lane teams of 64 (g = 128, 2048), 16 (32), 8 (48), 2 (12) and 1 (2, 6)
@pytest.mark.parametrize("N,K,g", [(64, 4096, 128), (37, 1024, 32), (5, 96, 48), (300, 8192, 2048),
                                   (3, 12, 2), (7, 30, 6), (9, 36, 12)])
def test_pack_int4_matches_oracle(ops, oracle, N, K, g):
    r = oracle.Rng(N + K + g)
    W = r.normal((N, K), 0.0, 0.02)
    W[0, :g] = 0.0                      # all-zero group -> scale 1e-10
    W[1, 3] = np.nan                    # NaN: never the max, code 0
    W[2, 5] = 7.0                       # outlier
    wq, s = ops.pack_weight_int4(dev(W), g)
    want_q, want_s = ref_pack(oracle, W, g)
    same_bits(host(s), want_s)
    same_bits(host(wq), want_q)


def test_pack_int4_unaligned_source(ops, oracle):
    """A weight that starts 4 bytes into an allocation (4-byte aligned only)."""
    N, K, g = 33, 256, 64
    r = oracle.Rng(91)
    W = r.normal((N, K), 0.0, 0.02)
    buf = torch.empty(N * K + 1, dtype=torch.float32, device=DEV)
    Wd = buf[1:].view(N, K)
    Wd.copy_(torch.from_numpy(W))
    assert Wd.data_ptr() % 8 == 4
    wq, s = ops.pack_weight_int4(Wd, g)
    want_q, want_s = ref_pack(oracle, W, g)
    same_bits(host(s), want_s)
    same_bits(host(wq), want_q)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 6, 8, 16])
# (11008, 4096) and (5000, 8192) make every workgroup of the dot4 kernel walk
# two blocks of rows (prefetch path); (19, 96) has 256-row blocks; the MFMA
# kernel (M >= 3) sees spans of several groups (32, 64, 128), a group of 96
# (spans of 480 codes: a partial last step), groups of 1024 and 2048 (one
# span per group or half a group), K below one round (96, 128), many rounds
# (8192), N not a multiple of 16
@pytest.mark.parametrize("N,K,g", [(4096, 4096, 128), (1000, 4096, 32), (77, 2048, 2048), (33, 8192, 64),
                                   (19, 96, 32), (11, 160, 80), (11008, 4096, 128), (5000, 8192, 64),
                                   (77, 1536, 96), (11, 4096, 1024), (5, 128, 32), (300, 1024, 64)])
def test_gemv_w4_matches_oracle(ops, oracle, M, N, K, g):
    r = oracle.Rng(M * 1000 + N + g)
    x = r.normal((M, K))
    W = r.normal((N, K), 0.0, 0.02)
    sx = oracle.scales_per_token(x)
    xq = oracle.quantize_rows(x, sx)
    wq4, sw = ref_pack(oracle, W, g)
    bias = r.uniform((N,), -0.1, 0.1)
    print(f"gemv_w4 M={M} N={N} K={K} g={g}", flush=True)
    for b, act in ((None, "none"), (bias, "silu")):
        want = oracle.gemv_w4(xq, sx, wq4, sw, K, g, bias=b, act=act)
        got = ops.qlinear_w4(dev(xq), dev(sx), dev(wq4), dev(sw), K, g,
                             bias=None if b is None else dev(b), act=act)
        same_bits(host(got), want)


@pytest.mark.parametrize("M", [1, 3, 16, 20, 33])
# K above 8192 / non-power-of-two groups (no dot4 plan: the MFMA kernel for
# every M, also M = 1), groups split over spans (1536: 3 spans of 512, so a
# round of 2048 codes sees up to two group ends; 640: spans of 320), an odd
# round count, and token blocks (M = 20, 33: a partial block of 16)
# (3000, 11008) with M = 33: more blocks than two per CU over several rounds,
# the 4-wave shape; (11008, 4096) with M = 20, 33: more than three per CU in
# one round, the 4-wave one-round kernel
@pytest.mark.parametrize("N,K,g", [(300, 11008, 128), (70, 11008, 32), (40, 3072, 1536), (33, 1280, 640),
                                   (17, 12288, 64), (129, 4096, 4096), (3000, 11008, 128),
                                   (11008, 4096, 128)])
def test_gemv_w4_mfma_rounds(ops, oracle, M, N, K, g):
    r = oracle.Rng(M * 7 + N + K + g)
    x = r.normal((M, K))
    W = r.normal((N, K), 0.0, 0.02)
    W[1, :g] = 0.0                      # an all-zero group
    sx = oracle.scales_per_token(x)
    xq = oracle.quantize_rows(x, sx)
    wq4, sw = ref_pack(oracle, W, g)
    bias = r.uniform((N,), -0.1, 0.1)
    print(f"gemv_w4 rounds M={M} N={N} K={K} g={g}", flush=True)
    for b, act in ((None, "none"), (bias, "relu")):
        want = oracle.gemv_w4(xq, sx, wq4, sw, K, g, bias=b, act=act)
        got = ops.qlinear_w4(dev(xq), dev(sx), dev(wq4), dev(sw), K, g,
                             bias=None if b is None else dev(b), act=act)
        same_bits(host(got), want)


@pytest.mark.parametrize("M,N,K,g", [(6, 300, 4096, 128), (1, 70, 11008, 32), (20, 33, 1024, 64)])
def test_gemv_w4_per_tensor_scale(ops, oracle, M, N, K, g):
    """One activation scale for every token (sx [1], read with stride 0)."""
    r = oracle.Rng(M + N + K + g + 5)
    x = r.normal((M, K))
    W = r.normal((N, K), 0.0, 0.02)
    s = oracle.scale_per_tensor(x)
    xq = oracle.quantize(x.reshape(-1), s).reshape(M, K)
    wq4, sw = ref_pack(oracle, W, g)
    print(f"gemv_w4 per-tensor M={M} N={N} K={K} g={g}", flush=True)
    want = oracle.gemv_w4(xq, np.full(M, s), wq4, sw, K, g, act="silu")
    got = ops.qlinear_w4(dev(xq), dev(np.array([s])), dev(wq4), dev(sw), K, g, act="silu")
    same_bits(host(got), want)
