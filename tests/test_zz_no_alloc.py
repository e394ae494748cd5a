"""q8_qlinear_dynamic_noalloc against q8_qlinear_dynamic, through the C ABI.

The allocation-free entry point stages the codes and scales of x in the
library's per-device scratch array instead of caller buffers.  Its output
must equal q8_qlinear_dynamic's bit for bit; two calls in a row, the second
on a smaller input, check that the staging left by the first call does not
leak into the second.  Runs alone in a fresh process or after the other
tests.
"""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from mlfw_amd import _lib
    _lib.call("q8_init", 0)
    return _lib


def vp(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def stream():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def rng_normal(seed, shape, std=1.0):
    g = np.random.default_rng(seed)
    return (g.standard_normal(shape) * std).astype(np.float32)


def packed_weight(lib, N, K, seed):
    W = torch.from_numpy(rng_normal(seed, (N, K), 0.02)).to(DEV)
    Wq = torch.empty((N, K), dtype=torch.int8, device=DEV)
    sW = torch.empty(N, dtype=torch.float64, device=DEV)
    lib.call("q8_pack_weight", vp(W), N, K, 0, lib.Q8_PER_CHANNEL, vp(Wq), vp(sW), stream())
    return Wq, sW


def run_both(lib, x, Wq, sW, mode, bias, act):
    M, K = x.shape
    N = Wq.shape[0]
    ref = torch.empty((M, N), dtype=torch.float32, device=DEV)
    got = torch.full((M, N), float("nan"), dtype=torch.float32, device=DEV)
    xq = torch.empty((M, K), dtype=torch.int8, device=DEV)
    sx = torch.empty(M if mode == lib.Q8_PER_TOKEN else 1, dtype=torch.float64, device=DEV)
    lib.call("q8_qlinear_dynamic", vp(x), M, K, mode, vp(Wq), vp(sW), lib.Q8_PER_CHANNEL, N,
             vp(bias), act, vp(ref), vp(xq), vp(sx), stream())
    lib.call("q8_qlinear_dynamic_noalloc", vp(x), M, K, mode, vp(Wq), vp(sW),
             lib.Q8_PER_CHANNEL, N, vp(bias), act, vp(got), stream())
    torch.cuda.synchronize()
    return ref.cpu().numpy(), got.cpu().numpy()


def same_bits(a, b):
    bad = np.count_nonzero(a.view(np.uint32) != b.view(np.uint32))
    assert bad == 0, f"{bad} of {a.size} outputs differ"


# (first shape, second shape): the second call is smaller than the first
CASES = [
    ((1, 4096), (1, 1024)),        # one token: the fused quantize + GEMV kernel
    ((16, 4096), (5, 4096)),       # GEMV kernels
    ((300, 2048), (40, 2048)),     # MFMA GEMM
    ((1000, 4096), (17, 4096)),    # staging near the 4 MiB limit, then a small one
]


@pytest.mark.parametrize("mode_name", ["per_token", "per_tensor"])
@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_matches_dynamic_twice(lib, mode_name, first, second):
    mode = lib.Q8_PER_TOKEN if mode_name == "per_token" else lib.Q8_PER_TENSOR
    for call, (M, K) in enumerate((first, second)):
        N = 96 if M > 16 else 4096
        Wq, sW = packed_weight(lib, N, K, seed=10 + call)
        xh = rng_normal(20 + call, (M, K))
        xh[0, 3] = 25.0 * (call + 1)               # a row (and tensor) absmax that changes
        x = torch.from_numpy(xh).to(DEV)
        bias = torch.from_numpy(rng_normal(30 + call, (N,), 0.05)).to(DEV)
        act = lib.Q8_ACT_RELU if call else lib.Q8_ACT_SILU
        ref, got = run_both(lib, x, Wq, sW, mode, bias, act)
        same_bits(ref, got)


def test_noalloc_rejects_inputs_beyond_the_scratch(lib):
    K = 4096
    M = lib.Q8_NOALLOC_SCRATCH_BYTES // K       # codes fill the scratch: no room for scales
    Wq, sW = packed_weight(lib, 64, K, seed=3)
    x = torch.zeros((M, K), dtype=torch.float32, device=DEV)
    out = torch.empty((M, 64), dtype=torch.float32, device=DEV)
    rc = lib.load().q8_qlinear_dynamic_noalloc(vp(x), M, K, lib.Q8_PER_TOKEN, vp(Wq), vp(sW),
                                                lib.Q8_PER_CHANNEL, 64, None, 0, vp(out), stream())
    assert rc == lib.Q8_ERR_INVALID
    assert "scratch" in lib.load().q8_last_error().decode()
    # the largest accepted per-token input still runs and matches
    M = (lib.Q8_NOALLOC_SCRATCH_BYTES - 8 * 900) // K
    x = torch.from_numpy(rng_normal(5, (M, K))).to(DEV)
    ref, got = run_both(lib, x, Wq, sW, lib.Q8_PER_TOKEN, None, 0)
    same_bits(ref, got)
