"""Golden vectors (tests/golden/golden.npz, written by golden_cases.js under a
JavaScript engine with the reference's arithmetic; regenerate with
tests/golden/make_golden.py).

CPU: the oracle must reproduce every vector.  GPU: the HIP path, through the
C ABI, must reproduce the compiled-op vectors and config C1 bit for bit.
"""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


@pytest.fixture(scope="module")
def g():
    z = np.load(GOLDEN, allow_pickle=False)
    d = {k: z[k] for k in z.files}
    d["meta"] = json.loads(bytes(d.pop("meta_json")).decode())
    return d


def same_bits(a, b, what=""):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype, (what, a.shape, b.shape, a.dtype, b.dtype)
    bad = np.nonzero(np.any(a.view(np.uint8).reshape(-1, a.itemsize) != b.view(np.uint8).reshape(-1, b.itemsize), axis=1))[0]
    assert bad.size == 0, f"{what}: {bad.size} of {a.size} differ; first at {bad[0]}"


# ---------------------------------------------------------------- CPU: oracle
def test_params_vectors(g, oracle):
    p = g["meta"]["params"]
    assert [oracle.scale_sym_from_range(a, b) for a, b in
            [(-3, 3), (-1, 5), (-6, 6), (-1, 1), (-10, 10), (-5, 5)]] == p["sym"]
    s, z = oracle.params_asym_from_range(0, 6)
    assert (s, z) == (p["asym_i8_0_6"]["scale"], p["asym_i8_0_6"]["zeroPoint"])
    s, z = oracle.params_asym_from_range(0, 1, unsigned=True)
    assert (s, z) == (p["asym_u8_0_1"]["scale"], p["asym_u8_0_1"]["zeroPoint"])
    assert oracle.scale_const_array(np.array([1, -2, 3, -0.5], np.float32)) == p["const_1m2_3"]
    assert oracle.scale_const_array(np.array([5, 5, 5], np.float32)) == p["const_555"]
    s66 = oracle.scale_sym_from_range(-6, 6)
    assert int(oracle.weight_quantize_per_tensor(np.array([3.5], np.float32), s66)[0]) == p["q_3p5"]
    s11 = oracle.scale_sym_from_range(-1, 1)
    assert oracle.weight_quantize_per_tensor(np.array([1000, -1000], np.float32), s11).tolist() == p["q_pm1000"]
    s1010 = oracle.scale_sym_from_range(-10, 10)
    assert oracle.weight_quantize_per_tensor(np.array([1.5, -3.2, 0.0, 7.8], np.float32),
                                             s1010).tolist() == p["q_array"]
    W = g["params_skewed_W"].reshape(4, 3)
    assert oracle.scales_per_channel(W, 1).tolist() == p["pc_axis1"]
    assert oracle.scales_per_channel(W, 0).tolist() == p["pc_axis0"]
    sc1 = oracle.scales_per_channel(W, 1)
    assert oracle.weight_quantize_per_channel(W, 1, sc1).reshape(-1).tolist() == p["pc_axis1_q"]
    data = g["params_group_data"]
    gs = oracle.scales_per_group(data, 16, num_bits=4)
    assert gs.tolist() == p["group_scales"]
    assert oracle.weight_quantize_per_group(data, 16, gs, -7, 7).tolist() == p["group_q"]


def test_fakequant_vectors(g, oracle):
    s = g["meta"]["fakequant"]["scale"]
    q = oracle.quantize(g["fakequant_x"], s)
    same_bits(q, g["fakequant_q"], "R1")
    same_bits(oracle.dequantize(q, s), g["fakequant_y"], "D1")


def test_pcmatmul_vectors(g, oracle):
    meta = g["meta"]["pcmatmul"]
    A = g["pcmatmul_A"].reshape(4, 8)
    aq = oracle.quantize(A, meta["aScale"])
    same_bits(aq.reshape(-1), g["pcmatmul_aq"], "activation codes")
    W = g["pcmatmul_W"].reshape(8, 6)
    sc = oracle.scales_per_channel(W, 1)
    same_bits(oracle.weight_quantize_per_channel(W, 1, sc).reshape(-1), g["pcmatmul_pc_wq"], "pc weight")
    for mode in ("pc", "pt"):
        wq = g[f"pcmatmul_{mode}_wq"].reshape(8, 6)
        acc = oracle.quantized_dot(aq, wq, b_layout=0)
        same_bits(acc.reshape(-1), g[f"pcmatmul_{mode}_acc"], f"{mode} acc")
        sv = np.array(meta[mode]["sv"], np.float64).astype(np.float32)
        # E-pc with the F32 scale vector already rounded: fround(acc * sv[n])
        y = (acc.astype(np.float64) * sv.astype(np.float64)[None, :]).astype(np.float32)
        same_bits(y.reshape(-1), g[f"pcmatmul_{mode}_y"], f"{mode} y")
        # and through the oracle epilogue (sA * sW rounded to f32 inside)
        sw = sc if mode == "pc" else np.full(6, oracle.scale_const_array(W))
        same_bits(oracle.epilogue(acc, "rowcol", meta["aScale"], sw).reshape(-1),
                  g[f"pcmatmul_{mode}_y"], f"{mode} oracle epilogue")


def test_edge_vectors(g, oracle):
    x = g["edges_x"]
    for j, s in enumerate(g["meta"]["edges"]["scales"]):
        same_bits(oracle.quantize(x, s), g[f"edges_q_{j}"], f"i8 scale {s}")
        same_bits(oracle.quantize(x, s, unsigned=True), g[f"edges_u_{j}"], f"u8 scale {s}")


def test_c1_vectors(g, oracle):
    X = g["c1_X"].reshape(32, 128)
    W = g["c1_W"].reshape(64, 128)
    sX = oracle.scale_per_tensor(X)
    assert sX == g["meta"]["c1"]["sX"]
    same_bits(oracle.quantize(X, sX).reshape(-1), g["c1_Xq"], "C1 activation codes")
    sW = oracle.scales_per_channel(W, 0)
    same_bits(sW, g["c1_sW"], "C1 weight scales")
    Wq = oracle.weight_quantize_per_channel(W, 0, sW)
    same_bits(Wq.reshape(-1), g["c1_Wq"], "C1 weight codes")
    acc = oracle.quantized_dot(g["c1_Xq"].reshape(32, 128), Wq, b_layout=1)
    same_bits(acc.reshape(-1), g["c1_acc"], "C1 acc")
    y = oracle.epilogue(acc, "rowcol", sX, sW, bias=g["c1_bias"])
    same_bits(y.reshape(-1), g["c1_y"], "C1 y")


# ---------------------------------------------------------------- GPU: HIP path
@pytest.fixture(scope="module")
def dev_ops():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from mlfw_amd import _lib, ops
    _lib.call("q8_init", 0)
    return torch, ops


@pytest.mark.gpu
def test_gpu_golden_compiled_ops(g, dev_ops):
    torch, O = dev_ops
    up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")  # noqa: E731
    down = lambda t: (torch.cuda.synchronize(), t.cpu().numpy())[1]      # noqa: E731
    x = up(g["edges_x"])
    for j, s in enumerate(g["meta"]["edges"]["scales"]):
        same_bits(down(O.quantize(x, s)), g[f"edges_q_{j}"], f"i8 scale {s}")
        same_bits(down(O.quantize(x, s, target_dtype="ui8")), g[f"edges_u_{j}"], f"u8 scale {s}")
    s = g["meta"]["fakequant"]["scale"]
    q = O.quantize(up(g["fakequant_x"]), s)
    same_bits(down(q), g["fakequant_q"], "R1")
    same_bits(down(O.dequantize(q, s)), g["fakequant_y"], "D1")
    for mode in ("pc", "pt"):
        wq_nk = np.ascontiguousarray(g[f"pcmatmul_{mode}_wq"].reshape(8, 6).T)
        acc = O.quantized_dot(up(g["pcmatmul_aq"].reshape(4, 8)), up(wq_nk))
        same_bits(down(acc).reshape(-1), g[f"pcmatmul_{mode}_acc"], f"{mode} acc")


@pytest.mark.gpu
def test_gpu_golden_c1(g, dev_ops):
    torch, O = dev_ops
    from mlfw_amd import configs as C
    up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")  # noqa: E731
    y = C.c1_run(up(g["c1_X"].reshape(32, 128)), up(g["c1_W"].reshape(64, 128)), up(g["c1_bias"]))
    torch.cuda.synchronize()
    same_bits(y.cpu().numpy().reshape(-1), g["c1_y"], "C1 y on the GPU")
