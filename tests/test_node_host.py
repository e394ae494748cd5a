"""The Node host side (mlfw_amd/node: N-API addon + hip_backend.js).

CPU: registration into mock registries shaped like the reference's, TIR
matching of QuantizationPass's lowered ops, argument errors (no device).
GPU: C1, an int8 linear with the fused static requant, a W4A8 decode
linear and a grouped, strided, dilated, padded quantized_conv through the
'hip' runtime backend and the eager library, every output compared bit for
bit with the oracle.
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCRIPT = os.path.join(ROOT, "tests", "node", "hip_backend_test.js")
ADDON = os.path.join(ROOT, "mlfw_amd", "node", "q8hip.node")
NODE = shutil.which("node")

needs_node = pytest.mark.skipif(NODE is None, reason="node is not installed")


def run_node(*args, timeout=120):
    r = subprocess.run([NODE, SCRIPT, *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    print(r.stderr)
    return r


@needs_node
def test_node_host_cpu():
    if not os.path.exists(ADDON):
        pytest.fail("q8hip.node is not built: run `python -m mlfw_amd.build`")
    r = run_node("cpu")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all passed" in r.stdout


def same_bits(a, b, what):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype, (what, a.shape, b.shape, a.dtype, b.dtype)
    bad = np.nonzero(a.view(np.uint8).reshape(-1, a.itemsize) != b.view(np.uint8).reshape(-1, b.itemsize))[0]
    assert bad.size == 0, f"{what}: {np.unique(bad).size} elements differ"


@needs_node
@pytest.mark.gpu
def test_node_host_gpu_c1(tmp_path, oracle):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from oracle import configs as OC
    inp, y_ref = OC.c1()
    X, W, bias = inp["X"], inp["W"], inp["bias"]
    M, K = X.shape
    N = W.shape[0]
    Wq, sW = OC.pack_pc(W, 0)
    sX = oracle.scale_per_tensor(X)
    Xq = oracle.quantize(X, sX)
    s_out = sX * float(sW[0])
    for name, arr in (("X", X), ("Xq", Xq), ("Wq", Wq), ("sW", sW), ("bias", bias)):
        np.ascontiguousarray(arr).tofile(tmp_path / f"{name}.bin")
    # per-token codes for the requant leg, 4-bit per-group weights for the W4 leg
    s_tok = oracle.scales_per_token(X)
    q_tok = oracle.quantize_rows(X, s_tok)
    y_rq = oracle.epilogue(oracle.quantized_dot(q_tok, Wq, b_layout=1), "rowcol", s_tok, sW, bias=bias,
                           act="relu")
    s_next = float(np.max(np.abs(y_rq))) / 127
    w4_group, w4_m = 32, 3
    from mlfw_amd.checkpoint import pack_int4
    sw4 = oracle.scales_per_group(W.reshape(-1), w4_group, num_bits=4)
    wq4 = pack_int4(oracle.weight_quantize_per_group(W.reshape(-1), w4_group, sw4, lo=-8, hi=7).reshape(W.shape))
    qdot_u8_a = np.random.default_rng(12).integers(0, 256, (M, K)).astype(np.uint8)
    for name, arr in (("sx_tok", s_tok), ("xq_tok", q_tok), ("w4_q", wq4), ("w4_s", sw4),
                      ("qdot_u8_a", qdot_u8_a)):
        np.ascontiguousarray(arr).tofile(tmp_path / f"{name}.bin")
    (tmp_path / "meta.json").write_text(json.dumps({"M": M, "N": N, "K": K, "sX": sX, "sOut": s_out,
                                                    "sNext": s_next, "w4Group": w4_group, "w4M": w4_m}))
    # CONV_CASE of hip_backend_test.js
    crng = np.random.default_rng(11)
    xc = crng.integers(-128, 128, (2, 4, 9, 7)).astype(np.int8)
    wc = crng.integers(-128, 128, (6, 2, 3, 2)).astype(np.int8)
    xc.tofile(tmp_path / "conv_x.bin")
    wc.tofile(tmp_path / "conv_w.bin")
    r = run_node("gpu", str(tmp_path))
    assert r.returncode == 0, r.stdout + r.stderr

    def out(name, dt, shape):
        return np.fromfile(tmp_path / f"{name}.bin", dtype=dt).reshape(shape)

    same_bits(out("out_quantize", np.int8, (M, K)), Xq, "compiled quantize")
    acc = oracle.quantized_dot(Xq, Wq, b_layout=1)
    same_bits(out("out_qdot_NK", np.int32, (M, N)), acc, "quantized_dot [N,K]")
    same_bits(out("out_qdot_KN", np.int32, (M, N)), acc, "quantized_dot [K,N]")
    same_bits(out("out_qdot_u8", np.int32, (M, N)), oracle.quantized_dot(qdot_u8_a, Wq, 1, 128, 3),
              "quantized_dot ui8 x i8 with zero points")
    same_bits(out("out_dequant_i32", np.float32, (M, N)), oracle.dequantize(acc, s_out), "E-pt")
    same_bits(out("out_c1", np.float32, (M, N)), y_ref, "C1 fused qlinear")
    same_bits(out("out_qpt_q", np.int8, (M, K)), q_tok, "eager quantize_per_token codes")
    same_bits(out("out_qpt_s", np.float64, (M,)), s_tok, "eager quantize_per_token scales")
    same_bits(out("out_dpt", np.float32, (M, K)), oracle.dequantize_rows(q_tok, s_tok),
              "eager dequantize_per_token")
    conv_ref = oracle.quantized_conv(xc, wc, [2, 1], [[1, 2], [0, 1]], [2, 1], 2)
    same_bits(out("out_conv", np.int32, conv_ref.shape), conv_ref, "quantized_conv PrimFunc")
    same_bits(out("out_requant", np.int8, (M, N)), oracle.quantize(y_rq.reshape(-1), s_next).reshape(M, N),
              "qlinear with fused static requant")
    same_bits(out("out_qlinear1", np.float32, (1, N)),
              OC.qlinear_rows(X[:1], Wq, sW, bias=bias, act="silu"), "one-token dynamic qlinear")
    xs = X[:w4_m]
    sxs = oracle.scales_per_token(xs)
    want_w4 = oracle.gemv_w4(oracle.quantize_rows(xs, sxs), sxs, wq4, sw4, K, w4_group, bias=bias, act="silu")
    same_bits(out("out_w4", np.float32, (w4_m, N)), want_w4, "W4A8 decode linear")
