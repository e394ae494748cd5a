"""Packed-weight checkpoint records (mlfw_amd/checkpoint.py) feeding the GPU
path: int8 per-channel, int8 per-tensor and 4-bit per-group records are
written to a checkpoint file, read back, and the weights and scales taken
from the records drive q8_gemm / q8_gemv_w4 bit for bit like the oracle on
the same inputs.  The device packers are checked against the records too,
so a checkpoint written from either side loads into the other."""
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
    bad = np.nonzero(np.any(a.view(np.uint8).reshape(-1, a.itemsize) != b.view(np.uint8).reshape(-1, b.itemsize),
                            axis=1))[0]
    assert bad.size == 0, f"{bad.size} of {a.size} differ, first at {bad[:5]}"


@pytest.mark.parametrize("M,N,K,g", [(64, 256, 512, 64), (3, 300, 1024, 128), (16, 96, 4096, 2048)])
def test_packed_records_drive_the_gpu_linear(ops, oracle, tmp_path, M, N, K, g):
    from mlfw_amd import checkpoint as ck
    r = oracle.Rng(M + 7 * N + K)
    W = r.normal((N, K), 0.0, 0.02)
    x = r.normal((M, K))
    bias = r.uniform((N,), -0.1, 0.1)
    # the records, written from the oracle's quantization
    s_pc = oracle.scales_per_channel(W, 0)
    q_pc = oracle.weight_quantize_per_channel(W, 0, s_pc)
    s_pg = oracle.scales_per_group(W.reshape(-1), g, num_bits=4)
    q_pg = oracle.weight_quantize_per_group(W.reshape(-1), g, s_pg, lo=-8, hi=7).reshape(W.shape)
    recs = {"fc.weight": ck.packed_linear_record(q_pc, s_pc, "per_channel"),
            "fc4.weight": ck.packed_linear_record(q_pg, s_pg, "per_group", num_bits=4, group_size=g),
            "pt.weight": ck.packed_linear_record(q_pc, [s_pc[0]], "per_tensor_symmetric")}
    path = tmp_path / "packed.ckpt"
    ck.save_packed(str(path), recs)
    back = ck.load_packed(str(path))
    assert list(back) == list(recs)

    # the device packers write what the records hold
    Wd = dev(W)
    Wq, sW = ops.pack_weight(Wd, axis=0)
    same_bits(host(Wq), ck.record_codes(back["fc.weight"]))
    same_bits(host(sW), back["fc.weight"]["params"]["scale"])
    wq4, sw4 = ops.pack_weight_int4(Wd, g)
    same_bits(host(wq4), back["fc4.weight"]["weight"].numpy())
    same_bits(host(sw4), back["fc4.weight"]["params"]["scale"])

    sx = oracle.scales_per_token(x)
    xq = oracle.quantize_rows(x, sx)
    print(f"records M={M} N={N} K={K} g={g}", flush=True)
    # int8 per-channel record -> q8_gemm (MFMA or GEMV route by M)
    rec = back["fc.weight"]
    codes, scale = ck.record_codes(rec), rec["params"]["scale"]
    acc = oracle.quantized_dot(xq, codes, b_layout=1)
    want = oracle.epilogue(acc, "rowcol", sx, scale, bias=bias, act="relu")
    got = ops.qlinear(dev(xq), dev(sx), dev(codes), dev(scale), bias=dev(bias), act="relu")
    same_bits(host(got), want)
    # int8 per-tensor record: its scale is a plain number
    rec = back["pt.weight"]
    s_pt = np.array([rec["params"]["scale"]], np.float64)
    want = oracle.epilogue(acc, "rowcol", sx, s_pt)
    got = ops.qlinear(dev(xq), dev(sx), dev(ck.record_codes(rec)), dev(s_pt))
    same_bits(host(got), want)
    # 4-bit per-group record: the packed nibbles go to q8_gemv_w4 as stored
    rec = back["fc4.weight"]
    packed, s4 = rec["weight"].numpy(), rec["params"]["scale"]
    want = oracle.gemv_w4(xq, sx, packed, s4, K, g, bias=bias, act="silu")
    got = ops.qlinear_w4(dev(xq), dev(sx), dev(packed), dev(s4), K, g, bias=dev(bias), act="silu")
    same_bits(host(got), want)
