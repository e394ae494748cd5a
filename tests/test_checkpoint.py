"""The mlfw checkpoint container (mlfw_amd/checkpoint.py) and packed-weight records.

Pinned three ways:
  1. the reference's own known answers for the container
     (tests/lightning/callbacks/checkpoint.test.js:17-62), restated;
  2. byte equality with oracle/ckpt_ref.js, a JavaScript restatement of
     src/lightning/io/checkpoint_format.ts run under Node, so JSON number /
     string formatting and buffer order are a real engine's: both sides
     serialize the same tree, and each re-encodes what the other wrote;
  3. packed int8 / int4 records round-trip their codes and f64 scales
     exactly, and int4 packing agrees with the reference's per-group
     quantization (fromConstantArrayPerGroup + quantizeArrayPerGroup, which
     the oracle pins against params.test.js:204-233).
"""
import json
import os
import shutil
import subprocess

import numpy as np
import pytest

from mlfw_amd import checkpoint as ck

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "oracle", "ckpt_ref.js")
NODE = shutil.which("node")
needs_node = pytest.mark.skipif(NODE is None, reason="node is not installed")


def test_reference_known_answers():
    w = ck.Tensor("f32", [2, 2], np.array([1.5, -2.25, 3.125, np.pi], np.float32))
    ids = ck.Tensor("i32", [3], np.array([7, 8, 9], np.int32))
    r = ck.deserialize_checkpoint(ck.serialize_checkpoint(
        {"epoch": 3, "globalStep": 42, "modelState": ck.JSMap([("w", w), ("ids", ids)])}))
    assert r["epoch"] == 3 and r["globalStep"] == 42
    assert isinstance(r["modelState"], ck.JSMap)
    rw = r["modelState"].get("w")
    assert rw.shape == [2, 2] and rw.dtype == "f32"
    assert rw.data.tobytes() == w.data.tobytes()
    assert r["modelState"].get("ids").dtype == "i32"
    assert list(r["modelState"].get("ids").data) == [7, 8, 9]
    r = ck.deserialize_checkpoint(ck.serialize_checkpoint({"optimizerStates": [{
        "paramGroups": [{"lr": 0.05, "betas": [0.9, 0.999]}],
        "state": ck.JSMap([(0, {"step": 5, "exp_avg": np.array([0.1, 0.2, 0.3], np.float32)})])}]}))
    opt = r["optimizerStates"][0]
    assert opt["paramGroups"][0]["lr"] == 0.05
    assert opt["paramGroups"][0]["betas"] == [0.9, 0.999]
    s = opt["state"].get(0)
    assert s["step"] == 5
    assert s["exp_avg"].dtype == np.float32
    assert [float(v) for v in s["exp_avg"]] == [0.10000000149011612, 0.20000000298023224,
                                                0.30000001192092896]
    big = ck.Tensor("f32", [4096], np.arange(4096, dtype=np.float32) * 0.5)
    assert len(ck.serialize_checkpoint({"modelState": ck.JSMap([("w", big)])})) < 4096 * 4 * 1.4


@needs_node
def test_js_restatement_known_answers():
    r = subprocess.run([NODE, JS, "known"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "known answers ok" in r.stdout, r.stdout + r.stderr


def _rich_tree(tmp_path):
    """The same tree as Python values and as a spec for ckpt_ref.js."""
    rng = np.random.default_rng(0)
    arrays = {
        "w8": ("i8", [4, 6], rng.integers(-128, 128, 24).astype(np.int8)),
        "s64": ("f64", [4], rng.random(4) * 1e-3),
        "h": ("f32", [3, 5], rng.normal(size=15).astype(np.float32)),
        "u4": ("ui8", [4, 3], rng.integers(0, 256, 12).astype(np.uint8)),
    }
    files = {}
    for name, (dt, shape, data) in arrays.items():
        data.tofile(tmp_path / f"{name}.bin")
        files[name] = (dt, shape, data)
    f64 = np.array([6 / 127, 1e-10, 0.1 + 0.2, 5e-324, 1.7976931348623157e308], np.float64)
    i32 = np.array([0, -1, 2 ** 31 - 1], np.int32)
    f64.tofile(tmp_path / "f64.bin")
    i32.tofile(tmp_path / "i32.bin")
    nums = [0, -0.0, 1.5, 1e21, 1e-7, 123456.789, -3.25e-300, 2 ** 53, 6 / 127]
    py = {
        "epoch": 7, "note": "int8 é \"quoted\"\n", "flags": [True, False, None], "nums": nums,
        "modelState": ck.JSMap([(n, ck.Tensor(dt, shape, data)) for n, (dt, shape, data) in files.items()]),
        "params": {"scheme": "per_group", "scale": f64, "zeroPoint": i32, "axis": None,
                   "groupSize": 128, "dtype": "i8", "numBits": 4},
        "byIndex": ck.JSMap([(0, {"step": 1}), (1, {"step": 2})]),
        # integer-like keys: JS enumerates "0", "2", "10" first, ascending
        # (which also fixes the $buf order), then the others as inserted
        "layers": {"name": "mlp", "10": ck.Tensor("f32", [3, 5], files["h"][2]), "01": 1,
                   "2": ck.Tensor("i8", [4, 6], files["w8"][2]), "0": {"b": 2, "1": 3}},
    }
    spec = {
        "epoch": 7, "note": "int8 é \"quoted\"\n", "flags": [True, False, None], "nums": nums,
        "modelState": {"__map": [[n, {"__tensor": {"dtype": dt, "shape": shape, "file": f"{n}.bin"}}]
                                 for n, (dt, shape, _) in files.items()]},
        "params": {"scheme": "per_group", "scale": {"__array": {"type": "Float64Array", "file": "f64.bin"}},
                   "zeroPoint": {"__array": {"type": "Int32Array", "file": "i32.bin"}}, "axis": None,
                   "groupSize": 128, "dtype": "i8", "numBits": 4},
        "byIndex": {"__map": [[0, {"step": 1}], [1, {"step": 2}]]},
        "layers": {"name": "mlp", "10": {"__tensor": {"dtype": "f32", "shape": [3, 5], "file": "h.bin"}},
                   "01": 1, "2": {"__tensor": {"dtype": "i8", "shape": [4, 6], "file": "w8.bin"}},
                   "0": {"b": 2, "1": 3}},
    }
    return py, spec


@needs_node
def test_bytes_match_the_js_restatement(tmp_path):
    py, spec = _rich_tree(tmp_path)
    ours = ck.serialize_checkpoint(py)
    (tmp_path / "spec.json").write_text(json.dumps(spec))
    out = tmp_path / "js.bin"
    r = subprocess.run([NODE, JS, "roundtrip", str(tmp_path / "spec.json"), str(tmp_path), str(out)],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    theirs = out.read_bytes()
    assert ours == theirs
    # each side re-encodes what the other wrote, byte for byte
    (tmp_path / "py.bin").write_bytes(ours)
    r = subprocess.run([NODE, JS, "reencode", str(tmp_path / "py.bin"), str(tmp_path / "re.bin")],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    assert (tmp_path / "re.bin").read_bytes() == ours
    assert ck.serialize_checkpoint(ck.deserialize_checkpoint(theirs)) == theirs


def test_plain_object_keys_follow_js_enumeration_order():
    tree = {"z": 1, "10": 2, "2": 3, "01": 4, "4294967295": 5, "4294967294": 6, "-1": 7, "0": 8}
    header = ck.serialize_checkpoint(tree)[8:].decode("utf-8")
    order = json.loads(header, object_pairs_hook=lambda kv: [k for k, _ in kv] if "z" in dict(kv) else dict(kv))
    assert order["tree"] == ["0", "2", "10", "4294967294", "z", "01", "4294967295", "-1"]


def test_int4_packing_round_trip_and_layout():
    rng = np.random.default_rng(1)
    for N, K in [(3, 8), (5, 7), (1, 1)]:
        q = rng.integers(-8, 8, (N, K)).astype(np.int8)
        p = ck.pack_int4(q)
        assert p.shape == (N, (K + 1) // 2)
        np.testing.assert_array_equal(ck.unpack_int4(p, K), q)
    # element 2j in the low nibble, two's complement
    p = ck.pack_int4(np.array([[-1, 3, -8, 7]], np.int8))
    assert p.tolist() == [[0x3F, 0x78]]
    with pytest.raises(ValueError):
        ck.pack_int4(np.array([[9]], np.int8))


def test_packed_records_round_trip(tmp_path, oracle):
    r = oracle.Rng(77)
    W = r.normal((48, 256), 0.0, 0.02)
    s_pc = oracle.scales_per_channel(W, 0)
    q_pc = oracle.weight_quantize_per_channel(W, 0, s_pc)
    g = 64
    s_pg = oracle.scales_per_group(W.reshape(-1), g, num_bits=4)
    q_pg = oracle.weight_quantize_per_group(W.reshape(-1), g, s_pg, lo=-8, hi=7).reshape(W.shape)
    assert q_pg.min() >= -7 and q_pg.max() <= 7          # params.test.js:204-233
    recs = {"fc.weight": ck.packed_linear_record(q_pc, s_pc, "per_channel"),
            "fc4.weight": ck.packed_linear_record(q_pg, s_pg, "per_group", num_bits=4, group_size=g),
            "pt.weight": ck.packed_linear_record(q_pc, [s_pc[0]], "per_tensor_symmetric")}
    path = tmp_path / "packed.ckpt"
    ck.save_packed(str(path), recs)
    back = ck.load_packed(str(path))
    assert list(back) == list(recs)
    for name, rec in recs.items():
        got = back[name]
        np.testing.assert_array_equal(ck.record_codes(got), ck.record_codes(rec))
        p, q = got["params"], rec["params"]
        assert list(p) == ["scheme", "scale", "zeroPoint", "axis", "groupSize", "dtype", "numBits"]
        if isinstance(q["scale"], float):
            assert p["scale"] == q["scale"]
        else:
            assert p["scale"].dtype == np.float64 and p["scale"].tobytes() == q["scale"].tobytes()
            assert p["zeroPoint"].dtype == np.int32 and not p["zeroPoint"].any()
    assert back["fc4.weight"]["weight"].dtype == "ui8"
    assert back["fc4.weight"]["params"]["groupSize"] == g
    assert back["fc.weight"]["params"]["axis"] == 0
