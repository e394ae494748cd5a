"""Regenerate tests/golden/golden.npz from golden_cases.js under Node.

The expectations are computed by a JavaScript engine with the reference's
arithmetic (see golden_cases.js); this script only packs the engine's
outputs into one numpy archive.  Run from the repository root:
    python tests/golden/make_golden.py
"""
import json
import os
import shutil
import subprocess
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BINS = {  # name -> dtype
    "params_skewed_W": np.float32, "params_group_data": np.float32,
    "fakequant_x": np.float32, "fakequant_q": np.int8, "fakequant_y": np.float32,
    "pcmatmul_A": np.float32, "pcmatmul_W": np.float32, "pcmatmul_aq": np.int8,
    "pcmatmul_pc_wq": np.int8, "pcmatmul_pc_acc": np.int32, "pcmatmul_pc_y": np.float32,
    "pcmatmul_pt_wq": np.int8, "pcmatmul_pt_acc": np.int32, "pcmatmul_pt_y": np.float32,
    "edges_x": np.float32,
    "c1_X": np.float32, "c1_W": np.float32, "c1_bias": np.float32, "c1_Xq": np.int8,
    "c1_Wq": np.int8, "c1_sW": np.float64, "c1_acc": np.int32, "c1_y": np.float32,
}


def main():
    node = shutil.which("node")
    if node is None:
        raise SystemExit("node is required to regenerate the golden vectors")
    with tempfile.TemporaryDirectory() as d:
        subprocess.run([node, os.path.join(HERE, "golden_cases.js"), d], check=True)
        arrays = {}
        for name, dt in BINS.items():
            arrays[name] = np.fromfile(os.path.join(d, name + ".bin"), dtype=dt)
        for j in range(5):
            arrays[f"edges_q_{j}"] = np.fromfile(os.path.join(d, f"edges_q_{j}.bin"), dtype=np.int8)
            arrays[f"edges_u_{j}"] = np.fromfile(os.path.join(d, f"edges_u_{j}.bin"), dtype=np.uint8)
        meta = {c: json.load(open(os.path.join(d, c + ".json")))
                for c in ("params", "fakequant", "pcmatmul", "edges", "c1")}
        arrays["meta_json"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
        np.savez_compressed(os.path.join(HERE, "golden.npz"), **arrays)
    print("wrote", os.path.join(HERE, "golden.npz"))


if __name__ == "__main__":
    main()
