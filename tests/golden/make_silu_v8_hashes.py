"""Writes silu_v8_hashes.json: the per-chunk hashes of the reference's SiLU
(V8's Math.exp, every f32 step rounded) over all 2^32 binary32 inputs, from
silu_v8_hashes.js run under Node in parallel processes.  Run from anywhere:
    python tests/golden/make_silu_v8_hashes.py
"""
import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CHUNKS = 256


def main(procs=8):
    step = CHUNKS // procs
    runs = [subprocess.Popen(["node", os.path.join(HERE, "silu_v8_hashes.js"), str(a), str(a + step)],
                             stdout=subprocess.PIPE, text=True) for a in range(0, CHUNKS, step)]
    rows = {}
    for p in runs:
        out, _ = p.communicate()
        if p.returncode != 0:
            sys.exit(f"node failed ({p.returncode})")
        for line in out.splitlines():
            c, s1, s2 = json.loads(line)
            rows[c] = [s1, s2]
    assert sorted(rows) == list(range(CHUNKS))
    doc = {"what": "SiLU of every binary32 input as the reference's CPU backend evaluates it "
                   "(Math.fround at every f32 op, Math.exp in f64) under Node " + subprocess.check_output(
                       ["node", "--version"], text=True).strip() + ", hashed per chunk of 2^24 "
                   "consecutive bit patterns (silu_v8_hashes.js)",
           "chunk_bits": 24,
           "hashes": [rows[c] for c in range(CHUNKS)]}
    with open(os.path.join(HERE, "silu_v8_hashes.json"), "w") as f:
        json.dump(doc, f)
        f.write("\n")


if __name__ == "__main__":
    main()
