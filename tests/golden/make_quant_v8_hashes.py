"""Writes quant_v8_hashes.json: per-chunk hashes of the compiled quantize R1
(V8, quant_v8_hashes.js) over all 2^32 binary32 inputs, for each scale in
SCALES (the typical absmax / 127 scales, an inexact decimal, a large and a
power-of-two scale with exact ties, small scales, and two outside the
f32 fast path's range).  Run: python tests/golden/make_quant_v8_hashes.py
"""
import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CHUNKS = 256
SCALES = [1 / 127, 6 / 127, 0.1, 3.0, 0.5, 1.2345e-6, 1e-10, 1e-35, 1e35]


def run(scale, procs=8):
    step = CHUNKS // procs
    runs = [subprocess.Popen(["node", os.path.join(HERE, "quant_v8_hashes.js"), repr(scale), str(a),
                              str(a + step)], stdout=subprocess.PIPE, text=True)
            for a in range(0, CHUNKS, step)]
    rows = {}
    for p in runs:
        out, _ = p.communicate()
        if p.returncode != 0:
            sys.exit(f"node failed ({p.returncode})")
        for line in out.splitlines():
            c, s1, s2 = json.loads(line)
            rows[c] = [s1, s2]
    assert sorted(rows) == list(range(CHUNKS))
    return [rows[c] for c in range(CHUNKS)]


def main():
    doc = {"what": "compiled quantize R1 of every binary32 input, per scale, as V8 evaluates it under Node "
                   + subprocess.check_output(["node", "--version"], text=True).strip()
                   + ", hashed per chunk of 2^24 consecutive bit patterns (quant_v8_hashes.js)",
           "chunk_bits": 24,
           "scales": [repr(s) for s in SCALES],
           "hashes": {repr(s): run(s) for s in SCALES}}
    with open(os.path.join(HERE, "quant_v8_hashes.json"), "w") as f:
        json.dump(doc, f)
        f.write("\n")


if __name__ == "__main__":
    main()
