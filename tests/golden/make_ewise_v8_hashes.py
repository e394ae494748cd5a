"""Writes ewise_v8_hashes.json: per-chunk hashes of Math.fround(Math.exp(x)),
Math.fround(Math.log(x)) and Math.fround(Math.tanh(x)) -- the reference CPU
backend's f32 exp / log / tanh externs -- over all 2^32 binary32 inputs,
from ewise_v8_hashes.js run under Node in parallel processes.  Run from
anywhere:
    python tests/golden/make_ewise_v8_hashes.py
"""
import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CHUNKS = 256
FUNCS = ("exp", "log", "tanh")


def hashes(fn, procs=8):
    step = CHUNKS // procs
    runs = [subprocess.Popen(["node", os.path.join(HERE, "ewise_v8_hashes.js"), fn, str(a), str(a + step)],
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
    return [rows[c] for c in range(CHUNKS)]


def main():
    node = subprocess.check_output(["node", "--version"], text=True).strip()
    doc = {"what": "Math.fround(Math.<fn>(x)) for every binary32 x (the reference CPU backend's f32 "
                   f"exp / log / tanh externs) under Node {node}, hashed per chunk of 2^24 consecutive "
                   "bit patterns (ewise_v8_hashes.js)",
           "chunk_bits": 24}
    for fn in FUNCS:
        doc[fn] = hashes(fn)
    with open(os.path.join(HERE, "ewise_v8_hashes.json"), "w") as f:
        json.dump(doc, f)
        f.write("\n")


if __name__ == "__main__":
    main()
