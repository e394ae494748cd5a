"""Elementwise PrimFuncs and whole-plan execution on the 'hip' target
(mlfw_amd/node/ewise.js, the runtime backend's runPlan, q8_ewise).

CPU: the oracle's restatement of the CPU codegen's expression emission is
pinned by the reference's own codegen-internals vectors; translated device
programs are emulated in JS against it; the per-channel epilogue matcher;
compile routing of tagged and untagged PrimFuncs.
GPU: every elementwise PrimFunc through runSync, and the per-channel
Linear + bias + ReLU PrimFunc set (quantize, qmatmul, the convert-mul tail,
add, max, relu+quantize) through runPlan with and without the fused GEMM
epilogue, bit for bit against the oracle, with upload byte counts.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SCRIPT = os.path.join(ROOT, "tests", "node", "ewise_test.js")
ADDON = os.path.join(ROOT, "mlfw_amd", "node", "q8hip.node")
NODE = shutil.which("node")

needs_node = pytest.mark.skipif(NODE is None, reason="node is not installed")


def run_node(mode, timeout=240):
    r = subprocess.run([NODE, SCRIPT, mode], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    print(r.stderr)
    return r


@needs_node
def test_node_ewise_cpu():
    if not os.path.exists(ADDON):
        pytest.fail("q8hip.node is not built: run `python -m mlfw_amd.build`")
    r = run_node("cpu")
    assert r.returncode == 0 and "all passed" in r.stdout, r.stdout + r.stderr


@needs_node
@pytest.mark.gpu
def test_node_ewise_gpu():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    r = run_node("gpu")
    assert r.returncode == 0 and "all passed" in r.stdout, r.stdout + r.stderr
