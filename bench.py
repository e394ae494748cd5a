#!/usr/bin/env python3
"""Benchmark of the int8 quantized-inference path on one MI355X.

Headline (value): config C3, the 4096^3 int8 qmatmul.  One step = dynamic
per-token quantize of A [4096,4096] fp32 + the int8 GEMM with the fused
per-row x per-column dequant epilogue (fp32 out); B is a prepacked int8
weight.  value = 2*4096^3 int ops / step time, in TOPS (10^12 int ops/s).

The step's two launches are prepared once (mlfw_amd.ops.prepare: arguments
validated and converted up front), so the host enqueues faster than the
GPU executes; the timed region is K steps back to back between two HIP
events on the stream the kernels run on.  The activations (A, its codes
and scales, the output) rotate over 8 sets, 1.1 GiB, so the Infinity Cache
cannot serve one step's tensors from the previous ones.

roofline: the GEMM kernel's average duration in the timed region, i.e.
the step time less the quantize's (timed alone over K launches between
two events on the same stream); peak = MI355X dense int8 MFMA, 5.0 POP/s.
(GEMMs launched back to back on their own run ~15-20% longer: without the
quantize between them the part holds the MFMA load and lowers its clock.)
`traffic` is the HBM bytes per launch from rocprofv3 FETCH_SIZE +
WRITE_SIZE runs (profiles/traffic.json, scaled by a copy-kernel
calibration), or null when that file is absent.

secondary: the HBM-bound kernels of C5 (per-token quantize and dequantize
of [16384,4096], GEMVs M in {1,4,16} x N in {4096,11008}, and the same
GEMVs for M <= 4 with 4-bit per-group weights, and the one-call dynamic
qlinear), the C4 projection set, quantized_conv on ResNet-style layers at
batch 32 (synthetic int8 data), and three elementwise programs through
q8_ewise.  Each is captured R times in a
HIP graph (rotating input buffers so the 256 MB Infinity Cache cannot
serve repeats, except conv, whose inputs are a few MB) and the graph is
replayed between two events: per-launch host overhead would otherwise
dominate kernels of a few microseconds.

cpu_baseline: the reference's generated single-thread CPU kernels, mirrored
in JavaScript (oracle/q8ref.js), timed under Node on one host core over a
row slice of the same GEMM.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import shutil
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "int8 qmatmul TOPS @4096³ (% MFMA peak); quant/dequant GB/s (% HBM peak)"
PEAK_INT8_TOPS = 5000.0        # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
GEMM_OPS = 2 * 4096 ** 3
GEMM_KERNEL = "k_qgemm<256, 256, 8>"   # tile 256x256, fp32 out, row x column scales
C3_SETS = 8                    # activation sets the C3 steps rotate over (1.1 GiB)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def ev():
    import torch
    return torch.cuda.Event(enable_timing=True)


def load_traffic():
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


# ---------------------------------------------------------------- headline
# Untimed load before the warm-up steps: the part raises its clocks over the
# first tens of milliseconds of load, so the C3 step runs for at least this
# long (wall time, synchronized) before the W warm-up steps and the timed K.
SETTLE_MS = 150.0


def bench_c3(steps, warmup, settle_ms=SETTLE_MS):
    import torch
    from mlfw_amd import configs as C
    from mlfw_amd import ops as O

    inp = C.c3_inputs("cuda")
    Bq, sB = C.c3_prepare(inp["B"])
    # The activations rotate over C3_SETS sets of (A fp32, Aq, sA, out):
    # 8 x 144 MiB = 1.1 GiB, so the 256 MB Infinity Cache cannot hold the
    # previous steps' tensors and every step reads A from HBM and writes out
    # to fresh memory.  B (the 16 MiB int8 weight) is shared, as a layer's
    # weight is across tokens.
    quants, gemms = [], []
    for i in range(C3_SETS):
        A = inp["A"] if i == 0 else inp["A"].clone()
        out = torch.empty((4096, 4096), dtype=torch.float32, device="cuda")
        Aq = torch.empty((4096, 4096), dtype=torch.int8, device="cuda")
        sA = torch.empty(4096, dtype=torch.float64, device="cuda")
        quants.append(O.prepare(O.quantize_per_token, A, Aq, sA))
        gemms.append(O.prepare(O.qlinear, Aq, sA, Bq, sB, out=out))
    # clock settling: chunks of 50 steps until settle_ms of wall time
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    settle_steps = 0
    while settle_ms > 0 and (time.perf_counter() - t0) * 1e3 < settle_ms:
        for w in range(50):
            quants[w % C3_SETS]()
            gemms[w % C3_SETS]()
        torch.cuda.synchronize()
        settle_steps += 50
    settled_ms = (time.perf_counter() - t0) * 1e3
    for w in range(warmup):
        quants[w % C3_SETS]()
        gemms[w % C3_SETS]()
    torch.cuda.synchronize()

    # (1) the timed steps: quantize + GEMM back to back, nothing in between
    t_begin, t_end = ev(), ev()
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_begin.record()
    for k in range(steps):
        quants[k % C3_SETS]()
        gemms[k % C3_SETS]()
    t_end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    step_ms = t_begin.elapsed_time(t_end) / steps

    # (2) the GEMM's average duration in the timed region: the step time
    # less the quantize's, the quantize timed alone over K launches back to
    # back between two events on the same stream (memory-bound, it runs
    # the same alone as between GEMMs).  Event pairs around every launch
    # would add a marker and a dispatch gap (~6 us) to each interval, and
    # GEMMs launched back to back on their own hold the MFMA load without
    # a break, so the part lowers its clock (~90 us instead of ~75-80 us).
    # The GEMM's share keeps one dispatch gap per step: it errs high.
    a, b = ev(), ev()
    torch.cuda.synchronize()
    a.record()
    for k in range(steps):
        quants[k % C3_SETS]()
    b.record()
    torch.cuda.synchronize()
    quant_ms = a.elapsed_time(b) / steps
    gemm_ms = step_ms - quant_ms
    return {
        "step_ms": step_ms,
        "settle_steps": settle_steps,
        "settle_ms": settled_ms,
        "wall_ms_per_step": 1e3 * wall / steps,
        "gemm_avg_ms": gemm_ms,
        "quant_avg_ms": quant_ms,
    }


# ---------------------------------------------------------------- secondary
_CAPTURE = []


def _capture_stream():
    """One side stream for every graph capture of the run."""
    import torch
    if not _CAPTURE:
        _CAPTURE.append(torch.cuda.Stream())
    return _CAPTURE[0]


GRAPH_SETTLE_MS = 20.0


def graph_time_us(body, copies, replays=5, batches=3, settle_ms=GRAPH_SETTLE_MS):
    """Microseconds per launch of body(i), i < copies, captured in one HIP
    graph: the median over `batches` batches of `replays` replays, each
    batch between two events, after at least settle_ms of untimed replays
    (freshly allocated and written buffers run unevenly for the first few
    milliseconds: the C5 quantize swings between 53 and 66 us over its first
    ~200 launches, then holds 53-54 us).  Falls back to eager launches if
    capture is not possible."""
    import torch
    try:
        # warm up on the stream the graph is captured on: per-stream state
        # (the GEMM's stream-K workspace) is made there, outside the capture
        s = _capture_stream()
        with torch.cuda.stream(s):
            for i in range(copies):
                body(i)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for i in range(copies):
                body(i)
        g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < settle_ms:
            g.replay()
            torch.cuda.synchronize()
        per = []
        for _ in range(batches):
            a, b = ev(), ev()
            a.record()
            for _ in range(replays):
                g.replay()
            b.record()
            torch.cuda.synchronize()
            per.append(1e3 * a.elapsed_time(b) / (replays * copies))
        return sorted(per)[len(per) // 2], "graph"
    except Exception as exc:            # eager fallback, reported
        log(f"[bench] graph capture failed ({exc!r}); timing eager launches")
        a, b = ev(), ev()
        a.record()
        for _ in range(replays):
            for i in range(copies):
                body(i)
        b.record()
        torch.cuda.synchronize()
        return 1e3 * a.elapsed_time(b) / (replays * copies), "eager"


def bench_c5_quant():
    import torch
    from mlfw_amd import configs as C
    from mlfw_amd import ops as O
    X0 = C.c5_inputs("cuda")["X"]
    M, K = X0.shape
    n_in = 5                                   # 5 x 256 MiB fp32 inputs: > 4 x the MALL
    Xs = [X0] + [X0.clone() for _ in range(n_in - 1)]
    qs = [torch.empty((M, K), dtype=torch.int8, device="cuda") for _ in range(n_in)]
    ss = [torch.empty(M, dtype=torch.float64, device="cuda") for _ in range(n_in)]
    ys = [torch.empty((M, K), dtype=torch.float32, device="cuda") for _ in range(n_in)]
    nbytes = M * K * 4 + M * K + M * 8
    q_us, q_how = graph_time_us(lambda i: O.quantize_per_token(Xs[i], qs[i], ss[i]), n_in)
    d_us, d_how = graph_time_us(lambda i: O.dequantize(qs[i], ss[i], out=ys[i]), n_in)
    res = {}
    for name, us, how in (("quantize_per_token_16384x4096", q_us, q_how),
                          ("dequantize_per_token_16384x4096", d_us, d_how)):
        gbs = nbytes / (us * 1e-6) / 1e9
        res[name] = {"avg_us": us, "bytes": nbytes, "GB/s": gbs,
                     "frac_hbm": gbs / PEAK_HBM_GBS, "timing": how}
    return res


def _ewise_compiled_launches():
    import ctypes
    from mlfw_amd import _lib
    n = ctypes.c_int64(0)
    _lib.call("q8_debug_ewise_jit", -1, None, ctypes.byref(n))
    return n.value


def bench_ewise():
    """q8_ewise on the elementwise PrimFuncs the GEMM chain fusion does not
    absorb, on [4096, 4096] (2^24 elements: the hiprtc-compiled route):
    graph replays over 4 rotating input and output sets (320-576 MiB, more
    than the 256 MB MALL)."""
    import torch
    from mlfw_amd import ops as O
    M = N = 4096
    res = {}
    g = torch.Generator(device="cuda").manual_seed(11)
    from mlfw_amd import configs as C
    for name, (prog, ins, odt, nbytes) in C.ewise_programs(M, N).items():
        n = 4
        sets = []
        for _ in range(n):
            ts = []
            for dt, shape in ins:
                if dt == torch.float32:
                    ts.append(torch.randn(shape, device="cuda", generator=g))
                else:
                    ts.append(torch.randint(-1000 if dt == torch.int32 else -128, 1000 if dt == torch.int32 else 128,
                                            shape, dtype=dt, device="cuda", generator=g))
            sets.append((ts, torch.empty((M, N), dtype=odt, device="cuda")))
        l0 = _ewise_compiled_launches()
        us, how = graph_time_us(lambda i: O.ewise(prog, sets[i][0], sets[i][1]), n)
        gbs = nbytes / (us * 1e-6) / 1e9
        # which of q8_ewise's routes ran: compiled launches counted by the library
        compiled = _ewise_compiled_launches() > l0
        res[f"ewise_{name}_4096x4096"] = {"avg_us": us, "bytes": nbytes, "GB/s": gbs,
                                           "frac_hbm": gbs / PEAK_HBM_GBS, "timing": how,
                                           "route": "compiled" if compiled else "interpreted"}
        if not compiled:
            res[f"ewise_{name}_4096x4096"]["compile_error"] = O.ewise_jit_error()[:400]
        del sets
    return res


def bench_c5_gemv():
    import torch
    from mlfw_amd import configs as C
    from mlfw_amd import ops as O
    inp = C.c5_inputs("cuda", with_quant_tensor=False)
    K = 4096
    res = {}
    for N, W in inp["W"].items():
        Wq0, sW = O.pack_weight(W, axis=0)
        R = max(8, math.ceil((1 << 30) / (N * K)))          # > 1 GiB of distinct weights
        Wqs = [Wq0] + [Wq0.clone() for _ in range(R - 1)]
        for M, x in inp["x"].items():
            xq, sx = O.quantize_per_token(x)
            outs = [torch.empty((M, N), dtype=torch.float32, device="cuda") for _ in range(R)]
            g_us, how = graph_time_us(lambda i: O.qlinear(xq, sx, Wqs[i], sW, out=outs[i]), R)
            q_us, _ = graph_time_us(lambda i: O.quantize_per_token(x, xq, sx), 8)
            # the whole dynamic linear in one call (one kernel for M <= 4)
            d_us, _ = graph_time_us(
                lambda i: O.qlinear_dynamic(x, Wqs[i], sW, out=outs[i], xq=xq, sx=sx), R)
            kb = N * K + 8 * N + M * K + 8 * M + 4 * M * N      # the GEMV kernel's own bytes
            sb = N * K + 8 * N + 4 * M * K + 4 * M * N          # step bytes (fp32 x in)
            res[f"gemv_M{M}_N{N}"] = {
                "gemv_avg_us": g_us, "gemv_GB/s": kb / (g_us * 1e-6) / 1e9,
                "gemv_frac_hbm": kb / (g_us * 1e-6) / 1e9 / PEAK_HBM_GBS,
                "quantize_x_avg_us": q_us,
                "step_GB/s": sb / ((g_us + q_us) * 1e-6) / 1e9,
                "qlinear_dynamic_avg_us": d_us, "qlinear_dynamic_GB/s": sb / (d_us * 1e-6) / 1e9,
                "qlinear_dynamic_frac_hbm": sb / (d_us * 1e-6) / 1e9 / PEAK_HBM_GBS,
                "timing": how,
            }
        # the same weights as 4-bit per-group codes (group 128): W4A8 decode GEMV
        g = 128
        Wq40, sW4 = O.pack_weight_int4(W, g)
        Wq4s = [Wq40] + [Wq40.clone() for _ in range(2 * R - 1)]      # same > 1 GiB rotation
        for M, x in inp["x"].items():
            xq, sx = O.quantize_per_token(x)
            outs = [torch.empty((M, N), dtype=torch.float32, device="cuda") for _ in range(2 * R)]
            g_us, how = graph_time_us(lambda i: O.qlinear_w4(xq, sx, Wq4s[i], sW4, K, g, out=outs[i]),
                                      2 * R)
            kb = N * K // 2 + 8 * N * K // g + M * K + 8 * M + 4 * M * N
            res[f"gemv_w4_M{M}_N{N}"] = {
                "gemv_avg_us": g_us, "gemv_GB/s": kb / (g_us * 1e-6) / 1e9,
                "gemv_frac_hbm": kb / (g_us * 1e-6) / 1e9 / PEAK_HBM_GBS,
                "bytes": kb, "group": g, "timing": how}
        del Wqs, Wq4s
    return res


def bench_c4(fused_requant=True):
    import torch
    from mlfw_amd import configs as C
    inp = C.c4_inputs("cuda")
    P = C.c4_prepare(inp["W"])
    del inp["W"]
    X = inp["X"]
    from mlfw_amd import ops as O
    us, how = graph_time_us(lambda i: C.c4_step(X, P), 1, replays=5)
    ms = us / 1e3
    res = {"avg_ms": ms, "ops": C.C4_OPS, "TOPS": C.C4_OPS / (ms * 1e-3) / 1e12,
           "frac_mfma": C.C4_OPS / (ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, "timing": how}
    if fused_requant:
        # the same step with the O projection's per-token requant fused into
        # its GEMM epilogue (no fp32 intermediate; the tiles meet once grid-wide)
        nb, fused = O.requant_dynamic_workspace(X.shape[0], *C.C4_SHAPES["o"])
        ws = torch.empty(nb, dtype=torch.int8, device="cuda")
        us_f, _ = graph_time_us(lambda i: C.c4_step(X, P, fused_requant=True, ws=ws), 1, replays=5)
        res.update({"fused_o_requant_ms": us_f / 1e3, "fused_o_route": fused})
    return {"c4_projection_set": res}


# ResNet-50-style conv layers at batch 32: N, C, H, W, O, kernel, padding
# (stride 1, one group)
CONV_LAYERS = [(32, 64, 56, 56, 64, 3, 1), (32, 128, 28, 28, 128, 3, 1), (32, 256, 14, 14, 256, 3, 1),
               (32, 512, 7, 7, 512, 3, 1), (32, 1024, 14, 14, 256, 1, 0)]


def bench_conv():
    """quantized_conv with the fused per-tensor dequant (fp32 out), int8
    operands: the whole call per launch (frame transpose, implicit GEMM,
    split-K finish where planned), 8 calls per graph.  The constant weight
    is prepacked once (conv_weight_taps); avg_us_unpacked_weight is the call
    that permutes the weight itself."""
    import torch
    from mlfw_amd import ops as O
    res = {}
    ws = torch.empty(1 << 28, dtype=torch.int8, device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(7)
    for (N, C, H, W, Oc, k, p) in CONV_LAYERS:
        x = torch.randint(-128, 128, (N, C, H, W), dtype=torch.int8, device="cuda", generator=gen)
        w = torch.randint(-128, 128, (Oc, C, k, k), dtype=torch.int8, device="cuda", generator=gen)
        pad = [[p, p], [p, p]]
        s_out = 1e-4
        wt = O.conv_weight_taps(w)
        out = O.quantized_conv(x, w, [1, 1], pad, s_out=s_out, workspace=ws, w_taps=wt)
        us, how = graph_time_us(
            lambda i: O.quantized_conv(x, w, [1, 1], pad, s_out=s_out, out=out, workspace=ws, w_taps=wt), 8)
        us_raw, _ = graph_time_us(
            lambda i: O.quantized_conv(x, w, [1, 1], pad, s_out=s_out, out=out, workspace=ws), 8)
        Ho, Wo = H + 2 * p - k + 1, W + 2 * p - k + 1
        ops = 2 * N * Oc * Ho * Wo * C * k * k
        tops = ops / (us * 1e-6) / 1e12
        res[f"conv_N{N}_C{C}_{H}x{W}_O{Oc}_k{k}"] = {
            "avg_us": us, "ops": ops, "TOPS": tops, "frac_mfma": tops / PEAK_INT8_TOPS, "timing": how,
            "weight": "prepacked" if wt is not None else "as given (1 x 1)", "avg_us_unpacked_weight": us_raw}
        del x, w, out, wt
    return res


def bench_napi_plans(calls=200):
    """Whole plans through the Node drop-in (mlfw_amd/node/plan_bench.js):
    the 'hip' runtime backend's runPlan over the N-API addon, per-call host
    time for C2 (batch 256) and a four-linear one-token decode chain, eager
    and as replayed HIP graphs, with inputs uploaded every call and pinned
    resident.  Runs in a child process (its own HIP context)."""
    node = shutil.which("node")
    if node is None:
        return {"napi_plans": {"error": "node is not installed"}}
    script = os.path.join(ROOT, "mlfw_amd", "node", "plan_bench.js")
    r = subprocess.run([node, script, str(calls)], capture_output=True, text=True, timeout=300)
    if r.returncode != 0:
        return {"napi_plans": {"error": f"plan_bench.js exited {r.returncode}: {r.stderr[-400:]}"}}
    return {"napi_plans": json.loads(r.stdout.strip().splitlines()[-1])}


# ---------------------------------------------------------------- ceilings
def ceilings():
    """Practical ceilings measured on this box (mlfw_amd/libq8ceiling.so):
    the C3 GEMM's MFMA work alone with random int8 operands (the clock the
    part holds under that load), and the streaming-read time of one kernel
    at the byte counts of the HBM-bound workloads (launch and ramp
    included).  Reported beside the roofline fractions, which stay against
    the datasheet peaks."""
    import ctypes as C
    from mlfw_amd import build as B
    lib = C.CDLL(B.CEILING_LIB)
    lib.q8c_mfma.argtypes = [C.c_int, C.c_int, C.POINTER(C.c_double), C.POINTER(C.c_double),
                             C.POINTER(C.c_double)]
    lib.q8c_stream.argtypes = [C.c_size_t, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double)]
    us, mhz, cyc = C.c_double(), C.c_double(), C.c_double()
    out = {}
    if lib.q8c_mfma(2048, 10, C.byref(us), C.byref(mhz), C.byref(cyc)) == 0:
        tops = GEMM_OPS / (us.value * 1e-6) / 1e12
        out["mfma_random_int8_4096cube"] = {
            "what": "256 workgroups x 4 waves x 2048 v_mfma_i32_32x32x32_i8 (the C3 GEMM's MFMA "
                    "count), random operands cycled through 16 register fragments, no loads, "
                    "stores or other instructions in the loop",
            "avg_us": us.value, "TOPS": tops, "frac_of_peak": tops / PEAK_INT8_TOPS,
            "shader_clock_mhz": mhz.value,
            "loop_mfma_busy": 2048 * 32 / cyc.value if cyc.value > 0 else None}
    for kind, name, nbytes in (("read", "gemv_N4096", 4096 * 4096 + 8 * 4096 + 4 * 4096),
                               ("read", "gemv_N11008", 11008 * 4096 + 8 * 11008 + 4 * 4096),
                               ("read", "quantize_16384x4096", 335675392),
                               ("write", "dequantize_out_16384x4096", 268435456)):
        bufs = max(5, math.ceil((1 << 30) / nbytes))
        # best of three timed batches: a ceiling is the fastest the box
        # reaches, and one batch now and then runs several times slower
        best = None
        for _ in range(3):
            if lib.q8c_stream(nbytes, bufs, 5, 1 if kind == "write" else 0, C.byref(us)) == 0:
                best = us.value if best is None else min(best, us.value)
        if best is not None:
            gbs = nbytes / (best * 1e-6) / 1e9
            out[f"{kind}_{name}"] = {"bytes": nbytes, "avg_us": best, "GB/s": gbs,
                                     "frac_of_peak": gbs / PEAK_HBM_GBS,
                                     "of": "best of 3 batches of 5 graph replays"}
    return out


# ---------------------------------------------------------------- CPU baseline
def host_cpu():
    """The host CPU's model name and the cores this process may use."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"cpu_model": model, "nproc": usable, "os_cpu_count": os.cpu_count()}


def cpu_baseline(rows=256):
    """Reference CPU path (mirrored generated JS, one core) on `rows` rows of
    the 4096^3 GEMM: quantized_dot triple loop + fused per-channel epilogue."""
    res = _cpu_baseline(rows)
    res.update(host_cpu())
    return res


def _cpu_baseline(rows):
    node = shutil.which("node")
    js = os.path.join(ROOT, "oracle", "q8ref.js")
    if node and os.path.exists(js):
        p = {"kind": "qdot", "M": rows, "N": 4096, "K": 4096, "reps": 3, "seed": 2}
        r = subprocess.run([node, js, "bench", json.dumps(p)], capture_output=True, text=True,
                           timeout=600, check=True)
        res = json.loads(r.stdout.strip().splitlines()[-1])
        tops = res["ops"] / res["seconds"] / 1e12
        return {"value": tops, "unit": "TOPS", "cores": 1, "kind": "port",
                "sample": (f"{rows} of 4096 rows of the 4096^3 qmatmul (quantized_dot + "
                           f"per-channel epilogue), median of 3 after 1 warm-up, JS kernels "
                           f"mirroring mlfw's CPU codegen on Node {res.get('node')}"),
                "seconds_per_sample": res["seconds"]}
    from oracle import q8ref
    import numpy as np
    rng = np.random.default_rng(2)
    A = rng.integers(-127, 128, (rows, 4096)).astype(np.int8)
    B = rng.integers(-127, 128, (4096, 4096)).astype(np.int8)
    t0 = time.perf_counter()
    acc = q8ref.quantized_dot(A, B, b_layout=1)
    q8ref.epilogue(acc, "rowcol", 1e-3, np.full(4096, 1e-3))
    dt = time.perf_counter() - t0
    return {"value": 2 * rows * 4096 * 4096 / dt / 1e12, "unit": "TOPS", "cores": 1,
            "kind": "port", "sample": f"{rows} rows of the 4096^3 qmatmul, C restatement -O2",
            "seconds_per_sample": dt}


# ---------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    # the part ramps its clocks over the first few tens of milliseconds of
    # load; an untimed settling phase (--settle-ms of the same step) comes
    # before the W warm-up steps, so a small W does not leave the timed
    # steps on the ramp
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="untimed wall time of C3 steps before the warm-up steps (0: none)")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-fused-requant", action="store_true",
                    help="skip the C4 step with the O projection's requant fused into its GEMM")
    ap.add_argument("--skip", action="append", default=[], metavar="NAME",
                    help="leave out one secondary workload (c5_quant, c5_gemv, c4, conv, ewise, napi_plans); repeatable")
    ap.add_argument("--no-ceilings", action="store_true",
                    help="skip the MFMA / streaming-read ceiling measurements")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB device copy three times: the known-size "
                         "reference that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "the int8 path has no multi-GPU code: every kernel runs on one GPU's share at its real shape",
              file=sys.stderr)
        return 2
    if args.steps < 1 or args.warmup < 0:
        print("bench.py: --steps must be >= 1 and --warmup >= 0", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    from mlfw_amd import _lib
    _lib.call("q8_init", 0)

    log(f"[bench] C3 4096^3: warmup {args.warmup}, steps {args.steps}")
    if args.settle_ms < 0:
        print("bench.py: --settle-ms must be >= 0", file=sys.stderr)
        return 2
    r = bench_c3(args.steps, args.warmup, args.settle_ms)
    tops = GEMM_OPS / (r["step_ms"] * 1e-3) / 1e12
    gemm_tops = GEMM_OPS / (r["gemm_avg_ms"] * 1e-3) / 1e12
    log(f"[bench] step {r['step_ms']:.4f} ms -> {tops:.1f} TOPS; gemm {r['gemm_avg_ms'] * 1e3:.1f} us "
        f"-> {gemm_tops:.1f} TOPS; host {r['wall_ms_per_step']:.4f} ms/step")

    traffic = load_traffic().get("gemm_4096", {})
    roofline = {"bound": "mfma", "achieved": gemm_tops, "peak": PEAK_INT8_TOPS, "unit": "TOPS",
                "frac": gemm_tops / PEAK_INT8_TOPS,
                "traffic": traffic.get("hbm_bytes_per_launch"),
                "kernel": GEMM_KERNEL, "avg_us": r["gemm_avg_ms"] * 1e3,
                "algorithmic_ops_per_launch": GEMM_OPS}

    if args.copy_calibration:
        # a plain elementwise copy of known size: 16384 rows of 16 KiB read from
        # every other 16 KiB of a 512 MiB buffer (a strided view, so torch runs
        # its direct-copy kernel rather than a DMA blit) and written densely
        big = torch.ones((16384, 8192), dtype=torch.float32, device="cuda")
        src = big[:, :4096]
        dst = torch.empty((16384, 4096), dtype=torch.float32, device="cuda")
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: 3 x {dst.numel() * 4} B read + {dst.numel() * 4} B written")
        del big, src, dst

    secondary = {}
    if not args.no_secondary:
        c4 = lambda: bench_c4(fused_requant=not args.no_fused_requant)
        for name, fn in (("c5_quant", bench_c5_quant), ("c5_gemv", bench_c5_gemv), ("c4", c4),
                         ("conv", bench_conv), ("ewise", bench_ewise), ("napi_plans", bench_napi_plans)):
            if name in args.skip:
                continue
            log(f"[bench] secondary {name}")
            try:
                secondary.update(fn())
            except Exception as exc:          # reported, never hidden
                secondary[name] = {"error": repr(exc)}
            torch.cuda.empty_cache()

    ceil = None
    if not args.no_ceilings:
        log("[bench] ceilings (random-operand MFMA, single-kernel streaming reads)")
        try:
            ceil = ceilings()
            m = ceil.get("mfma_random_int8_4096cube")
            if m:
                roofline["practical_ceiling"] = {
                    "achieved": m["TOPS"], "unit": "TOPS", "frac_of_peak": m["frac_of_peak"],
                    "shader_clock_mhz": m["shader_clock_mhz"],
                    "gemm_frac_of_ceiling": gemm_tops / m["TOPS"]}
        except Exception as exc:
            ceil = {"error": repr(exc)}

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline (JS mirror of the reference CPU kernels, 1 core)")
        try:
            cpu = cpu_baseline()
        except Exception as exc:
            cpu = {"error": repr(exc)}

    line = {
        "metric": METRIC,
        "value": tops,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["step_ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded mulberry32 + Box-Muller on the device, config seed 2)",
        "config": {"workload": "C3: int8 qmatmul M=N=K=4096, A fp32 N(0,1) per-token dynamic "
                               "int8, B N(0,0.02) per-column int8 (prepacked), int32 acc, "
                               "fp32 out = fround(acc*fround(sA[m]*sB[n]))",
                   "M": 4096, "N": 4096, "K": 4096, "step": "quantize_per_token(A) + gemm",
                   "residency": (f"A fp32, Aq, sA and out rotate over {C3_SETS} sets (1.1 GiB > the "
                                 "256 MB Infinity Cache); B (16 MiB int8) is shared by every step"),
                   "quantize_avg_us": r["quant_avg_ms"] * 1e3,
                   "clock_settle": {"ms": r["settle_ms"], "steps": r["settle_steps"],
                                    "what": "untimed C3 steps before the W warm-up steps"},
                   "wall_ms_per_step": r["wall_ms_per_step"]},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "ceilings": ceil,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
