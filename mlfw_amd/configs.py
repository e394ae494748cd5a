"""The five synthetic workloads of the int8 path, built and run on the device.

Inputs follow the reference's seeded generators (mulberry32 +
Box-Muller / uniform, src/util/random.ts:5-14, src/nn/init.ts:31-52): each
config seeds one stream and draws its tensors from it in the order listed,
so the i-th tensor starts at the draw count the previous ones consumed.
The device generator is the counter form of the same stream.

C1 qlinear 32x128 -> 64 (seed 0): X N(0,1) [32,128], W N(0,0.02) [64,128],
   bias U(-0.1,0.1) [64].  X per-tensor dynamic (= calibration on X),
   W per-output-channel; y = fround(fround(acc*fround(sX*sW[n])) + b[n]).
C2 MLP 784 -> 256 -> 128 -> 10, batch 256 (seed 1): x U(0,1) [256,784],
   W_l N(0, 1/sqrt(fan_in)) [out,in], per-output-channel; each layer's input
   is quantized per tensor (dynamic); ReLU after layers 1 and 2; fp32 logits.
C3 4096^3 (seed 2): A N(0,1) [M,K] per-token; B N(0,0.02) [K,N] per-column;
   y = fround(acc * fround(sA[m] * sB[n])).
C4 decoder projections, 2048 tokens, hidden 4096 (seed 3): X [2048,4096];
   Wqkv [12288,4096], Wo [4096,4096], Wg, Wu [11008,4096], Wd [4096,11008],
   all N(0,0.02) per-output-channel.  Chain (per-token int8 between
   projections, bias 0): qkv = X Wqkv^T; o = V Wo^T with V = qkv[:, 8192:];
   g = o Wg^T, u = o Wu^T; h = fround(silu(g) * u); d = h Wd^T.
C5 decode shapes (seed 4): GEMV weights W_N N(0,0.02) [N,4096] for
   N = 4096, 11008, then activations x_M N(0,1) [M,4096] for M = 1, 4, 16;
   and the quantize/dequantize tensor X N(0,1) [16384,4096] with 1 % of the
   elements (second stream seeded 4 ^ 0x9e3779b9, draw < 0.01) scaled by 50.
"""
from __future__ import annotations

import math

import torch

from . import ops

SEEDS = {"C1": 0, "C2": 1, "C3": 2, "C4": 3, "C5": 4}
C5_OUTLIER_SEED = (4 ^ 0x9E3779B9) & 0xFFFFFFFF
C4_SHAPES = {"qkv": (12288, 4096), "o": (4096, 4096), "gate": (11008, 4096),
             "up": (11008, 4096), "down": (4096, 11008)}
C5_GEMV_N = (4096, 11008)
C5_GEMV_M = (1, 4, 16)
C5_QUANT_SHAPE = (16384, 4096)


class DeviceStream:
    """A seeded mulberry32 stream consumed in order, filling device tensors."""

    def __init__(self, seed: int, device="cuda"):
        self.seed = seed
        self.offset = 0
        self.device = device

    def normal(self, shape, mean=0.0, std=1.0) -> torch.Tensor:
        t = torch.empty(shape, dtype=torch.float32, device=self.device)
        self.offset += ops.fill_normal(t, self.seed, self.offset, mean, std)
        return t

    def uniform(self, shape, a=0.0, b=1.0) -> torch.Tensor:
        t = torch.empty(shape, dtype=torch.float32, device=self.device)
        self.offset += ops.fill_uniform(t, self.seed, self.offset, a, b)
        return t


# ------------------------------------------------------------------ C1
def c1_inputs(device="cuda"):
    s = DeviceStream(SEEDS["C1"], device)
    return {"X": s.normal((32, 128)), "W": s.normal((64, 128), 0.0, 0.02),
            "bias": s.uniform((64,), -0.1, 0.1)}


def c1_run(X, W, bias):
    Wq, sW = ops.pack_weight(W, axis=0)
    Xq, sX = ops.quantize_per_tensor(X)
    return ops.qlinear(Xq, sX, Wq, sW, bias=bias)


# ------------------------------------------------------------------ C2
C2_DIMS = (784, 256, 128, 10)


def c2_inputs(device="cuda"):
    s = DeviceStream(SEEDS["C2"], device)
    x = s.uniform((256, 784), 0.0, 1.0)
    Ws = [s.normal((C2_DIMS[i + 1], C2_DIMS[i]), 0.0, 1.0 / math.sqrt(C2_DIMS[i]))
          for i in range(3)]
    return {"x": x, "W": Ws}


def c2_prepare(Ws):
    return [ops.pack_weight(W, axis=0) for W in Ws]


def c2_run(x, packed):
    h = x
    for i, (Wq, sW) in enumerate(packed):
        hq, sh = ops.quantize_per_tensor(h)
        h = ops.qlinear(hq, sh, Wq, sW, act="relu" if i < 2 else None)
    return h


# ------------------------------------------------------------------ C3
def c3_inputs(device="cuda", M=4096, N=4096, K=4096):
    s = DeviceStream(SEEDS["C3"], device)
    return {"A": s.normal((M, K)), "B": s.normal((K, N), 0.0, 0.02)}


def c3_prepare(B):
    return ops.pack_weight(B, axis=1)          # [K,N] per column -> [N,K]


def c3_step(A, Bq, sB, out=None, bufs=None):
    Aq, sA = ops.quantize_per_token(A, *(bufs or (None, None)))
    return ops.qlinear(Aq, sA, Bq, sB, out=out)


# ------------------------------------------------------------------ C4
def c4_inputs(device="cuda", tokens=2048):
    s = DeviceStream(SEEDS["C4"], device)
    X = s.normal((tokens, 4096))
    W = {k: s.normal(shape, 0.0, 0.02) for k, shape in C4_SHAPES.items()}
    return {"X": X, "W": W}


def c4_prepare(W):
    """Per-channel int8 weights of the projection set.  Gate and up are
    packed apart (codes and scales are per row) and interleaved into one
    [2 * 11008, 4096] weight in groups of 32 rows ("gate_up_glu"), so one
    GEMM computes both and applies SiLU(gate) * up in its epilogue; the
    plain concatenation [gate; up] ("gate_up") serves the unfused route."""
    P = {k: ops.pack_weight(w, axis=0) for k, w in W.items()}
    P["gate_up_glu"] = ops.glu_interleave(P["gate"], P["up"])
    P["gate_up"] = tuple(torch.cat([P["gate"][i], P["up"][i]], 0) for i in (0, 1))
    del P["gate"], P["up"]
    return P


def c4_step(X, P, fused_requant=False, ws=None, glu=False):
    """One pass of the projection set.  With fused_requant the O projection
    writes its per-token int8 codes and scales directly from the GEMM
    epilogue (q8_gemm_requant_dynamic: 128 co-resident 256 x 256 tiles that
    meet once grid-wide), so its fp32 output never reaches memory; otherwise
    (the default, faster on MI355X at this shape: the fused kernel runs on
    128 of the 256 CUs) it is written and quantized by a second kernel.
    With glu, gate|up runs as q8_gemm_glu (SiLU(gate) * up in the GEMM
    epilogue) followed by the per-token quantize of h; the default runs the
    [gate; up] GEMM and the fused SiLU*up requant kernel.
    Returns every stage's tensors."""
    xq, sx = ops.quantize_per_token(X)
    qkv = ops.qlinear(xq, sx, *P["qkv"])
    vq, sv = ops.quantize_per_token(qkv[:, 8192:])         # row-strided V slice
    out = {"xq": xq, "sx": sx, "qkv": qkv, "vq": vq, "sv": sv}
    if fused_requant:
        oq, so = ops.qlinear_requant_dynamic(vq, sv, *P["o"], workspace=ws)
    else:
        o = ops.qlinear(vq, sv, *P["o"])
        oq, so = ops.quantize_per_token(o)
        out["o"] = o
    if glu:
        # gate and up in one GEMM with h = SiLU(gate) * up in its epilogue
        # (gate and up never reach memory), then the per-token quantize of h.
        # Not the default: on MI355X the epilogue's f64-exp SiLU runs at one
        # wave per SIMD with nothing to hide it (GEMM 219-228 us against 182
        # us without it), more than the 86 MiB of g|u traffic it saves.
        h = ops.qlinear_glu(oq, so, *P["gate_up_glu"])
        hq, sh = ops.quantize_per_token(h)
        out["h"] = h
    else:
        gu = ops.qlinear(oq, so, *P["gate_up"])           # [tokens, gate | up]
        nf = gu.shape[1] // 2
        g, u = gu[:, :nf], gu[:, nf:]                      # row-strided halves
        hq, sh = ops.silu_mul_quantize(g, u)
        out.update({"gate": g, "up": u})
    d = ops.qlinear(hq, sh, *P["down"])
    out.update({"oq": oq, "so": so, "hq": hq, "sh": sh, "down": d})
    return out


C4_OPS = sum(2 * 2048 * n * k for n, k in C4_SHAPES.values())


# ------------------------------------------------------------------ C5
def c5_inputs(device="cuda", with_quant_tensor=True):
    s = DeviceStream(SEEDS["C5"], device)
    W = {n: s.normal((n, 4096), 0.0, 0.02) for n in C5_GEMV_N}
    x = {m: s.normal((m, 4096)) for m in C5_GEMV_M}
    out = {"W": W, "x": x}
    if with_quant_tensor:
        X = s.normal(C5_QUANT_SHAPE)
        ops.apply_outliers(X, C5_OUTLIER_SEED, 0.01, 50.0)
        out["X"] = X
    return out


def c5_gemv(x, Wq, sW, out=None):
    xq, sx = ops.quantize_per_token(x)
    return ops.qlinear(xq, sx, Wq, sW, out=out)


def c5_quant_dequant(X):
    q, s = ops.quantize_per_token(X)
    return q, s, ops.dequantize(q, s)


# ------------------------------------------------------------------ elementwise programs
def ewise_programs(M, N, s_q=0.05, s_dq=0.01):
    """Three elementwise PrimFuncs as q8_ewise runs them on [M, N] (the forms
    QuantizationPass and the fusion rules leave when the chain fusion does
    not take them, quantization_pass.ts:431-456, rules/fusion.ts:66-79):
    (program, input dtypes and shapes, output dtype, bytes per launch)."""
    f32, i32, i8 = torch.float32, torch.int32, torch.int8
    row, col = (N, 1), (0, 1)
    progs = {}
    # fround(fround(acc * sv[n]) + b[n]): the per-channel dequant and bias
    progs["dequant_bias"] = (ops.ew_program((M, N), [(i32, row), (f32, col), (f32, col)], [
        ("load", 0, 0, 0, 0, 0, 0), ("load", 1, 0, 0, 0, 1, 0), ("mul", 2, 0, 1, 0, 0, 1),
        ("load", 3, 0, 0, 0, 2, 0), ("add", 4, 2, 3, 0, 0, 1)], 4, f32),
        [(i32, (M, N)), (f32, (N,)), (f32, (N,))], f32, M * N * 8 + N * 8)
    # (min(max(Math.round(Math.fround(max(x, 0) / s)), -128), 127) | 0): ReLU fused with quantize
    progs["relu_quantize"] = (ops.ew_program((M, N), [(f32, row)], [
        ("load", 0, 0, 0, 0, 0, 0), ("const", 1, 0, 0, 0, 0, 0), ("max", 2, 0, 1, 0, 0, 0),
        ("const", 3, 0, 0, 0, 1, 0), ("div", 4, 2, 3, 0, 0, 1), ("round", 5, 4, 0, 0, 0, 0),
        ("const", 6, 0, 0, 0, 2, 0), ("max", 7, 5, 6, 0, 0, 0), ("const", 8, 0, 0, 0, 3, 0),
        ("min", 9, 7, 8, 0, 0, 0), ("toint32", 10, 9, 0, 0, 0, 0)], 10, i8, konst=(0.0, s_q, -128.0, 127.0)),
        [(f32, (M, N))], i8, M * N * 5)
    # fround(fround(q * s) + y): a dequantize feeding an add
    progs["dequant_add"] = (ops.ew_program((M, N), [(i8, row), (f32, row)], [
        ("load", 0, 0, 0, 0, 0, 0), ("const", 1, 0, 0, 0, 0, 0), ("mul", 2, 0, 1, 0, 0, 1),
        ("load", 3, 0, 0, 0, 1, 0), ("add", 4, 2, 3, 0, 0, 1)], 4, f32, konst=(s_dq,)),
        [(i8, (M, N)), (f32, (M, N))], f32, M * N * 9)
    return progs
