"""End-to-end parity of the five BASELINE workloads on the GPU.

Inputs are drawn by the oracle's seeded stream on the host and uploaded, so
the device pipeline (mlfw_amd/configs.py) and the oracle pipeline
(oracle/configs.py) see identical bits.  Every comparison is bit-exact.
For the 4096^3 GEMM and the decoder projections the oracle computes a row
subset (rows are independent: per-token scales, per-channel weights), and
the full-size result is checked stage by stage: codes and scales against
the oracle, int32 accumulators against an exact f64 matmul of the same int8
values, and the epilogue against the oracle epilogue applied to those
accumulators.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module")
def mods():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from mlfw_amd import configs as C
    from mlfw_amd import ops as O
    from oracle import configs as OC
    return C, O, OC


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def same_bits(a, b, what=""):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    av = a.view(np.uint8).reshape(-1, a.itemsize)
    bv = b.view(np.uint8).reshape(-1, b.itemsize)
    bad = np.nonzero(np.any(av != bv, axis=1))[0]
    assert bad.size == 0, (f"{what}: {bad.size} of {a.size} differ; first at {bad[0]}: "
                           f"{a.reshape(-1)[bad[0]]!r} vs {b.reshape(-1)[bad[0]]!r}")


def test_c1_qlinear(mods, oracle):
    C, O, OC = mods
    inp, y_ref = OC.c1()
    y = C.c1_run(dev(inp["X"]), dev(inp["W"]), dev(inp["bias"]))
    same_bits(host(y), y_ref, "C1")


def test_c2_mlp(mods, oracle):
    C, O, OC = mods
    inp, y_ref = OC.c2()
    packed = C.c2_prepare([dev(w) for w in inp["W"]])
    y = C.c2_run(dev(inp["x"]), packed)
    same_bits(host(y), y_ref, "C2 logits")


def test_c3_gemm_4096(mods, oracle):
    C, O, OC = mods
    inp = OC.c3_inputs()
    A, B = dev(inp["A"]), dev(inp["B"])
    Bq, sB = C.c3_prepare(B)
    y = C.c3_step(A, Bq, sB)
    y_h = host(y)
    # exact expected values for a spread of rows
    rows = np.r_[0:16, 2040:2056, 4080:4096, np.random.default_rng(2).integers(0, 4096, 16)]
    same_bits(y_h[rows], OC.c3_expected_rows(inp, rows), "C3 rows")
    # full size, stage by stage
    Aq, sA = O.quantize_per_token(A)
    s_ref = oracle.scales_per_token(inp["A"])
    same_bits(host(sA), s_ref, "C3 sA")
    Aq_ref = oracle.quantize_rows(inp["A"], s_ref)
    same_bits(host(Aq), Aq_ref, "C3 Aq")
    Bq_ref, sB_ref = OC.pack_pc(inp["B"], 1)
    same_bits(host(sB), sB_ref, "C3 sB")
    same_bits(host(Bq), Bq_ref, "C3 Bq")
    acc = O.quantized_dot(Aq, Bq)
    exact = Aq.double() @ Bq.double().t().contiguous()
    torch.cuda.synchronize()
    assert torch.equal(acc.double(), exact), "C3 int32 accumulators"
    same_bits(y_h, oracle.epilogue(host(acc), "rowcol", s_ref, sB_ref), "C3 epilogue")


def exact_acc(Aq, Bq):
    """int32 accumulators of int8 [M,K] x [N,K]^T through an f64 matmul:
    every partial sum is an integer below 2^53 (|acc| <= K * 128 * 128)."""
    return (Aq.astype(np.float64) @ Bq.astype(np.float64).T).astype(np.int32)


def interleave_rows(g, u):
    """numpy form of the GLU weight layout (groups of 32 gate rows, then the
    same 32 up rows)."""
    F = g.shape[0]
    out = np.empty((2 * F,) + g.shape[1:], g.dtype)
    for j in range(F // 32):
        out[64 * j:64 * j + 32] = g[32 * j:32 * j + 32]
        out[64 * j + 32:64 * j + 64] = u[32 * j:32 * j + 32]
    return out


@pytest.mark.parametrize("fused,glu", [(False, True), (True, True), (False, False)])
def test_c4_decoder_projections(mods, oracle, fused, glu):
    """Every stage of the projection set on all 2048 tokens, each fed the
    device's own inputs: int32 accumulators against an exact f64 matmul, the
    per-channel epilogue, the per-token quantizes (the O projection's fused
    into its GEMM when `fused`), SiLU*up (in the gate|up GEMM's epilogue
    when `glu`) and its requant against the oracle; plus 8 tokens end to end
    from X."""
    C, O, OC = mods
    inp = OC.c4_inputs()
    packed_ref = {k: OC.pack_pc(w, 0) for k, w in inp["W"].items()}
    P = C.c4_prepare({k: dev(w) for k, w in inp["W"].items()})
    # gate and up run as one GEMM: over the concatenated weight, or the
    # interleaved one with SiLU*up fused
    packed_ref["gate_up"] = tuple(np.concatenate([packed_ref["gate"][i], packed_ref["up"][i]]) for i in (0, 1))
    packed_ref["gate_up_glu"] = tuple(interleave_rows(packed_ref["gate"][i], packed_ref["up"][i]) for i in (0, 1))
    for k in P:
        same_bits(host(P[k][1]), packed_ref[k][1], f"C4 {k} scales")
        same_bits(host(P[k][0]), packed_ref[k][0], f"C4 {k} codes")
    out = C.c4_step(dev(inp["X"]), P, fused_requant=fused, glu=glu)
    h = {k: host(v) for k, v in out.items()}

    def quant(x, q, s, what):
        s_ref = oracle.scales_per_token(x)
        same_bits(s, s_ref, f"{what} scales")
        same_bits(q, oracle.quantize_rows(x, s_ref), f"{what} codes")

    def linear(xq, sx, wname, y, what):
        Wq, sW = packed_ref[wname]
        same_bits(y, oracle.epilogue(exact_acc(xq, Wq), "rowcol", sx, sW), what)

    quant(inp["X"], h["xq"], h["sx"], "C4 x quantize")
    linear(h["xq"], h["sx"], "qkv", h["qkv"], "C4 qkv (all rows)")
    quant(np.ascontiguousarray(h["qkv"][:, 8192:]), h["vq"], h["sv"], "C4 v quantize")
    o_ref = oracle.epilogue(exact_acc(h["vq"], packed_ref["o"][0]), "rowcol", h["sv"], packed_ref["o"][1])
    if not fused:
        same_bits(h["o"], o_ref, "C4 o (all rows)")
    quant(o_ref, h["oq"], h["so"], "C4 o requant" + (" (fused in the GEMM)" if fused else ""))
    if glu:
        g_ref = oracle.epilogue(exact_acc(h["oq"], packed_ref["gate"][0]), "rowcol", h["so"], packed_ref["gate"][1])
        u_ref = oracle.epilogue(exact_acc(h["oq"], packed_ref["up"][0]), "rowcol", h["so"], packed_ref["up"][1])
        hh = oracle.silu_mul(g_ref, u_ref)
        same_bits(h["h"], hh, "C4 silu(gate)*up in the gate|up epilogue (all rows)")
    else:
        gu = np.concatenate([h["gate"], h["up"]], 1)
        linear(h["oq"], h["so"], "gate_up", gu, "C4 gate|up (all rows)")
        hh = oracle.silu_mul(h["gate"], h["up"])
    quant(hh, h["hq"], h["sh"], "C4 silu*up requant")
    linear(h["hq"], h["sh"], "down", h["down"], "C4 down (all rows)")
    # 8 tokens end to end from X
    rows = np.array([0, 1, 777, 1023, 1024, 1500, 2046, 2047])
    ref = OC.c4_expected_rows(inp, rows, packed_ref)
    for k in ("qkv", "down") + (("h",) if glu else ("gate", "up")):
        same_bits(h[k][rows], ref[k], f"C4 {k} end to end")
    so_ref = oracle.scales_per_token(ref["o"])
    same_bits(h["so"][rows], so_ref, "C4 o scales end to end")
    same_bits(h["oq"][rows], oracle.quantize_rows(ref["o"], so_ref), "C4 o codes end to end")


def test_c5_gemv(mods, oracle):
    C, O, OC = mods
    inp = OC.c5_inputs(with_quant_tensor=False)
    for n, W in inp["W"].items():
        Wq_ref, sW_ref = OC.pack_pc(W, 0)
        Wq, sW = O.pack_weight(dev(W), axis=0)
        same_bits(host(Wq), Wq_ref, f"C5 W{n}")
        for m, x in inp["x"].items():
            y = C.c5_gemv(dev(x), Wq, sW)
            same_bits(host(y), OC.qlinear_rows(x, Wq_ref, sW_ref), f"C5 gemv M={m} N={n}")


def test_c5_quant_dequant(mods, oracle):
    C, O, OC = mods
    X = OC.c5_inputs()["X"]
    q, s, y = C.c5_quant_dequant(dev(X))
    s_ref = oracle.scales_per_token(X)
    same_bits(host(s), s_ref, "C5 scales")
    q_ref = oracle.quantize_rows(X, s_ref)
    same_bits(host(q), q_ref, "C5 codes")
    same_bits(host(y), oracle.dequantize_rows(q_ref, s_ref), "C5 dequantized")


def test_device_inputs_match_oracle_stream(mods, oracle):
    """The device generator reproduces the config streams: uniforms exactly,
    normals to within one f32 ulp (device libm vs glibc in Box-Muller)."""
    C, O, OC = mods
    inp, _ = OC.c1()
    d = C.c1_inputs(DEV)
    same_bits(host(d["bias"]), inp["bias"], "C1 bias (uniform)")
    for k in ("X", "W"):
        a = host(d[k]).view(np.int32).astype(np.int64)
        b = inp[k].view(np.int32).astype(np.int64)
        assert np.abs(a - b).max() <= 1, k
    d3 = C.c3_inputs(DEV)
    r3 = OC.c3_inputs()
    for k in ("A", "B"):
        a = host(d3[k]).view(np.int32).astype(np.int64)
        b = r3[k].view(np.int32).astype(np.int64)
        diff = np.abs(a - b)
        assert diff.max() <= 1 and (diff != 0).mean() < 1e-3, k
