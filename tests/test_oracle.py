"""CPU checks that pin the oracle (oracle/q8ref.c) before it is trusted.

Three kinds of evidence, none of which retypes the oracle's own formulas:
  1. the reference's own known-answer tests, restated case by case
     (tests/compiler/passes/quantization/params.test.js, pass.test.js);
  2. closed forms and brute force: ECMA-262 Math.round on its defining
     cases, int64 brute-force dot products, ToInt32 wrap-around, absmax via
     numpy's NaN-aware reductions;
  3. a real JavaScript engine: oracle/q8ref.js builds kernels of the same
     source shape the reference's CPU backend emits and runs them under
     Node, so Math.round / Math.fround / `| 0` / typed-array stores are the
     engine's, not a restatement.  The C oracle must agree bit for bit.
"""
import json
import math
import os
import shutil
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
JS = os.path.join(ROOT, "oracle", "q8ref.js")
NODE = shutil.which("node")


def same_bits(a, b, what=""):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape and a.dtype == b.dtype, (what, a.shape, b.shape, a.dtype, b.dtype)
    av = a.view(np.uint8).reshape(-1, a.itemsize)
    bv = b.view(np.uint8).reshape(-1, b.itemsize)
    bad = np.nonzero(np.any(av != bv, axis=1))[0]
    assert bad.size == 0, (f"{what}: {bad.size} of {a.size} differ; first at {bad[0]}: "
                           f"{a.reshape(-1)[bad[0]]!r} vs {b.reshape(-1)[bad[0]]!r}")


# ---------------------------------------------------------------- params.test.js
class TestParamsKnownAnswers:
    """tests/compiler/passes/quantization/params.test.js, case by case."""

    def test_symmetric_scale(self, oracle):                      # :5-17
        assert oracle.scale_sym_from_range(-3, 3) == pytest.approx(3 / 127, abs=5e-11)
        assert oracle.scale_sym_from_range(-1, 5) == pytest.approx(5 / 127, abs=5e-11)

    def test_clamp_ranges(self, oracle):                         # :19-24, :35-40
        assert oracle.clamp_range(symmetric=True) == (-127, 127)
        assert oracle.clamp_range(symmetric=False, unsigned=True) == (0, 255)
        assert oracle.clamp_range(symmetric=False) == (-128, 127)
        assert oracle.clamp_range(symmetric=True, num_bits=4) == (-7, 7)

    def test_asymmetric(self, oracle):                           # :27-33
        s, zp = oracle.params_asym_from_range(0, 6)
        assert s == pytest.approx(6 / 255, abs=5e-11)
        assert -128 <= zp <= 127
        # closed form: zp = round(-128 - 0/s) = -128
        assert zp == -128

    def test_roundtrip_and_clamp(self, oracle):                  # :43-74
        s = oracle.scale_sym_from_range(-6, 6)
        q = oracle.weight_quantize_per_tensor(np.array([3.5], np.float32), s)[0]
        assert abs(int(q) * s - 3.5) < s
        s1 = oracle.scale_sym_from_range(-1, 1)
        q = oracle.weight_quantize_per_tensor(np.array([1000, -1000], np.float32), s1)
        assert q.tolist() == [127, -127]
        s10 = oracle.scale_sym_from_range(-10, 10)
        orig = np.array([1.5, -3.2, 0.0, 7.8], np.float32)
        q = oracle.weight_quantize_per_tensor(orig, s10)
        assert np.all(np.abs(q.astype(np.float64) * s10 - orig) < s10)
        s5 = oracle.scale_sym_from_range(-5, 5)
        assert oracle.weight_quantize_per_tensor(np.zeros(1, np.float32), s5)[0] == 0

    def test_from_constant_array(self, oracle):                  # :77-90
        assert oracle.scale_const_array(np.array([1.0, -2.0, 3.0, -0.5], np.float32)) == \
            pytest.approx(3 / 127, abs=5e-11)
        assert oracle.scale_const_array(np.array([5.0, 5.0, 5.0], np.float32)) == \
            pytest.approx(5.5 / 127, abs=5e-11)

    def test_per_channel_from_ranges(self, oracle):              # :93-115
        # fromRangePerChannel(mins=[-1,-2,-3], maxs=[1,2,3]) via a weight whose
        # channel c holds exactly {min_c, max_c}
        W = np.array([[-1, 1], [-2, 2], [-3, 3]], np.float32)
        s = oracle.scales_per_channel(W, axis=0)
        assert s == pytest.approx([1 / 127, 2 / 127, 3 / 127], abs=5e-11)

    def test_default_for_activation(self, oracle):               # :117-123
        assert oracle.scale_sym_from_range(-6, 6) == pytest.approx(6 / 127, abs=5e-11)

    def _skewed(self):                                           # :148-151
        K, N = 4, 3
        W = np.array([[math.sin(k * 1.7 + n) * (n + 1) * 3 for n in range(N)] for k in range(K)],
                     np.float32)
        return W

    def test_per_channel_axis1_and_axis0(self, oracle):          # :153-184
        W = self._skewed()
        s1 = oracle.scales_per_channel(W, axis=1)
        assert s1 == pytest.approx(np.abs(W).max(axis=0).astype(np.float64) / 127, abs=5e-11)
        q = oracle.weight_quantize_per_channel(W, 1, s1)
        d = q.astype(np.float64) * s1[None, :]
        assert np.all(np.abs(d - W) <= s1[None, :] / 2 + 1e-9)
        s0 = oracle.scales_per_channel(W, axis=0)
        assert s0 == pytest.approx(np.abs(W).max(axis=1).astype(np.float64) / 127, abs=5e-11)

    def test_per_channel_beats_per_tensor(self, oracle):         # :186-202
        W = self._skewed()
        spt = oracle.scale_const_array(W)
        ept = np.abs(oracle.weight_quantize_per_tensor(W, spt) * spt - W).mean()
        spc = oracle.scales_per_channel(W, axis=1)
        epc = np.abs(oracle.weight_quantize_per_channel(W, 1, spc) * spc[None, :] - W).mean()
        assert epc < ept and ept / epc > 1.5

    def test_int4_per_group(self, oracle):                       # :205-233
        N, G = 64, 16
        data = np.array([math.sin(i * 0.9) * (1 + (i % G) * 0.1) for i in range(N)], np.float32)
        s = oracle.scales_per_group(data, G, num_bits=4)
        assert s.size == math.ceil(N / G)
        q = oracle.weight_quantize_per_group(data, G, s, -7, 7)
        assert q.min() >= -7 and q.max() <= 7
        deq = q.astype(np.float64) * np.repeat(s, G)
        grp_err = np.abs(deq - data).max()
        assert grp_err <= s.max() / 2 + 1e-9
        spt = oracle.scale_const_array(data, num_bits=4)
        pt_err = np.abs(oracle.weight_quantize_per_tensor(data, spt, -7, 7) * spt - data).max()
        assert grp_err < pt_err


# ---------------------------------------------------------------- pass.test.js
def test_fake_quant_is_lossy_and_matches_host_math(oracle):      # pass.test.js:461-491
    s = oracle.scale_sym_from_range(-6, 6)
    data = np.array([3.5, -2.1, 5.9, 1.234, -5.9, 0.001], np.float32)
    out = oracle.dequantize(oracle.quantize(data, s), s)          # compiled R1 then D1
    host = oracle.weight_quantize_per_tensor(data, s).astype(np.float64) * s   # R2 + host dequant
    assert np.all(np.abs(out - host) < 1e-4)
    assert np.all(np.abs(out - data) <= s + 1e-6)
    assert np.any(np.abs(out - data) > 1e-6)


def test_per_channel_matmul_beats_per_tensor(oracle):            # pass.test.js:493-549
    M, K, N = 4, 8, 6
    A = np.array([math.sin(i * 0.7) for i in range(M * K)], np.float32).reshape(M, K)
    W = np.array([[math.sin(k * 1.3 + n) * (n + 1) * 2 for n in range(N)] for k in range(K)],
                 np.float32)
    ref = (A.astype(np.float64) @ W.astype(np.float64)).astype(np.float32)
    a_scale = float(np.abs(A).max()) / 127
    aq = oracle.quantize(A, a_scale)

    def run(per_channel):
        if per_channel:
            sw = oracle.scales_per_channel(W, axis=1)
            wq = oracle.weight_quantize_per_channel(W, 1, sw)
        else:
            s = oracle.scale_const_array(W)
            wq = oracle.weight_quantize_per_tensor(W, s)
            sw = np.full(N, s)
        acc = oracle.quantized_dot(aq, wq, b_layout=0)
        y = oracle.epilogue(acc, "rowcol", a_scale, sw)
        return np.abs(y - ref).mean()

    ept, epc = run(False), run(True)
    assert epc < ept and ept / epc > 1.5


# ---------------------------------------------------------------- closed forms
def test_js_round_defining_cases(oracle):
    """ECMA-262 Math.round: nearest, ties toward +inf, -0 for [-0.5, -0]."""
    cases = {0.5: 1.0, -0.5: -0.0, 1.5: 2.0, -1.5: -1.0, 2.5: 3.0, -2.5: -2.0,
             0.49999999999999994: 0.0, -0.49999999999999994: -0.0, 4503599627370495.5: 4503599627370496.0,
             -4503599627370495.5: -4503599627370495.0, 127.5: 128.0, -128.5: -128.0, 3.7: 4.0,
             -3.7: -4.0, 0.0: 0.0}
    for y, want in cases.items():
        got = oracle.js_round(y)
        assert got == want and math.copysign(1, got) == math.copysign(1, want), (y, got, want)
    assert math.isnan(oracle.js_round(float("nan")))
    assert oracle.js_round(float("inf")) == float("inf")


def test_quantize_edge_values(oracle):
    """R1 on the values whose JS behaviour is fixed by the spec."""
    x = np.array([np.nan, np.inf, -np.inf, -0.0, 0.5, -0.5, 1.5, -1.5, 127.49, 127.5, -128.5,
                  -128.51, 1e30, -1e30], np.float32)
    q = oracle.quantize(x, 1.0)
    assert q.tolist() == [0, 127, -128, 0, 1, 0, 2, -1, 127, 127, -128, -128, 127, -128]
    qu = oracle.quantize(x, 1.0, unsigned=True)
    assert qu.tolist() == [0, 255, 0, 0, 1, 0, 2, 0, 127, 128, 0, 0, 255, 0]


def test_quantize_rounds_fround_of_quotient(oracle):
    """fround(x/s) is taken before Math.round: x/s just below k+0.5 in f64
    that rounds up to k+0.5 in f32 quantizes to k+1 (the CPU backend's
    Math.fround(x / s)); the f64 quotient alone would give k."""
    s = 6 / 127
    x = np.float32(0.11811023205518723)        # x / s = 2.49999991.. in f64
    y64 = float(x) / s
    assert y64 < 2.5 and np.float32(y64) == np.float32(2.5)
    assert oracle.quantize(np.array([x]), s)[0] == 3
    assert oracle.quantize(np.array([-x]), s)[0] == -2          # tie toward +inf


def test_quantized_dot_brute_force(oracle):
    rng = np.random.default_rng(0)
    for M, N, K in [(1, 1, 1), (3, 5, 7), (16, 9, 64), (5, 4, 300)]:
        A = rng.integers(-128, 128, (M, K)).astype(np.int8)
        B = rng.integers(-128, 128, (N, K)).astype(np.int8)
        want = (A.astype(np.int64) @ B.astype(np.int64).T).astype(np.int32)
        same_bits(oracle.quantized_dot(A, B, b_layout=1), want)
        same_bits(oracle.quantized_dot(A, np.ascontiguousarray(B.T), b_layout=0), want)
        zpA, zpB = 3, -5
        want_zp = ((A.astype(np.int64) - zpA) @ (B.astype(np.int64) - zpB).T).astype(np.int32)
        same_bits(oracle.quantized_dot(A, B, 1, zpA, zpB), want_zp)


def test_quantized_dot_ui8_operands_and_zero_points(oracle):
    """ui8 operands are read as 0..255 (CastNode of a Uint8Array load,
    rules/quantization.ts:33-36; the verifier admits i8 and ui8,
    ops/quantization.ts:141-146); checked against an int64 brute force.  A
    mistake that reads ui8 bytes as signed, or drops a zero point, changes
    the result for bytes >= 128."""
    rng = np.random.default_rng(3)
    for M, N, K in [(1, 1, 1), (4, 6, 33), (7, 3, 128)]:
        for a_u8 in (False, True):
            for b_u8 in (False, True):
                A = rng.integers(0, 256, (M, K)).astype(np.uint8)
                B = rng.integers(0, 256, (N, K)).astype(np.uint8)
                A_ = A if a_u8 else A.view(np.int8)
                B_ = B if b_u8 else B.view(np.int8)
                for zpA, zpB in ((0, 0), (128, 0), (0, -7), (131, 255), (-128, 127)):
                    want = ((A_.astype(np.int64) - zpA) @ (B_.astype(np.int64) - zpB).T).astype(np.int32)
                    same_bits(oracle.quantized_dot(A_, B_, 1, zpA, zpB), want)
                    same_bits(oracle.quantized_dot(A_, np.ascontiguousarray(B_.T), 0, zpA, zpB), want)
    # the signed and unsigned readings of the same bytes differ
    A = np.full((1, 4), 200, np.uint8)
    B = np.ones((1, 4), np.int8)
    assert oracle.quantized_dot(A, B)[0, 0] == 800
    assert oracle.quantized_dot(A.view(np.int8), B)[0, 0] == -224


def test_quantized_dot_int32_wrap(oracle):
    """The JS double accumulator is exact; the Int32Array store wraps mod 2^32."""
    K = 1 << 17
    A = np.full((1, K), -128, np.int8)
    B = np.full((2, K), -128, np.int8)
    B[1] = 127
    acc = oracle.quantized_dot(A, B, b_layout=1)
    assert acc[0, 0] == np.int32(np.int64(K * 16384) - (1 << 32))      # 2^31 wraps to -2^31
    assert acc[0, 1] == -128 * 127 * K


def _conv_windows(x, w, strides, padding, dilation, groups, zpx=0, zpw=0):
    """Independent formulation of the convolution: pad the input with zpx
    (so padded taps contribute (zpx - zpx) * (w - zpw) = 0), take strided
    windows per kernel position and contract with numpy in int64."""
    import itertools
    N, C = x.shape[:2]
    O, Cg = w.shape[:2]
    d = len(strides)
    pad = [(0, 0), (0, 0)] + [tuple(p) for p in padding]
    xp = np.pad(x.astype(np.int64) - zpx, pad)            # padding = 0 after the shift
    wz = w.astype(np.int64) - zpw
    out_sp = [(xp.shape[2 + i] - ((w.shape[2 + i] - 1) * dilation[i] + 1)) // strides[i] + 1
              for i in range(d)]
    out = np.zeros([N, O] + out_sp, np.int64)
    Og = O // groups
    for kk in itertools.product(*[range(w.shape[2 + i]) for i in range(d)]):
        sl = tuple(slice(kk[i] * dilation[i], kk[i] * dilation[i] + (out_sp[i] - 1) * strides[i] + 1,
                         strides[i]) for i in range(d))
        for g in range(groups):
            xs = xp[(slice(None), slice(g * Cg, (g + 1) * Cg)) + sl]
            ws = wz[(slice(g * Og, (g + 1) * Og), slice(None)) + tuple(kk)]
            out[:, g * Og:(g + 1) * Og] += np.einsum("nc...,oc->no...", xs, ws)
    return out.astype(np.int32)


def test_conv_ui8_operands_and_zero_points(oracle):
    """ui8 inputs / kernels read as 0..255, with zero points, against the
    independent windowed formulation (which pads with zpx, so a padded tap
    adds 0)."""
    rng = np.random.default_rng(5)
    for xs, ws, st, pad, dl, g in [((2, 4, 9, 7), (6, 2, 3, 2), [2, 1], [[1, 2], [0, 1]], [2, 1], 2),
                                   ((1, 3, 8), (4, 3, 3), [1], [[2, 1]], [1], 1)]:
        for x_u8 in (False, True):
            for w_u8 in (False, True):
                x = rng.integers(0, 256, xs).astype(np.uint8)
                w = rng.integers(0, 256, ws).astype(np.uint8)
                x = x if x_u8 else x.view(np.int8)
                w = w if w_u8 else w.view(np.int8)
                for zpx, zpw in ((0, 0), (128, 0), (5, 130)):
                    want = _conv_windows(x, w, st, pad, dl, g, zpx, zpw)
                    same_bits(oracle.quantized_conv(x, w, st, pad, dl, g, zpx, zpw), want)


CONV_CASES = [
    # x shape, w shape, strides, padding, dilation, groups
    ((1, 3, 8, 8), (16, 3, 3, 3), [1, 1], [[0, 0], [0, 0]], [1, 1], 1),   # pass.test.js:255-274
    ((1, 3, 8, 8), (16, 3, 3, 3), [2, 2], [[1, 1], [1, 1]], [1, 1], 1),   # pass.test.js:308-320
    ((2, 4, 9, 7), (6, 2, 3, 2), [2, 1], [[1, 2], [0, 1]], [2, 1], 2),
    ((1, 6, 10), (6, 1, 3), [1], [[1, 1]], [2], 6),                       # depthwise 1-D
    ((1, 2, 5, 6, 4), (3, 2, 2, 3, 2), [1, 2, 1], [[1, 0], [0, 1], [1, 1]], [1, 1, 2], 1),
]


@pytest.mark.parametrize("case", CONV_CASES)
def test_quantized_conv_matches_window_formulation(oracle, case):
    xs, ws, st, pd, dl, g = case
    rng = np.random.default_rng(len(xs) * 7 + g)
    x = rng.integers(-128, 128, xs).astype(np.int8)
    w = rng.integers(-128, 128, ws).astype(np.int8)
    same_bits(oracle.quantized_conv(x, w, st, pd, dl, g), _conv_windows(x, w, st, pd, dl, g))
    # zero points: a padded tap adds 0, not (0 - zpx) * (w - zpw)
    same_bits(oracle.quantized_conv(x, w, st, pd, dl, g, zpx=3, zpw=-2),
              _conv_windows(x, w, st, pd, dl, g, zpx=3, zpw=-2))


def test_quantized_conv_counts_valid_taps(oracle):
    """(x - zpx) = (w - zpw) = 1 everywhere: every output is the number of
    taps whose input coordinate is inside the image, a closed form."""
    x = np.full((1, 2, 5, 4), 4, np.int8)
    w = np.full((3, 2, 3, 2), -1, np.int8)
    out = oracle.quantized_conv(x, w, [1, 1], [[1, 1], [0, 1]], [1, 1], 1, zpx=3, zpw=-2)
    for oh in range(out.shape[2]):
        for ow in range(out.shape[3]):
            rows = sum(1 for kh in range(3) if 0 <= oh + kh - 1 < 5)
            cols = sum(1 for kw in range(2) if 0 <= ow + kw < 4)
            assert (out[0, :, oh, ow] == 2 * rows * cols).all()


def test_quantized_conv_1x1_is_a_matmul(oracle):
    """A 1x1 stride-1 conv is quantized_dot of the [C, H*W] image with the
    [O, C] weight (the brute-forced M1 above)."""
    rng = np.random.default_rng(5)
    x = rng.integers(-128, 128, (1, 40, 3, 5)).astype(np.int8)
    w = rng.integers(-128, 128, (24, 40, 1, 1)).astype(np.int8)
    out = oracle.quantized_conv(x, w, [1, 1], [[0, 0], [0, 0]], [1, 1], 1)
    mat = oracle.quantized_dot(np.ascontiguousarray(w.reshape(24, 40)),
                               np.ascontiguousarray(x.reshape(40, 15).T), b_layout=1)
    same_bits(out.reshape(24, 15), mat)


def test_scales_per_token_closed_form(oracle):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((6, 33)).astype(np.float32)
    x[1, 3] = np.nan
    x[2] = 0.0
    x[3] = np.nan
    x[4, 0] = -np.inf
    want = np.nanmax(np.abs(x.astype(np.float64)), axis=1, initial=0.0) / 127
    want[2] = 1e-10                      # absmax 0 -> `|| 1e-10`
    want[3] = np.inf                     # only NaN: observer stays (+inf, -inf)
    same_bits(oracle.scales_per_token(x), want)


# ---------------------------------------------------------------- JS engine
needs_node = pytest.mark.skipif(NODE is None, reason="node is not installed")


def run_js(tmp_path, cmd, params, ins, out_specs):
    """Run oracle/q8ref.js: inputs are numpy arrays, outputs (name, dtype, shape)."""
    in_files = []
    for i, a in enumerate(ins):
        f = tmp_path / f"in{i}.bin"
        np.ascontiguousarray(a).tofile(f)
        in_files.append(str(f))
    out_files = [str(tmp_path / f"out{i}.bin") for i in range(len(out_specs))]
    subprocess.run([NODE, JS, cmd, json.dumps(params), *in_files, "--", *out_files],
                   check=True, timeout=120)
    return [np.fromfile(f, dtype=dt).reshape(shape) for f, (dt, shape) in zip(out_files, out_specs)]


def edge_floats(oracle, n=4096, seed=3):
    x = oracle.Rng(seed).normal((n,), 0.0, 3.0)
    special = [np.nan, np.inf, -np.inf, -0.0, 0.0, 0.5, -0.5, 2.5, -2.5, 1e-40, -1e-40,
               3.4e38, -3.4e38, 127.5, -128.5, 0.001]
    x[:len(special)] = special
    return x.astype(np.float32)


@needs_node
def test_js_rng_matches(oracle, tmp_path):
    (draws,) = run_js(tmp_path, "rng", {"seed": 0x9E3779B9, "n": 5000}, [], [(np.float64, (5000,))])
    r = oracle.Rng(0x9E3779B9)
    same_bits(np.array([r.next() for _ in range(5000)]), draws, "mulberry32")
    (u,) = run_js(tmp_path, "uniform", {"seed": 7, "n": 1001, "a": -0.1, "b": 0.1}, [],
                  [(np.float32, (1001,))])
    same_bits(oracle.Rng(7).uniform((1001,), -0.1, 0.1), u, "uniform_")


@needs_node
def test_js_normal_matches_within_libm(oracle, tmp_path):
    """Box-Muller goes through log/cos/sin: V8's and glibc's may differ in the
    last f64 bit, so a few f32 values may differ by one ulp."""
    (y,) = run_js(tmp_path, "normal", {"seed": 5, "n": 20001, "mean": 0.0, "std": 0.02}, [],
                  [(np.float32, (20001,))])
    x = oracle.Rng(5).normal((20001,), 0.0, 0.02)
    d = np.abs(x.view(np.int32).astype(np.int64) - y.view(np.int32).astype(np.int64))
    assert d.max() <= 1 and (d != 0).mean() < 1e-3


@needs_node
@pytest.mark.parametrize("scale,zp,unsigned", [(6 / 127, 0.0, False), (0.0123, 0.0, False),
                                               (6 / 255, -128.0, False), (1 / 255, 0.0, True),
                                               (6 / 255, 3.0, True), (1e-10, 0.0, False),
                                               (1.0, 0.0, False), (3.0, 0.0, False)])
def test_js_quantize_matches(oracle, tmp_path, scale, zp, unsigned):
    x = edge_floats(oracle)
    (q,) = run_js(tmp_path, "quantize", {"scale": scale, "zero_point": zp, "unsigned": unsigned},
                  [x], [(np.uint8 if unsigned else np.int8, x.shape)])
    same_bits(oracle.quantize(x, scale, zp, unsigned), q, "R1")


@needs_node
def test_js_scales_per_token_matches(oracle, tmp_path):
    x = edge_floats(oracle, 64 * 128, seed=6).reshape(64, 128)
    x[5] = 0.0                       # all zeros: 1e-10
    x[6] = np.nan                    # no value ever compares: +-inf range, absmax inf
    x[7, :64] = np.nan
    x[9] = -0.0
    (s,) = run_js(tmp_path, "scales_rows", {"M": 64, "K": 128}, [x], [(np.float64, (64,))])
    same_bits(oracle.scales_per_token(x), s, "S-token")
    (s0,) = run_js(tmp_path, "scales_rows", {"M": 3, "K": 0}, [np.zeros(0, np.float32)], [(np.float64, (3,))])
    same_bits(oracle.scales_per_token(np.zeros((3, 0), np.float32)), s0, "S-token, empty rows")


@needs_node
def test_js_quantize_rows_matches(oracle, tmp_path):
    x = edge_floats(oracle, 64 * 128, seed=4).reshape(64, 128)
    x[5] = 0.0
    s = oracle.scales_per_token(x)
    (q,) = run_js(tmp_path, "quantize_rows", {"M": 64, "K": 128}, [x, s], [(np.int8, x.shape)])
    same_bits(oracle.quantize_rows(x, s), q, "R1 per-token")


@needs_node
@pytest.mark.parametrize("src,zp", [("i8", 0.0), ("i8", 5.0), ("u8", 128.0), ("i32", 0.0),
                                    ("i32", -7.0)])
def test_js_dequantize_matches(oracle, tmp_path, src, zp):
    rng = np.random.default_rng(2)
    dt = {"i8": np.int8, "u8": np.uint8, "i32": np.int32}[src]
    info = np.iinfo(dt)
    q = rng.integers(info.min, info.max, 3000, dtype=np.int64, endpoint=True).astype(dt)
    for s in (6 / 127, 0.0012345678901234, 2.3e-6):
        (y,) = run_js(tmp_path, "dequantize", {"src": src, "scale": s, "zero_point": zp}, [q],
                      [(np.float32, q.shape)])
        same_bits(oracle.dequantize(q, s, zp), y, "D1")


@needs_node
@pytest.mark.parametrize("b_layout,zpA,zpB", [(1, 0, 0), (0, 0, 0), (1, 2, -3)])
def test_js_quantized_dot_matches(oracle, tmp_path, b_layout, zpA, zpB):
    rng = np.random.default_rng(4)
    M, N, K = 9, 13, 200
    A = rng.integers(-128, 128, (M, K)).astype(np.int8)
    B = rng.integers(-128, 128, (N, K) if b_layout else (K, N)).astype(np.int8)
    (acc,) = run_js(tmp_path, "qdot", {"M": M, "N": N, "K": K, "b_layout": b_layout,
                                       "zpA": zpA, "zpB": zpB}, [A, B], [(np.int32, (M, N))])
    same_bits(oracle.quantized_dot(A, B, b_layout, zpA, zpB), acc, "M1")


@needs_node
@pytest.mark.parametrize("with_bias,relu", [(False, False), (True, False), (True, True)])
def test_js_epilogue_matches(oracle, tmp_path, with_bias, relu):
    rng = np.random.default_rng(5)
    M, N = 17, 40
    acc = rng.integers(-3_000_000, 3_000_000, (M, N)).astype(np.int32)
    acc[0, :4] = [0, 1 << 24, -(1 << 30), (1 << 31) - 1]
    sa = 0.0173
    sw = oracle.Rng(6).uniform((N,), 1e-5, 1e-3).astype(np.float64)
    sv = (sa * sw).astype(np.float32)                  # the F32 scale constant
    bias = oracle.Rng(8).uniform((N,), -0.1, 0.1)
    ins = [acc, sv] + ([bias] if with_bias else [])
    (y,) = run_js(tmp_path, "epilogue_pc", {"M": M, "N": N, "relu": relu}, ins,
                  [(np.float32, (M, N))])
    want = oracle.epilogue(acc, "rowcol", sa, sw, bias=bias if with_bias else None,
                           act="relu" if relu else "none")
    same_bits(want, y, "E-pc")


@needs_node
def test_js_silu_mul_matches(oracle, tmp_path):
    g = oracle.Rng(9).normal((5000,), 0.0, 4.0)
    g[:6] = [0.0, -0.0, 88.0, -104.0, 1e-30, -20.0]
    u = oracle.Rng(10).normal((5000,))
    (h,) = run_js(tmp_path, "silu_mul", {}, [g, u], [(np.float32, g.shape)])
    # exp goes through V8's and glibc's libm: allow the last f32 ulp
    got = oracle.silu_mul(g, u)
    d = np.abs(got.view(np.int32).astype(np.int64) - h.view(np.int32).astype(np.int64))
    assert d.max() <= 1 and (d != 0).mean() < 1e-3


def test_gemv_w4_matches_independent_evaluation(oracle):
    """The W4A8 per-group GEMV (a composition defined in oracle/q8ref.h; the
    reference has no such op) evaluated independently: nibbles unpacked with
    numpy, per-group int64 sums by einsum, the f64 sum over groups by a Python
    loop in ascending order, one binary32 rounding at the end."""
    from mlfw_amd.checkpoint import pack_int4
    rng = np.random.default_rng(9)
    for M, N, K, g in [(1, 5, 64, 32), (3, 7, 256, 64), (4, 3, 96, 32), (2, 4, 128, 128)]:
        xq = rng.integers(-128, 128, (M, K)).astype(np.int8)
        q = rng.integers(-8, 8, (N, K)).astype(np.int8)
        G = K // g
        sw = rng.random(N * G) * 1e-2 + 1e-6
        sx = rng.random(M) * 1e-1 + 1e-4
        got = oracle.gemv_w4(xq, sx, pack_int4(q), sw, K, g)
        parts = np.einsum("mgk,ngk->mng", xq.astype(np.int64).reshape(M, G, g),
                          q.astype(np.int64).reshape(N, G, g))
        want = np.empty((M, N), np.float32)
        for m in range(M):
            for n in range(N):
                S = float(parts[m, n, 0]) * sw[n * G]
                for gi in range(1, G):
                    S = S + float(parts[m, n, gi]) * sw[n * G + gi]
                want[m, n] = np.float32(S * sx[m])
        same_bits(got, want)


# The oracle's SiLU (glibc exp) against V8's on whole chunks of 2^24 inputs:
# the chunks where 1 / (1 + exp(-x)) is neither 0, 1/2 nor 1 in f32 (|x|
# from ~1e-4 to ~100, both signs), the zero / subnormal chunks and the
# chunks holding the infinities and NaNs.  The hashes are those of
# tests/golden/silu_v8_hashes.json (see silu_v8_hashes.js).
SILU_CHUNKS = [0, 1] + list(range(56, 68)) + [127, 128, 129] + list(range(184, 196)) + [255]


def test_oracle_silu_equals_v8_on_whole_chunks(oracle):
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "silu_v8_hashes.json")) as f:
        golden = json.load(f)["hashes"]
    n = 1 << 24
    w = 2 * np.arange(n, dtype=np.uint64) + 1
    ones = np.ones(n, np.float32)
    for c in SILU_CHUNKS:
        x = (np.arange(n, dtype=np.uint64) + np.uint64(c * n)).astype(np.uint32).view(np.float32)
        h = oracle.silu_mul(x, ones)
        v = h.view(np.uint32).astype(np.uint64)
        v[np.isnan(h)] = 0x7FC00000
        v ^= v >> np.uint64(16)
        v = (v * np.uint64(0x7FEB352D)) & np.uint64(0xFFFFFFFF)
        v ^= v >> np.uint64(15)
        s1 = int(((v * w) & np.uint64(0xFFFFFFFF)).sum()) & 0xFFFFFFFF
        s2 = int(v.sum()) & 0xFFFFFFFF
        assert [s1, s2] == golden[c], f"chunk {c}"


def _chunk_hash_np(h, w):
    v = h.view(np.uint32).astype(np.uint64)
    v[np.isnan(h)] = 0x7FC00000
    v ^= v >> np.uint64(16)
    v = (v * np.uint64(0x7FEB352D)) & np.uint64(0xFFFFFFFF)
    v ^= v >> np.uint64(15)
    return [int(((v * w) & np.uint64(0xFFFFFFFF)).sum()) & 0xFFFFFFFF, int(v.sum()) & 0xFFFFFFFF]


def test_ewise_v8_hashes_on_chunks_with_closed_forms():
    """tests/golden/ewise_v8_hashes.json (V8's Math.fround(Math.exp / log /
    tanh (x)) per chunk of 2^24 bit patterns) against results fixed by the
    mathematics, so the file and its hash definition are pinned without an
    engine.  Chunk 0 (+0, the subnormals and normals below 2^-103): exp(x)
    rounds to 1 and tanh(x) to x.  Chunk 255 (bits 0xff000000..): the
    negative finite values of exponent 254 and -Inf give exp = +0,
    tanh = -1 and log = NaN, the patterns after -Inf are NaN for all three."""
    import json
    import os
    with open(os.path.join(os.path.dirname(__file__), "golden", "ewise_v8_hashes.json")) as f:
        golden = json.load(f)
    n = 1 << 24
    w = 2 * np.arange(n, dtype=np.uint64) + 1
    x0 = np.arange(n, dtype=np.uint32).view(np.float32)
    assert _chunk_hash_np(np.ones(n, np.float32), w) == golden["exp"][0]
    assert _chunk_hash_np(x0.copy(), w) == golden["tanh"][0]
    finite_and_inf = 0x800001                       # 0xff000000 .. 0xff800000 (-Inf)
    want = {"exp": 0.0, "log": np.nan, "tanh": -1.0}
    for fn, v in want.items():
        h = np.full(n, np.nan, np.float32)
        h[:finite_and_inf] = v
        assert _chunk_hash_np(h, w) == golden[fn][255], fn
