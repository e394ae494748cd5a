"""numpy front end of the C oracle (oracle/q8ref.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker and by bench.py's cpu_baseline leg.  The product (mlfw_amd/)
never imports it.

Each function forwards to the C restatement of one reference function; the
docstrings name the reference file:line they follow.  `build()` compiles the
library with oracle/Makefile when it is missing.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq8ref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_i64 = C.c_int64
_dbl = C.c_double
_int = C.c_int


class _Rng(C.Structure):
    _fields_ = [("a", C.c_uint32)]


class _Observer(C.Structure):
    _fields_ = [("min", C.c_double), ("max", C.c_double), ("count", C.c_double),
                ("has_hist", C.c_int), ("num_bins", C.c_int), ("initialized", C.c_int),
                ("range_min", C.c_double), ("range_max", C.c_double),
                ("total_count", C.c_double), ("bins", C.POINTER(C.c_double))]


def build(force: bool = False) -> str:
    # make rebuilds only when q8ref.c / q8ref.h are newer than the library
    subprocess.run(["make", "-s"] + (["-B"] if force else []) + ["-C", HERE],
                   check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    build()
    L = C.CDLL(LIB_PATH)
    sig = {
        "q8r_rng_seed": (None, [C.POINTER(_Rng), C.c_uint32]),
        "q8r_rng_next": (_dbl, [C.POINTER(_Rng)]),
        "q8r_fill_normal": (None, [C.POINTER(_Rng), _f32p, _i64, _dbl, _dbl]),
        "q8r_fill_uniform": (None, [C.POINTER(_Rng), _f32p, _i64, _dbl, _dbl]),
        "q8r_apply_outliers": (None, [_f32p, _i64, C.c_uint32, _dbl, _dbl]),
        "q8r_scale_sym_from_range": (_dbl, [_dbl, _dbl, _int]),
        "q8r_params_asym_from_range": (None, [_dbl, _dbl, _int, _int, C.POINTER(_dbl), C.POINTER(_dbl)]),
        "q8r_observe_minmax": (None, [_f32p, _i64, C.POINTER(_dbl), C.POINTER(_dbl)]),
        "q8r_scale_const_array": (_dbl, [_f32p, _i64, _int]),
        "q8r_scales_per_channel": (None, [_f32p, _i64, _i64, _int, _int, _f64p]),
        "q8r_scales_per_group": (None, [_f32p, _i64, _i64, _int, _f64p]),
        "q8r_scales_per_token": (None, [_f32p, _i64, _i64, _f64p]),
        "q8r_scale_per_tensor_dynamic": (_dbl, [_f32p, _i64]),
        "q8r_js_round": (_dbl, [_dbl]),
        "q8r_fround": (C.c_float, [_dbl]),
        "q8r_quantize_value": (_int, [C.c_float, _dbl, _dbl, _int]),
        "q8r_quantize": (None, [_f32p, _i64, _dbl, _dbl, _int, C.c_void_p]),
        "q8r_quantize_rows": (None, [_f32p, _i64, _i64, _f64p, _i8p]),
        "q8r_weight_quantize_value": (_int, [_dbl, _dbl, _dbl, _int, _int]),
        "q8r_clamp_range": (None, [_int, _int, _int, C.POINTER(_int), C.POINTER(_int)]),
        "q8r_weight_quantize_per_channel": (None, [_f32p, _i64, _i64, _int, _f64p, _i8p]),
        "q8r_weight_quantize_per_tensor": (None, [_f32p, _i64, _dbl, _int, _int, _i8p]),
        "q8r_weight_quantize_per_group": (None, [_f32p, _i64, _i64, _f64p, _int, _int, _i8p]),
        "q8r_dequantize_value": (C.c_float, [_dbl, _dbl, _dbl]),
        "q8r_dequantize_i8": (None, [_i8p, _i64, _dbl, _dbl, _f32p]),
        "q8r_dequantize_u8": (None, [_u8p, _i64, _dbl, _dbl, _f32p]),
        "q8r_dequantize_i32": (None, [_i32p, _i64, _dbl, _dbl, _f32p]),
        "q8r_dequantize_rows_i8": (None, [_i8p, _i64, _i64, _f64p, _f32p]),
        "q8r_quantized_dot": (None, [_i8p, _i8p, _i64, _i64, _i64, _int, C.c_int32, C.c_int32, _i32p]),
        "q8r_quantized_dot_ex": (None, [_i8p, _int, _i8p, _int, _i64, _i64, _i64, _int, C.c_int32,
                                        C.c_int32, _i32p]),
        "q8r_quantized_conv": (None, [_i8p, _i8p, _int, _i64p, _i64p, _i64p, _i64p, _i64p, _i64p,
                                      _i64, C.c_int32, C.c_int32, _i32p]),
        "q8r_quantized_conv_ex": (None, [_i8p, _int, _i8p, _int, _int, _i64p, _i64p, _i64p, _i64p, _i64p,
                                         _i64p, _i64, C.c_int32, C.c_int32, _i32p]),
        "q8r_gemv_w4": (None, [_i8p, _f64p, _i64, _u8p, _f64p, _i64, _i64, _i64, _i64, C.c_void_p,
                               _int, _f32p]),
        "q8r_epilogue": (None, [_i32p, _i64, _i64, _int, _f64p, _i64, _f64p, _i64, _dbl,
                                C.c_void_p, _int, _f32p]),
        "q8r_relu": (C.c_float, [C.c_float]),
        "q8r_silu": (C.c_float, [C.c_float]),
        "q8r_mul": (C.c_float, [C.c_float, C.c_float]),
        "q8r_silu_mul": (None, [_f32p, _f32p, _i64, _f32p]),
        "q8r_observer_init": (None, [C.POINTER(_Observer), C.POINTER(C.c_double), _int, _int]),
        "q8r_observer_update": (None, [C.POINTER(_Observer), _f32p, _i64]),
        "q8r_hist_percentile": (_dbl, [C.POINTER(_Observer), _dbl]),
        "q8r_hist_entropy": (_dbl, [C.POINTER(_Observer), _int]),
        "q8r_calib_params": (_int, [C.POINTER(_Observer), _int, _int, _int, C.POINTER(_dbl),
                                    C.POINTER(_dbl)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---------------------------------------------------------------- inputs
class Rng:
    """mulberry32 stream (src/util/random.ts:5-14), consumed in order."""

    def __init__(self, seed: int):
        self._s = _Rng()
        lib().q8r_rng_seed(C.byref(self._s), seed & 0xFFFFFFFF)

    @property
    def state(self) -> int:
        return int(self._s.a)

    def skip(self, n: int) -> None:
        """Advance by n draws (the state moves by n * 0x6D2B79F5)."""
        self._s.a = (self._s.a + n * 0x6D2B79F5) & 0xFFFFFFFF

    def next(self) -> float:
        return lib().q8r_rng_next(C.byref(self._s))

    def normal(self, shape, mean=0.0, std=1.0) -> np.ndarray:
        """normal_ (src/nn/init.ts:40-52)."""
        out = np.empty(shape, np.float32)
        lib().q8r_fill_normal(C.byref(self._s), out.reshape(-1), out.size, mean, std)
        return out

    def uniform(self, shape, a=0.0, b=1.0) -> np.ndarray:
        """uniform_ (src/nn/init.ts:31-37)."""
        out = np.empty(shape, np.float32)
        lib().q8r_fill_uniform(C.byref(self._s), out.reshape(-1), out.size, a, b)
        return out


def apply_outliers(x: np.ndarray, seed: int, p: float = 0.01, factor: float = 50.0) -> None:
    """In place: C5 outlier protocol (second mulberry32 stream)."""
    assert x.dtype == np.float32 and x.flags.c_contiguous
    lib().q8r_apply_outliers(x.reshape(-1), x.size, seed & 0xFFFFFFFF, p, factor)


# ---------------------------------------------------------------- scales
def scale_sym_from_range(mn, mx, num_bits=8) -> float:
    """QuantizationParams.fromRange(.., PER_TENSOR_SYMMETRIC) (quantization_types.ts:248-254)."""
    return lib().q8r_scale_sym_from_range(mn, mx, num_bits)


def params_asym_from_range(mn, mx, unsigned=False, num_bits=8):
    """fromRange asymmetric (quantization_types.ts:256-263) -> (scale, zero_point)."""
    s, z = _dbl(), _dbl()
    lib().q8r_params_asym_from_range(mn, mx, int(unsigned), num_bits, C.byref(s), C.byref(z))
    return s.value, z.value


def observe_minmax(x):
    """ValueObserver.update (calibration.ts:24-34)."""
    x = _c(x, np.float32).reshape(-1)
    mn, mx = _dbl(), _dbl()
    lib().q8r_observe_minmax(x, x.size, C.byref(mn), C.byref(mx))
    return mn.value, mx.value


def scale_const_array(x, num_bits=8) -> float:
    """fromConstantArray, symmetric (quantization_types.ts:287-297)."""
    x = _c(x, np.float32).reshape(-1)
    return lib().q8r_scale_const_array(x, x.size, num_bits)


def scales_per_channel(w, axis, num_bits=8) -> np.ndarray:
    """fromConstantArrayPerChannel for a 2-D weight (quantization_types.ts:299-317)."""
    w = _c(w, np.float32)
    rows, cols = w.shape
    out = np.empty(rows if axis == 0 else cols, np.float64)
    lib().q8r_scales_per_channel(w.reshape(-1), rows, cols, axis, num_bits, out)
    return out


def scales_per_group(x, group, num_bits=4) -> np.ndarray:
    """fromConstantArrayPerGroup (quantization_types.ts:319-340)."""
    x = _c(x, np.float32).reshape(-1)
    out = np.empty((x.size + group - 1) // group, np.float64)
    lib().q8r_scales_per_group(x, x.size, group, num_bits, out)
    return out


def scales_per_token(x) -> np.ndarray:
    """Per-row ValueObserver + fromRange(SYMMETRIC); empty rows -> 6/127."""
    x = _c(x, np.float32)
    M, K = x.shape
    out = np.empty(M, np.float64)
    lib().q8r_scales_per_token(x.reshape(-1), M, K, out)
    return out


def scale_per_tensor(x) -> float:
    x = _c(x, np.float32).reshape(-1)
    return lib().q8r_scale_per_tensor_dynamic(x, x.size)


# ---------------------------------------------------------------- R1 / R2 / D1
def js_round(y: float) -> float:
    return lib().q8r_js_round(y)


def quantize(x, scale, zero_point=0.0, unsigned=False) -> np.ndarray:
    """Compiled quantize (quant_math.ts:16-27)."""
    x = _c(x, np.float32)
    q = np.empty(x.shape, np.uint8 if unsigned else np.int8)
    lib().q8r_quantize(x.reshape(-1), x.size, scale, zero_point, int(unsigned),
                       q.ctypes.data_as(C.c_void_p))
    return q


def quantize_rows(x, scales) -> np.ndarray:
    x = _c(x, np.float32)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    lib().q8r_quantize_rows(x.reshape(-1), M, K, _c(scales, np.float64), q.reshape(-1))
    return q


def clamp_range(symmetric, unsigned=False, num_bits=8):
    """QuantizationParams.clampRange (quantization_types.ts:62-73)."""
    lo, hi = _int(), _int()
    lib().q8r_clamp_range(int(symmetric), int(unsigned), num_bits, C.byref(lo), C.byref(hi))
    return lo.value, hi.value


def weight_quantize_per_channel(w, axis, scales) -> np.ndarray:
    """quantizeArrayPerChannel (quantization_types.ts:118-130)."""
    w = _c(w, np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    lib().q8r_weight_quantize_per_channel(w.reshape(-1), rows, cols, axis,
                                          _c(scales, np.float64), q.reshape(-1))
    return q


def weight_quantize_per_tensor(w, scale, lo=-127, hi=127) -> np.ndarray:
    """quantizeArray (quantization_types.ts:85-97)."""
    w = _c(w, np.float32)
    q = np.empty(w.shape, np.int8)
    lib().q8r_weight_quantize_per_tensor(w.reshape(-1), w.size, scale, lo, hi, q.reshape(-1))
    return q


def weight_quantize_per_group(w, group, scales, lo=-7, hi=7) -> np.ndarray:
    """quantizeArrayPerGroup (quantization_types.ts:143-153)."""
    w = _c(w, np.float32).reshape(-1)
    q = np.empty(w.size, np.int8)
    lib().q8r_weight_quantize_per_group(w, w.size, group, _c(scales, np.float64), lo, hi, q)
    return q


def dequantize(q, scale, zero_point=0.0) -> np.ndarray:
    """Compiled dequantize (quant_math.ts:29-34) for i8 / u8 / i32 inputs."""
    y = np.empty(q.shape, np.float32)
    if q.dtype == np.int8:
        lib().q8r_dequantize_i8(_c(q, np.int8).reshape(-1), q.size, scale, zero_point, y.reshape(-1))
    elif q.dtype == np.uint8:
        lib().q8r_dequantize_u8(_c(q, np.uint8).reshape(-1), q.size, scale, zero_point, y.reshape(-1))
    elif q.dtype == np.int32:
        lib().q8r_dequantize_i32(_c(q, np.int32).reshape(-1), q.size, scale, zero_point, y.reshape(-1))
    else:
        raise TypeError(q.dtype)
    return y


def dequantize_rows(q, scales) -> np.ndarray:
    q = _c(q, np.int8)
    M, K = q.shape
    y = np.empty((M, K), np.float32)
    lib().q8r_dequantize_rows_i8(q.reshape(-1), M, K, _c(scales, np.float64), y.reshape(-1))
    return y


# ---------------------------------------------------------------- M1 + epilogue
def quantized_dot(A, B, b_layout=1, zpA=0, zpB=0) -> np.ndarray:
    """quantized_dot (rules/quantization.ts:57-76).  b_layout 1: B is [N,K].
    A uint8 operand is read as ui8 (0..255), an int8 one as i8."""
    a_u8 = np.asarray(A).dtype == np.uint8
    b_u8 = np.asarray(B).dtype == np.uint8
    A = _c(np.asarray(A).view(np.int8) if a_u8 else A, np.int8)
    B = _c(np.asarray(B).view(np.int8) if b_u8 else B, np.int8)
    M, K = A.shape
    N = B.shape[1] if b_layout == 0 else B.shape[0]
    acc = np.empty((M, N), np.int32)
    lib().q8r_quantized_dot_ex(A.reshape(-1), int(a_u8), B.reshape(-1), int(b_u8), M, N, K, b_layout,
                               zpA, zpB, acc.reshape(-1))
    return acc


def conv_out_shape(x_shape, w_shape, strides, padding, dilation):
    """inferConvResultTypes (src/compiler/ir/graph/ops/linalg.ts:222-248):
    [N, O, P_0..]; padding is a list of [lo, hi] pairs."""
    out = [int(x_shape[0]), int(w_shape[0])]
    for i in range(len(strides)):
        eff = (int(w_shape[2 + i]) - 1) * dilation[i] + 1
        out.append((int(x_shape[2 + i]) + padding[i][0] + padding[i][1] - eff) // strides[i] + 1)
    return out


def quantized_conv(x, w, strides, padding, dilation=None, groups=1, zpx=0, zpw=0) -> np.ndarray:
    """quantized_conv with NC(spatial) input / OI(spatial) kernel, int32 out
    (ops/quantization.ts:156-190, buildConvNest lowering_registry.ts:335-449).
    A uint8 operand is read as ui8 (0..255), an int8 one as i8."""
    x_u8 = np.asarray(x).dtype == np.uint8
    w_u8 = np.asarray(w).dtype == np.uint8
    x = _c(np.asarray(x).view(np.int8) if x_u8 else x, np.int8)
    w = _c(np.asarray(w).view(np.int8) if w_u8 else w, np.int8)
    d = len(strides)
    dilation = list(dilation) if dilation is not None else [1] * d
    shp = conv_out_shape(x.shape, w.shape, strides, padding, dilation)
    out = np.empty(shp, np.int32)
    a64 = lambda v: _c(list(v), np.int64)  # noqa: E731
    lib().q8r_quantized_conv_ex(x.reshape(-1), int(x_u8), w.reshape(-1), int(w_u8), d, a64(x.shape),
                                a64(w.shape), a64(strides), a64([p[0] for p in padding]),
                                a64([p[1] for p in padding]), a64(dilation), groups, zpx, zpw,
                                out.reshape(-1))
    return out


ACT = {"none": 0, "relu": 1, "silu": 2}


def gemv_w4(xq, sx, wq4, sw, K, group, bias=None, act="none") -> np.ndarray:
    """W4A8 per-group GEMV (composition defined in q8ref.h): exact per-group
    int sums, f64 sum over groups in ascending order, fround(S * sx[m])."""
    xq = _c(xq, np.int8)
    M = xq.shape[0]
    wq4 = _c(wq4, np.uint8)
    N = wq4.shape[0]
    sx = np.atleast_1d(_c(sx, np.float64))
    y = np.empty((M, N), np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().q8r_gemv_w4(xq.reshape(-1), sx, 1 if sx.size > 1 else 0, wq4.reshape(-1),
                      _c(sw, np.float64).reshape(-1), M, N, K, group,
                      None if b is None else b.ctypes.data_as(C.c_void_p), ACT[act], y.reshape(-1))
    return y


def epilogue(acc, mode, sA=None, sB=None, s_out=0.0, bias=None, act="none") -> np.ndarray:
    """mode 'pt': fround(acc*s_out) (quantization_pass.ts:335-355);
    mode 'rowcol': fround(acc * fround(sA[m]*sB[n])) (per-channel form, :431-456).
    sA / sB: arrays (per row / per column) or scalars."""
    acc = _c(acc, np.int32)
    M, N = acc.shape
    y = np.empty((M, N), np.float32)
    sa = np.atleast_1d(_c(sA if sA is not None else 1.0, np.float64))
    sb = np.atleast_1d(_c(sB if sB is not None else 1.0, np.float64))
    b = None if bias is None else _c(bias, np.float32)
    lib().q8r_epilogue(acc.reshape(-1), M, N, 0 if mode == "pt" else 1,
                       sa, 1 if sa.size > 1 else 0, sb, 1 if sb.size > 1 else 0, s_out,
                       None if b is None else b.ctypes.data_as(C.c_void_p), ACT[act], y.reshape(-1))
    return y


def relu(x) -> np.ndarray:
    f = lib().q8r_relu
    x = _c(x, np.float32)
    return np.array([f(float(v)) for v in x.reshape(-1)], np.float32).reshape(x.shape)


def silu_mul(g, u) -> np.ndarray:
    g = _c(g, np.float32)
    u = _c(u, np.float32)
    h = np.empty(g.shape, np.float32)
    lib().q8r_silu_mul(g.reshape(-1), u.reshape(-1), g.size, h.reshape(-1))
    return h


# ---------------------------------------------------------------- calibration
CALIB_MODES = {"minmax": 0, "percentile": 1, "entropy": 2}
SCHEMES = {"per_tensor_symmetric": 0, "per_tensor_asymmetric": 1, "per_channel": 2}


class Observer:
    """ValueObserver + HistogramCollector (src/compiler/analysis/calibration.ts:11-189)."""

    def __init__(self, num_bins: int = 2048, histogram: bool = True):
        self._bins = np.zeros(num_bins, np.float64)
        self._o = _Observer()
        lib().q8r_observer_init(C.byref(self._o), self._bins.ctypes.data_as(C.POINTER(C.c_double)),
                                num_bins, int(histogram))

    def update(self, x) -> None:
        x = _c(x, np.float32).reshape(-1)
        lib().q8r_observer_update(C.byref(self._o), x, x.size)

    @property
    def state(self) -> dict:
        o = self._o
        return {"min": o.min, "max": o.max, "count": o.count, "initialized": o.initialized,
                "range_min": o.range_min, "range_max": o.range_max,
                "total_count": o.total_count, "bins": self._bins.copy()}

    def percentile(self, p: float = 0.999) -> float:
        return lib().q8r_hist_percentile(C.byref(self._o), p)

    def entropy(self, num_quant_bins: int = 255) -> float:
        return lib().q8r_hist_entropy(C.byref(self._o), num_quant_bins)

    def params(self, mode: str = "minmax", scheme: str = "per_tensor_symmetric",
               unsigned: bool = False):
        """getQuantParams (calibration.ts:246-268) -> (scale, zero_point) or None."""
        s, z = _dbl(), _dbl()
        ok = lib().q8r_calib_params(C.byref(self._o), CALIB_MODES[mode], SCHEMES[scheme],
                                    int(unsigned), C.byref(s), C.byref(z))
        return (s.value, z.value) if ok else None
