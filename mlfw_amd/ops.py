"""Device ops of the int8 path, on torch tensors, computed by libq8hip.so.

PyTorch only provides device memory and the stream: every op below is one
call through the C ABI (include/q8hip.h) on torch's current stream.  Each
op mirrors a reference operator (src/compiler/ir/graph/ops/quantization.ts)
and reproduces the reference CPU backend's arithmetic bit for bit.

Tensors must be contiguous and live on the current HIP device; the ops
check dtype, shape and device before calling, and the C ABI validates again.
"""
from __future__ import annotations

import ctypes as C
import math

import torch

from . import _lib as L


def _stream() -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


class Launch:
    """One C-ABI call with its arguments validated and converted once.

    Calling it enqueues the op again on the stream captured at preparation
    time, with the same tensors (their storage must stay alive and keep its
    shape).  This is the host-side analogue of the reference runtime's
    prepared plans (src/runtime/runtime.ts:290-329): a serving or benchmark
    loop pays one foreign call per op instead of re-validating arguments.
    """

    __slots__ = ("name", "_fn", "_args", "_keep", "outputs")

    def __init__(self, name: str, args: tuple, keep: tuple = ()):
        self.name = name
        self._fn = getattr(L.load(), name)
        self._args = args
        self._keep = keep          # temporaries the raw pointers refer to
        self.outputs = None        # what the op returned (keeps the tensors alive)

    def __call__(self) -> None:
        rc = self._fn(*self._args)
        if rc != L.Q8_OK:
            L.check(rc)


_capture: list | None = None


def _call(name: str, *args, keep: tuple = ()) -> None:
    """Run one C-ABI entry point now, or record it while prepare() is active.
    `keep` lists temporaries a recorded launch must hold on to."""
    if _capture is not None:
        _capture.append(Launch(name, args, keep))
    else:
        L.call(name, *args)


def prepare(op, *args, **kwargs) -> Launch:
    """Validate `op(*args, **kwargs)` once and return its launch unrun.

    `op` is one of this module's single-launch ops (quantize_per_token,
    quantize_per_tensor, quantize, dequantize, quantized_dot, qlinear,
    qlinear_pt, silu_mul_quantize).  The returned Launch re-enqueues exactly
    that call; Launch.outputs holds what the op returned."""
    global _capture
    prev, _capture = _capture, []
    try:
        result = op(*args, **kwargs)
        recorded = _capture
    finally:
        _capture = prev
    if len(recorded) != 1:
        raise ValueError(f"prepare: {getattr(op, '__name__', op)} issued {len(recorded)} "
                         "launches; only single-launch ops can be prepared")
    recorded[0].outputs = result
    return recorded[0]


def _ptr(t) -> C.c_void_p:
    return C.c_void_p(0 if t is None else t.data_ptr())


def _need(t: torch.Tensor, dtype: torch.dtype, name: str, ndim: int | None = None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected dtype {dtype}, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name}: tensor must be on a HIP device (got {t.device})")
    if not t.is_contiguous():
        raise ValueError(f"{name}: tensor must be contiguous")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{name}: expected {ndim}-D, got shape {tuple(t.shape)}")


def _out(t, shape, dtype: torch.dtype, like: torch.Tensor, name: str = "out") -> torch.Tensor:
    """The caller's output tensor, checked (dtype, device, contiguity, element
    count -- the kernels write exactly that many elements), or a new one."""
    shape = tuple(shape) if isinstance(shape, (tuple, list, torch.Size)) else (int(shape),)
    if t is None:
        return torch.empty(shape, dtype=dtype, device=like.device)
    _need(t, dtype, name)
    if t.numel() != math.prod(shape):
        raise ValueError(f"{name}: expected {math.prod(shape)} elements (shape {shape}), got {tuple(t.shape)}")
    if t.device != like.device:
        raise ValueError(f"{name}: must be on {like.device}, got {t.device}")
    return t


def _rows(x: torch.Tensor):
    """[..., K] viewed as [M, K] with M the product of the leading dims."""
    if x.dim() == 0:
        return 1, 1
    M = 1
    for d in x.shape[:-1]:
        M *= d
    return M, x.shape[-1]


# ---------------------------------------------------------------- inputs
def fill_normal(t: torch.Tensor, seed: int, offset: int = 0, mean: float = 0.0,
                std: float = 1.0) -> int:
    """normal_ (src/nn/init.ts:40-52) on the device; returns draws consumed."""
    _need(t, torch.float32, "fill_normal")
    _call("q8_fill_normal", _ptr(t), t.numel(), seed & 0xFFFFFFFF, offset, mean, std, _stream())
    return 2 * ((t.numel() + 1) // 2)


def fill_uniform(t: torch.Tensor, seed: int, offset: int = 0, a: float = 0.0,
                 b: float = 1.0) -> int:
    """uniform_ (src/nn/init.ts:31-37) on the device; returns draws consumed."""
    _need(t, torch.float32, "fill_uniform")
    _call("q8_fill_uniform", _ptr(t), t.numel(), seed & 0xFFFFFFFF, offset, a, b, _stream())
    return t.numel()


def apply_outliers(t: torch.Tensor, seed: int, p: float = 0.01, factor: float = 50.0) -> None:
    """Scale the elements a second mulberry32 stream marks (draw < p) by factor."""
    _need(t, torch.float32, "apply_outliers")
    _call("q8_apply_outliers", _ptr(t), t.numel(), seed & 0xFFFFFFFF, p, factor, _stream())


# ---------------------------------------------------------------- quantize
def quantize(x: torch.Tensor, scale: float, zero_point: float = 0.0,
             target_dtype: str = "i8") -> torch.Tensor:
    """The `quantize` op with its static attrs (ops/quantization.ts:12-59,
    lowering quant_math.ts:16-27).  target_dtype 'i8' or 'ui8'."""
    _need(x, torch.float32, "quantize")
    if target_dtype not in ("i8", "ui8"):
        raise ValueError(f"quantize target_dtype must be i8 or ui8, got {target_dtype}")
    q = torch.empty(x.shape, dtype=torch.int8 if target_dtype == "i8" else torch.uint8,
                    device=x.device)
    _call("q8_quantize_static", _ptr(x), x.numel(), float(scale), float(zero_point),
           L.Q8_I8 if target_dtype == "i8" else L.Q8_U8, _ptr(q), _stream())
    return q


def quantize_per_token(x: torch.Tensor, q: torch.Tensor | None = None,
                       scales: torch.Tensor | None = None):
    """Dynamic symmetric int8 quantize with one f64 scale per row of the last
    dimension (calibration scale of each row, calibration.ts:24-34 +
    quantization_types.ts:248-254).  x is contiguous, or a 2-D row-strided
    view (e.g. a column slice of a wider projection output); the codes are
    [M, K] contiguous either way.  Returns (int8 codes, f64 scales[M])."""
    if isinstance(x, torch.Tensor) and not x.is_contiguous():
        if x.dtype != torch.float32 or not x.is_cuda or x.dim() != 2 or x.stride(1) != 1:
            raise ValueError("quantize_per_token: x must be contiguous or a 2-D fp32 device view "
                             "with unit column stride")
        M, K = x.shape
        q = _out(q, (M, K), torch.int8, x, "q")
        scales = _out(scales, M, torch.float64, x, "scales")
        _call("q8_quantize_rows_ld", _ptr(x), x.stride(0), M, K, _ptr(q), _ptr(scales), _stream())
        return q, scales
    _need(x, torch.float32, "quantize_per_token")
    M, K = _rows(x)
    q = _out(q, x.shape, torch.int8, x, "q")
    scales = _out(scales, M, torch.float64, x, "scales")
    _call("q8_quantize_rows", _ptr(x), M, K, L.Q8_PER_TOKEN, _ptr(q), _ptr(scales), _stream())
    return q, scales


def quantize_per_tensor(x: torch.Tensor, q: torch.Tensor | None = None,
                        scales: torch.Tensor | None = None):
    """Dynamic symmetric int8 quantize with one scale for the whole tensor.
    Returns (int8 codes, f64 scale tensor of one element)."""
    _need(x, torch.float32, "quantize_per_tensor")
    q = _out(q, x.shape, torch.int8, x, "q")
    scales = _out(scales, 1, torch.float64, x, "scales")
    _call("q8_quantize_rows", _ptr(x), 1, x.numel(), L.Q8_PER_TENSOR, _ptr(q), _ptr(scales),
           _stream())
    return q, scales


# ---------------------------------------------------------------- dequantize
_SRC = {torch.int8: L.Q8_I8, torch.uint8: L.Q8_U8, torch.int32: L.Q8_I32}


def dequantize(q: torch.Tensor, scale, zero_point: float = 0.0,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """The `dequantize` op (quant_math.ts:29-34).  `scale` is a python float
    (the op's static attr), a 1-element f64 tensor (per tensor) or an f64
    tensor with one scale per row (per token)."""
    if q.dtype not in _SRC:
        raise TypeError(f"dequantize: input must be int8, uint8 or int32, got {q.dtype}")
    _need(q, q.dtype, "dequantize")
    M, K = _rows(q)
    if isinstance(scale, torch.Tensor):
        _need(scale, torch.float64, "dequantize scale")
        gran = L.Q8_PER_TENSOR if scale.numel() == 1 else L.Q8_PER_TOKEN
        if gran == L.Q8_PER_TOKEN and scale.numel() != M:
            raise ValueError(f"dequantize: {scale.numel()} scales for {M} rows")
        s = scale
    else:
        gran = L.Q8_PER_TENSOR
        s = torch.tensor([float(scale)], dtype=torch.float64, device=q.device)
    y = _out(out, q.shape, torch.float32, q, "out")
    _call("q8_dequantize", _ptr(q), _SRC[q.dtype], M, K, _ptr(s), gran, float(zero_point),
          _ptr(y), _stream(), keep=(s,))
    return y


# ---------------------------------------------------------------- weights
def pack_weight(W: torch.Tensor, axis: int = 0, granularity: str = "per_channel"):
    """Quantize an fp32 weight on the device the way QuantizationPass does on
    the host (quantization_pass.ts:390-400; quantization_types.ts:299-317,
    :118-130).  axis 0: W is [N,K] (nn.Linear); axis 1: W is [K,N].
    Returns (int8 [N,K], f64 scales[N] or [1])."""
    _need(W, torch.float32, "pack_weight", ndim=2)
    rows, cols = W.shape
    N, K = (rows, cols) if axis == 0 else (cols, rows)
    if granularity not in ("per_channel", "per_tensor"):
        raise ValueError(f"pack_weight: unknown granularity {granularity}")
    per_tensor = granularity == "per_tensor"
    Wq = torch.empty((N, K), dtype=torch.int8, device=W.device)
    scales = torch.empty(1 if per_tensor else N, dtype=torch.float64, device=W.device)
    _call("q8_pack_weight", _ptr(W), rows, cols, axis,
           L.Q8_PER_TENSOR if per_tensor else L.Q8_PER_CHANNEL, _ptr(Wq), _ptr(scales), _stream())
    return Wq, scales


# ---------------------------------------------------------------- matmul
_ACT = {None: L.Q8_ACT_NONE, "none": L.Q8_ACT_NONE, "relu": L.Q8_ACT_RELU, "silu": L.Q8_ACT_SILU}


def _mk(A, B):
    _need(A, torch.int8, "A", ndim=2)
    _need(B, torch.int8, "B", ndim=2)
    M, K = A.shape
    N, K2 = B.shape
    if K != K2:
        raise ValueError(f"contraction mismatch: A is {tuple(A.shape)}, B is {tuple(B.shape)} ([N,K])")
    return M, N, K


def qlinear(A: torch.Tensor, sA: torch.Tensor, B: torch.Tensor, sB: torch.Tensor,
            bias: torch.Tensor | None = None, act: str | None = None,
            out: torch.Tensor | None = None) -> torch.Tensor:
    """int8 linear with the per-channel epilogue fused:
    y = act(fround(fround(acc * fround(sA[m] * sB[n])) + bias[n])).
    sA: f64 [M] (per token) or [1] (per tensor); sB: f64 [N] or [1]."""
    M, N, K = _mk(A, B)
    _need(sA, torch.float64, "sA")
    _need(sB, torch.float64, "sB")
    if sA.numel() not in (1, M) or sB.numel() not in (1, N):
        raise ValueError("qlinear: scale sizes must be 1 or M (sA) and 1 or N (sB)")
    if bias is not None:
        _need(bias, torch.float32, "bias")
        if bias.numel() != N:
            raise ValueError("qlinear: bias must have N elements")
    out = _out(out, (M, N), torch.float32, A, "out")
    _call("q8_gemm", _ptr(A), _ptr(B), M, N, K, 0, 0,
           _ptr(sA), L.Q8_PER_TOKEN if sA.numel() == M and M != 1 else L.Q8_PER_TENSOR,
           _ptr(sB), L.Q8_PER_CHANNEL if sB.numel() == N and N != 1 else L.Q8_PER_TENSOR,
           L.Q8_EPI_ROWCOL, 0.0, _ptr(bias), _ACT[act], L.Q8_F32, _ptr(out), _stream())
    return out


def glu_interleave(gate, up, gate_bias: torch.Tensor | None = None, up_bias: torch.Tensor | None = None):
    """The weight of qlinear_glu from two per-channel packed weights
    (pack_weight results (int8 [F,K], f64 [F]) for gate and up, F a multiple
    of 32): rows interleaved in groups of 32 (packed row 64 j + c is gate row
    32 j + c, 64 j + 32 + c is up row 32 j + c), scales and optional biases
    alike.  Returns (int8 [2F,K], f64 [2F]) or, with biases, (..., f32 [2F])."""
    (Wg, sg), (Wu, su) = gate, up
    for t, dt, what in ((Wg, torch.int8, "gate codes"), (Wu, torch.int8, "up codes")):
        _need(t, dt, what, ndim=2)
    F, K = Wg.shape
    if tuple(Wu.shape) != (F, K):
        raise ValueError("glu_interleave: gate and up weights must have the same shape")
    for t, what in ((sg, "gate scales"), (su, "up scales")):
        _need(t, torch.float64, what)
        if t.numel() != F:
            raise ValueError(f"glu_interleave: {what} must be per channel ({F} values)")
    if (gate_bias is None) != (up_bias is None):
        raise ValueError("glu_interleave: give both biases or none")
    W = torch.empty((2 * F, K), dtype=torch.int8, device=Wg.device)
    s = torch.empty(2 * F, dtype=torch.float64, device=Wg.device)
    b = None
    if gate_bias is not None:
        for t, what in ((gate_bias, "gate bias"), (up_bias, "up bias")):
            _need(t, torch.float32, what)
            if t.numel() != F:
                raise ValueError(f"glu_interleave: {what} must have {F} elements")
        b = torch.empty(2 * F, dtype=torch.float32, device=Wg.device)
    _call("q8_glu_interleave", _ptr(Wg), _ptr(sg), _ptr(gate_bias), _ptr(Wu), _ptr(su), _ptr(up_bias), F, K,
          _ptr(W), _ptr(s), _ptr(b), _stream())
    return (W, s) if b is None else (W, s, b)


def qlinear_glu(A: torch.Tensor, sA: torch.Tensor, W: torch.Tensor, sW: torch.Tensor,
                bias: torch.Tensor | None = None, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Gate and up linears with h = fround(silu(g) * u) fused into one GEMM
    (q8_gemm_glu): W, sW (and bias) from glu_interleave; returns h fp32
    [M, F], bit for bit qlinear of each half followed by silu_mul."""
    M, N, K = _mk(A, W)
    _need(sA, torch.float64, "sA")
    _need(sW, torch.float64, "sW")
    if N % 64 != 0:
        raise ValueError("qlinear_glu: the interleaved weight must have 2F rows, F a multiple of 32")
    F = N // 2
    if sA.numel() not in (1, M) or sW.numel() not in (1, N):
        raise ValueError("qlinear_glu: scale sizes must be 1 or M (sA) and 1 or 2F (sW)")
    if bias is not None:
        _need(bias, torch.float32, "bias")
        if bias.numel() != N:
            raise ValueError("qlinear_glu: bias must have 2F elements (interleaved)")
    out = _out(out, (M, F), torch.float32, A, "out")
    nb = C.c_size_t(0)
    L.call("q8_gemm_glu_workspace", M, F, K, C.byref(nb))
    if nb.value and (workspace is None or workspace.numel() < nb.value):
        workspace = torch.empty(nb.value, dtype=torch.int8, device=A.device)
    _call("q8_gemm_glu", _ptr(A), _ptr(W), M, F, K,
          _ptr(sA), L.Q8_PER_TOKEN if sA.numel() == M and M != 1 else L.Q8_PER_TENSOR,
          _ptr(sW), L.Q8_PER_CHANNEL if sW.numel() == N else L.Q8_PER_TENSOR,
          _ptr(bias), _ptr(out), _ptr(workspace), workspace.numel() if workspace is not None else 0, _stream(),
          keep=(workspace,) if workspace is not None else ())
    return out


def quantized_dot(A: torch.Tensor, B: torch.Tensor, zpA: int = 0, zpB: int = 0,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's quantized_dot: int32 [M,N] = sum_k (A[m,k] - zpA) *
    (B[n,k] - zpB), exact, stored ToInt32.  A [M,K] and B [N,K] are int8
    (read as i8) or uint8 (read as ui8) tensors."""
    codes = {torch.int8: L.Q8_I8, torch.uint8: L.Q8_U8}
    for t, name in ((A, "A"), (B, "B")):
        if t.dtype not in codes or t.dim() != 2 or not t.is_contiguous():
            raise ValueError(f"quantized_dot: {name} must be a contiguous 2-D int8 or uint8 tensor")
    M, K = A.shape
    N = B.shape[0]
    if B.shape[1] != K:
        raise ValueError("quantized_dot: A [M,K] and B [N,K] must share K")
    ws_bytes = C.c_size_t(0)
    _call("q8_quantized_dot_workspace", M, N, K, codes[A.dtype], codes[B.dtype], int(zpA), int(zpB),
           C.byref(ws_bytes))
    ws = torch.empty(max(ws_bytes.value, 1), dtype=torch.uint8, device=A.device)
    out = _out(out, (M, N), torch.int32, A, "out")
    _call("q8_quantized_dot", _ptr(A), codes[A.dtype], _ptr(B), codes[B.dtype], M, N, K, int(zpA),
           int(zpB), _ptr(ws), ws_bytes.value, _ptr(out), _stream())
    return out


def qlinear_dynamic(x: torch.Tensor, Wq: torch.Tensor, sW: torch.Tensor,
                    bias: torch.Tensor | None = None, act: str | None = None,
                    per_tensor: bool = False, out: torch.Tensor | None = None,
                    xq: torch.Tensor | None = None, sx: torch.Tensor | None = None):
    """Dynamic int8 linear in one call: quantize x (fp32 [M,K]) per token (or
    per tensor), then the int8 GEMM with the qlinear epilogue.  Equal bit
    for bit to quantize_per_token / quantize_per_tensor followed by qlinear;
    one-token decode (M = 1, K <= 4096) runs as one kernel, larger M as the
    quantize and the GEMM / GEMV back to back.
    Returns (y fp32 [M,N], int8 codes [M,K], f64 scales [M] or [1])."""
    _need(x, torch.float32, "x")
    M, K = _rows(x)
    _need(Wq, torch.int8, "Wq")
    if Wq.dim() != 2 or Wq.shape[1] != K or not Wq.is_contiguous():
        raise ValueError("qlinear_dynamic: Wq must be a contiguous [N, K] int8 tensor")
    N = Wq.shape[0]
    _need(sW, torch.float64, "sW")
    if sW.numel() not in (1, N):
        raise ValueError("qlinear_dynamic: sW must have 1 or N elements")
    if bias is not None:
        _need(bias, torch.float32, "bias")
        if bias.numel() != N:
            raise ValueError("qlinear_dynamic: bias must have N elements")
    out = _out(out, (M, N), torch.float32, x, "out")
    xq = _out(xq, (M, K), torch.int8, x, "xq")
    sx = _out(sx, 1 if per_tensor else M, torch.float64, x, "sx")
    _call("q8_qlinear_dynamic", _ptr(x), M, K, L.Q8_PER_TENSOR if per_tensor else L.Q8_PER_TOKEN,
           _ptr(Wq), _ptr(sW), L.Q8_PER_CHANNEL if sW.numel() == N and N != 1 else L.Q8_PER_TENSOR,
           N, _ptr(bias), _ACT[act], _ptr(out), _ptr(xq), _ptr(sx), _stream())
    return out, xq, sx


def qlinear_pt(A: torch.Tensor, B: torch.Tensor, s_out: float,
               bias: torch.Tensor | None = None, act: str | None = None,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-tensor form (quantization_pass.ts:335-355): y = fround(acc * s_out),
    s_out = lhs_scale * rhs_scale in f64."""
    M, N, K = _mk(A, B)
    out = _out(out, (M, N), torch.float32, A, "out")
    _call("q8_gemm", _ptr(A), _ptr(B), M, N, K, 0, 0, None, 0, None, 0, L.Q8_EPI_PT,
           float(s_out), _ptr(bias), _ACT[act], L.Q8_F32, _ptr(out), _stream())
    return out


def qlinear_requant(A: torch.Tensor, sA: torch.Tensor | None, B: torch.Tensor,
                    sB: torch.Tensor | None, s_next: float, bias: torch.Tensor | None = None,
                    act: str | None = None, s_out: float | None = None,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """int8 linear whose fp32 result (the qlinear epilogue, or with s_out
    the per-tensor one) is requantized in the epilogue with the next layer's
    static scale s_next: the calibrated dequantize -> [bias] -> [relu] ->
    quantize chain of QuantizationPass, returned as int8 [M, N]."""
    M, N, K = _mk(A, B)
    if bias is not None:
        _need(bias, torch.float32, "bias")
        if bias.numel() != N:
            raise ValueError("qlinear_requant: bias must have N elements")
    out = _out(out, (M, N), torch.int8, A, "out")
    _need(out, torch.int8, "qlinear_requant out")
    if s_out is None:
        _need(sA, torch.float64, "sA")
        _need(sB, torch.float64, "sB")
        if sA.numel() not in (1, M) or sB.numel() not in (1, N):
            raise ValueError("qlinear_requant: scale sizes must be 1 or M (sA) and 1 or N (sB)")
        _call("q8_gemm_requant", _ptr(A), _ptr(B), M, N, K,
               _ptr(sA), L.Q8_PER_TOKEN if sA.numel() == M and M != 1 else L.Q8_PER_TENSOR,
               _ptr(sB), L.Q8_PER_CHANNEL if sB.numel() == N and N != 1 else L.Q8_PER_TENSOR,
               L.Q8_EPI_ROWCOL, 0.0, _ptr(bias), _ACT[act], float(s_next), _ptr(out), _stream())
    else:
        _call("q8_gemm_requant", _ptr(A), _ptr(B), M, N, K, None, 0, None, 0, L.Q8_EPI_PT,
               float(s_out), _ptr(bias), _ACT[act], float(s_next), _ptr(out), _stream())
    return out


def generic_gemm_launches() -> int:
    """Launches of the generic (non-MFMA) GEMM kernel so far in this process:
    GEMMs whose K is not a multiple of 16 or whose operands are not 16-byte
    aligned take it."""
    n = C.c_int64(0)
    L.call("q8_generic_gemm_launches", C.byref(n))
    return n.value


def requant_dynamic_workspace(M: int, N: int, K: int):
    """(bytes, fused) of q8_gemm_requant_dynamic for this shape."""
    nb, fused = C.c_size_t(0), C.c_int(0)
    L.call("q8_gemm_requant_dynamic_workspace", M, N, K, C.byref(nb), C.byref(fused))
    return nb.value, bool(fused.value)


def qlinear_requant_dynamic(A: torch.Tensor, sA: torch.Tensor, B: torch.Tensor, sB: torch.Tensor,
                            bias: torch.Tensor | None = None, act: str | None = None,
                            out: torch.Tensor | None = None, scales: torch.Tensor | None = None,
                            workspace: torch.Tensor | None = None, check: bool = False):
    """int8 linear whose fp32 result (the qlinear epilogue) is requantized per
    row with the row's own dynamic absmax scale, as the next layer's
    per-token quantize takes it: returns (int8 codes [M, N], f64 scales [M]),
    bit for bit qlinear followed by quantize_per_token.  When every tile of
    the MFMA GEMM has a CU of its own the fp32 tensor never reaches memory
    (one launch whose tiles meet once grid-wide); the workspace holds the
    row keys then, or the fp32 result on the fallback route.

    The grid-wide wait is bounded: if other streams or processes hold CUs
    long enough for it to run out, the result is unreliable and the status
    word says so.  check=True reads that word (a stream synchronization) and
    raises RuntimeError on a timeout; callers that share the device should
    check, callers that cannot synchronize (graph capture) read it later
    with requant_dynamic_timed_out."""
    M, N, K = _mk(A, B)
    _need(sA, torch.float64, "sA")
    _need(sB, torch.float64, "sB")
    if sA.numel() not in (1, M) or sB.numel() not in (1, N):
        raise ValueError("qlinear_requant_dynamic: scale sizes must be 1 or M (sA) and 1 or N (sB)")
    if bias is not None:
        _need(bias, torch.float32, "bias")
        if bias.numel() != N:
            raise ValueError("qlinear_requant_dynamic: bias must have N elements")
    out = _out(out, (M, N), torch.int8, A, "out")
    scales = _out(scales, M, torch.float64, A, "scales")
    nb, fused = requant_dynamic_workspace(M, N, K)
    if workspace is None or workspace.numel() < nb:
        workspace = torch.empty(max(nb, 1), dtype=torch.int8, device=A.device)
    _call("q8_gemm_requant_dynamic", _ptr(A), _ptr(B), M, N, K,
          _ptr(sA), L.Q8_PER_TOKEN if sA.numel() == M and M != 1 else L.Q8_PER_TENSOR,
          _ptr(sB), L.Q8_PER_CHANNEL if sB.numel() == N and N != 1 else L.Q8_PER_TENSOR,
          L.Q8_EPI_ROWCOL, 0.0, _ptr(bias), _ACT[act], _ptr(out), _ptr(scales), _ptr(workspace),
          workspace.numel(), _stream(), keep=(workspace,))
    if check and fused and requant_dynamic_timed_out(workspace, M):
        raise RuntimeError("qlinear_requant_dynamic: the grid-wide wait ran out (other work held CUs); "
                           "the codes and scales of this call are unreliable")
    return out, scales


def requant_dynamic_timed_out(workspace: torch.Tensor, M: int) -> bool:
    """Whether the last qlinear_requant_dynamic call on this workspace (M
    rows) ran out of its grid-wide wait; meaningful after a call that took
    the fused route (requant_dynamic_workspace).  Synchronizes the current
    stream."""
    flag = C.c_int(0)
    L.call("q8_gemm_requant_dynamic_status", _ptr(workspace), M, C.byref(flag), _stream())
    return flag.value != 0


def pack_weight_int4(W: torch.Tensor, group_size: int):
    """4-bit per-group weight packing (fromConstantArrayPerGroup +
    quantizeArrayPerGroup, quantization_types.ts:319-340, :143-153) of an
    fp32 [N, K] weight -> (uint8 [N, K/2] nibbles, f64 scales [N*K/group])."""
    _need(W, torch.float32, "pack_weight_int4", ndim=2)
    N, K = W.shape
    wq = torch.empty((N, K // 2), dtype=torch.uint8, device=W.device)
    s = torch.empty(N * K // max(group_size, 1), dtype=torch.float64, device=W.device)
    _call("q8_pack_weight_int4", _ptr(W), N, K, group_size, _ptr(wq), _ptr(s), _stream())
    return wq, s


def qlinear_w4(xq: torch.Tensor, sx: torch.Tensor, Wq4: torch.Tensor, sw: torch.Tensor,
               K: int, group_size: int, bias: torch.Tensor | None = None,
               act: str | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """W4A8 linear (q8_gemv_w4): int8 [M, K] activations with f64 scales
    ([M] per token or [1]) times 4-bit per-group weights -> fp32 [M, N]."""
    _need(xq, torch.int8, "qlinear_w4 xq", ndim=2)
    _need(sx, torch.float64, "qlinear_w4 sx")
    _need(Wq4, torch.uint8, "qlinear_w4 Wq4", ndim=2)
    _need(sw, torch.float64, "qlinear_w4 sw")
    M, N = xq.shape[0], Wq4.shape[0]
    if xq.shape[1] != K or Wq4.shape[1] != K // 2:
        raise ValueError("qlinear_w4: shapes do not match K")
    if bias is not None:
        _need(bias, torch.float32, "bias")
    out = _out(out, (M, N), torch.float32, xq, "out")
    _call("q8_gemv_w4", _ptr(xq), _ptr(sx), L.Q8_PER_TOKEN if sx.numel() == M and M != 1 else L.Q8_PER_TENSOR,
          _ptr(Wq4), _ptr(sw), M, N, K, group_size, _ptr(bias), _ACT[act], _ptr(out), _stream())
    return out


def _i64_array(vals):
    arr = (C.c_int64 * max(1, len(vals)))(*[int(v) for v in vals])
    return arr


def conv_out_shape(x_shape, w_shape, strides, padding, dilation=None):
    """[N, O, P_0..] of quantized_conv (inferConvResultTypes,
    src/compiler/ir/graph/ops/linalg.ts:222-248); padding is [[lo, hi], ...]."""
    d = len(strides)
    dilation = list(dilation) if dilation is not None else [1] * d
    out = [int(x_shape[0]), int(w_shape[0])]
    for i in range(d):
        eff = (int(w_shape[2 + i]) - 1) * dilation[i] + 1
        out.append((int(x_shape[2 + i]) + padding[i][0] + padding[i][1] - eff) // strides[i] + 1)
    return out


def conv_weight_taps(w: torch.Tensor, groups: int = 1):
    """The tap-major copy of a constant int8 conv weight [O, C/groups, K..]
    that quantized_conv(..., w_taps=) uses instead of permuting w on every
    call (q8_conv_weight_taps); None for weight shapes that are used as
    given (channels per group not a multiple of 16, one kernel position)."""
    _need(w, torch.int8, "conv_weight_taps w")
    d = w.dim() - 2
    if d < 1 or d > 3:
        raise ValueError("conv_weight_taps: w must be [O, C/groups, K..] with 1-3 spatial dims")
    kn = math.prod(w.shape[2:])
    if w.shape[1] % 16 != 0 or kn < 2 or kn > 1024:
        return None
    wt = torch.empty(w.numel(), dtype=torch.int8, device=w.device)
    ws = _i64_array(w.shape)
    _call("q8_conv_weight_taps", _ptr(w), d, ws, groups, _ptr(wt), _stream(), keep=(ws,))
    return wt


def quantized_conv(x: torch.Tensor, w: torch.Tensor, strides, padding, dilation=None,
                   groups: int = 1, s_out: float | None = None, out: torch.Tensor | None = None,
                   workspace: torch.Tensor | None = None, zpx: int = 0,
                   zpw: int = 0, w_taps: torch.Tensor | None = None) -> torch.Tensor:
    """quantized_conv (src/compiler/ir/graph/ops/quantization.ts:156-190):
    x [N, C, S..] (NCHW and its 1-D / 3-D forms) and w [O, C/groups, K..]
    (OIHW), each int8 (read as i8) or uint8 (read as ui8), padding as
    [[lo, hi], ...] per spatial dim, zero points zpx / zpw.  s_out None: the
    int32 accumulator; otherwise the fused per-tensor dequantize
    fround(acc * s_out) as fp32 (the `dequantize` QuantizationPass appends,
    output_scale = input_scale * kernel_scale).  w_taps: conv_weight_taps(w)
    of a constant weight, so the call does not permute it (int8 operands,
    same output bits)."""
    codes = {torch.int8: L.Q8_I8, torch.uint8: L.Q8_U8}
    for t, name in ((x, "x"), (w, "w")):
        if t.dtype not in codes:
            raise ValueError(f"quantized_conv: {name} must be int8 or uint8")
        _need(t, t.dtype, f"quantized_conv {name}")
    d = len(strides)
    if x.dim() != 2 + d or w.dim() != 2 + d or len(padding) != d:
        raise ValueError(f"quantized_conv: {d} spatial dims need {2 + d}-D x and w and {d} padding pairs")
    dilation = list(dilation) if dilation is not None else [1] * d
    xs, ws = _i64_array(x.shape), _i64_array(w.shape)
    st, dl = _i64_array(strides), _i64_array(dilation)
    lo, hi = _i64_array([p[0] for p in padding]), _i64_array([p[1] for p in padding])
    need = C.c_size_t(0)
    L.call("q8_quantized_conv_workspace", d, xs, ws, st, lo, hi, dl, groups, C.byref(need))
    shape = conv_out_shape(x.shape, w.shape, strides, padding, dilation)
    dtype = torch.int32 if s_out is None else torch.float32
    if out is None:
        out = torch.empty(shape, dtype=dtype, device=x.device)
    else:
        _need(out, dtype, "quantized_conv out")
        if list(out.shape) != shape:
            raise ValueError(f"quantized_conv: out must have shape {shape}")
    if need.value and (workspace is None or workspace.numel() < need.value):
        workspace = torch.empty(need.value, dtype=torch.int8, device=x.device)
    if w_taps is not None:
        if x.dtype != torch.int8 or w.dtype != torch.int8:
            raise ValueError("quantized_conv: w_taps is for int8 operands")
        _need(w_taps, torch.int8, "quantized_conv w_taps")
        if w_taps.numel() != w.numel():
            raise ValueError("quantized_conv: w_taps must be conv_weight_taps(w)")
        _call("q8_quantized_conv_prepacked", _ptr(x), _ptr(w), _ptr(w_taps), d, xs, ws, st, lo, hi, dl, groups,
              int(zpx), int(zpw), L.Q8_I32 if s_out is None else L.Q8_F32, 0.0 if s_out is None else float(s_out),
              _ptr(workspace if need.value else None), need.value, _ptr(out), _stream(),
              keep=(xs, ws, st, lo, hi, dl, workspace, w_taps))
        return out
    _call("q8_quantized_conv_ex", _ptr(x), codes[x.dtype], _ptr(w), codes[w.dtype], d, xs, ws, st, lo,
          hi, dl, groups, int(zpx), int(zpw),
          L.Q8_I32 if s_out is None else L.Q8_F32, 0.0 if s_out is None else float(s_out),
          _ptr(workspace if need.value else None), need.value, _ptr(out), _stream(),
          keep=(xs, ws, st, lo, hi, dl, workspace))
    return out


def silu_mul_quantize(g: torch.Tensor, u: torch.Tensor, h_out: torch.Tensor | None = None):
    """h = fround(silu(g) * u), then per-token int8 quantize of h.
    g and u are contiguous, or 2-D row-strided views (e.g. the two halves of
    one [M, 2K] GEMM output).  Returns (int8 codes [M, K], f64 scales[M])."""
    if g.shape != u.shape:
        raise ValueError("silu_mul_quantize: g and u shapes differ")
    lds = []
    for t, name in ((g, "g"), (u, "u")):
        if t.is_contiguous():
            _need(t, torch.float32, name)
            lds.append(None)
        else:
            if t.dtype != torch.float32 or not t.is_cuda or t.dim() != 2 or t.stride(1) != 1:
                raise ValueError(f"silu_mul_quantize: {name} must be contiguous or a 2-D fp32 device "
                                 "view with unit column stride")
            lds.append(t.stride(0))
    M, K = _rows(g) if g.is_contiguous() else g.shape
    ldg = K if lds[0] is None else lds[0]
    ldu = K if lds[1] is None else lds[1]
    q = torch.empty(g.shape, dtype=torch.int8, device=g.device)
    scales = torch.empty(M, dtype=torch.float64, device=g.device)
    if h_out is not None:
        _out(h_out, (M, K), torch.float32, g, "h_out")
    _call("q8_silu_mul_quantize_rows_ld", _ptr(g), ldg, _ptr(u), ldu, M, K, _ptr(h_out), _ptr(q),
          _ptr(scales), _stream())
    return q, scales


# ------------------------------------------------------------------ elementwise programs
# Python form of q8_ew_prog (include/q8hip.h): a loop nest of up to 6 loops,
# inputs read at affine offsets of the loop indices, and straight-line code
# over 16 f64 registers with the reference CPU codegen's rounding
# (src/backend/cpu/codegen.ts:428-552).  The Node host builds these from
# PrimFuncs (mlfw_amd/node/ewise.js); this form serves the tests and bench.
EW_MAX_DIMS, EW_MAX_INPUTS, EW_MAX_CODE, EW_MAX_CONST = 6, 8, 96, 32
EW_OPS = {name: i for i, name in enumerate(
    ["load", "const", "index", "add", "sub", "mul", "div", "idiv", "mod", "floordiv", "tmod", "tdiv", "neg",
     "cmp", "select", "toint32", "tobool", "max", "min", "abs", "floor", "ceil", "round", "sign", "sqrt",
     "fmod", "exp", "log", "tanh", "rsqrt", "pow"])}
_EW_DTYPES = {torch.int8: L.Q8_I8, torch.uint8: L.Q8_U8, torch.int32: L.Q8_I32, torch.float32: L.Q8_F32,
              torch.float64: 4}


class EwInstr(C.Structure):
    _fields_ = [(n, C.c_uint8) for n in ("op", "dst", "a", "b", "c", "aux", "rnd", "pad")]


class EwProg(C.Structure):
    _fields_ = [("ndims", C.c_int32), ("ninputs", C.c_int32), ("extent", C.c_int64 * EW_MAX_DIMS),
                ("in_dtype", C.c_int32 * EW_MAX_INPUTS),
                ("in_coef", (C.c_int64 * (EW_MAX_DIMS + 1)) * EW_MAX_INPUTS),
                ("out_dtype", C.c_int32), ("ncode", C.c_int32), ("result", C.c_int32), ("nconst", C.c_int32),
                ("code", EwInstr * EW_MAX_CODE), ("konst", C.c_double * EW_MAX_CONST)]


def ew_program(extents, inputs, code, result, out_dtype, konst=()):
    """An EwProg.  inputs: [(dtype, coefs)] with coefs the per-loop element
    strides (len(extents) of them, 0 for a broadcast loop) plus an optional
    constant offset; code: [(op, dst, a, b, c, aux, rnd)] with op a name of
    EW_OPS; result: the register stored; out_dtype a torch dtype."""
    p = EwProg()
    p.ndims, p.ninputs = len(extents), len(inputs)
    if not 1 <= p.ndims <= EW_MAX_DIMS or p.ninputs > EW_MAX_INPUTS or len(code) > EW_MAX_CODE:
        raise ValueError("ew_program: too many loops, inputs or instructions")
    for d, x in enumerate(extents):
        p.extent[d] = int(x)
    for j, (dt, coefs) in enumerate(inputs):
        p.in_dtype[j] = _EW_DTYPES[dt]
        coefs = list(coefs)
        for d in range(p.ndims):
            p.in_coef[j][d] = int(coefs[d])
        p.in_coef[j][EW_MAX_DIMS] = int(coefs[p.ndims]) if len(coefs) > p.ndims else 0
    for i, (op, dst, a, b, c, aux, rnd) in enumerate(code):
        p.code[i] = EwInstr(EW_OPS[op], dst, a, b, c, aux, rnd, 0)
    p.ncode, p.result, p.out_dtype = len(code), int(result), _EW_DTYPES[out_dtype]
    for i, k in enumerate(konst):
        p.konst[i] = float(k)
    p.nconst = len(konst)
    return p


def ewise(prog: EwProg, inputs, out: torch.Tensor) -> torch.Tensor:
    """Runs an elementwise program over device tensors (contiguous, the
    program's dtypes); out holds the product of the extents."""
    n = len(inputs)
    ins = (C.c_void_p * max(n, 1))(*[t.data_ptr() for t in inputs])
    nums = (C.c_int64 * max(n, 1))(*[t.numel() for t in inputs])
    _call("q8_ewise", C.c_void_p(C.addressof(prog)), C.cast(ins, C.c_void_p), C.cast(nums, C.c_void_p),
          _ptr(out), out.numel(), _stream(), keep=(prog, ins, nums))
    return out


def ewise_jit_error() -> str:
    """Why the last program that hiprtc could not compile fell back to the
    interpreter ("" if none has)."""
    n = C.c_size_t(0)
    buf = C.create_string_buffer(4096)
    _call("q8_debug_ewise_jit_error", C.cast(buf, C.c_void_p), C.sizeof(buf), C.byref(n))
    return buf.value.decode(errors="replace")
