"""CPU checks of the C ABI (include/q8hip.h <-> mlfw_amd/libq8hip.so).

No kernel is launched here: the library is loaded, every entry point the
header declares must be exported, and calls that fail host-side validation
must return Q8_ERR_INVALID with a message before anything reaches a device.
"""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "q8hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(q8_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    from mlfw_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail("libq8hip.so is not built: run `python -m mlfw_amd.build`")
    return _lib


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("q8_init", "q8_last_error", "q8_quantize_rows", "q8_quantize_static",
                 "q8_dequantize", "q8_pack_weight", "q8_gemm", "q8_gemv"):
        assert must in names


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared_functions()
    raw = C.CDLL(lib.LIB_PATH)
    for n in names:
        assert hasattr(raw, n), f"{n} declared in q8hip.h but not exported"
    assert sorted(lib.exported_symbols()) == names, "ctypes binding and header disagree"


def test_version_and_clean_error(lib):
    L = lib.load()
    assert L.q8_version() == 1
    assert L.q8_last_error() in (b"",)


def test_device_count_does_not_fail_without_gpu(lib):
    n = C.c_int(-1)
    assert lib.load().q8_device_count(C.byref(n)) == lib.Q8_OK
    assert n.value >= 0


def expect_invalid(lib, name, *args, match=""):
    rc = getattr(lib.load(), name)(*args)
    assert rc == lib.Q8_ERR_INVALID, (name, rc)
    msg = lib.load().q8_last_error().decode()
    assert name in msg or match in msg, msg


def test_validation_happens_before_any_launch(lib):
    vp, nil = C.c_void_p, None
    fake = vp(0x1000)
    expect_invalid(lib, "q8_quantize_static", fake, 10, 0.0, 0.0, lib.Q8_I8, fake, nil)
    expect_invalid(lib, "q8_quantize_static", fake, 10, -1.0, 0.0, lib.Q8_I8, fake, nil)
    expect_invalid(lib, "q8_quantize_static", fake, 10, 0.1, 0.0, lib.Q8_I32, fake, nil)
    expect_invalid(lib, "q8_quantize_static", fake, -1, 0.1, 0.0, lib.Q8_I8, fake, nil)
    expect_invalid(lib, "q8_quantize_rows", fake, 4, 8, 7, fake, fake, nil)
    expect_invalid(lib, "q8_quantize_rows", fake, -4, 8, lib.Q8_PER_TOKEN, fake, fake, nil)
    expect_invalid(lib, "q8_quantize_rows", nil, 4, 8, lib.Q8_PER_TOKEN, fake, fake, nil)
    # row-strided forms: the row stride may not be below the row length
    expect_invalid(lib, "q8_quantize_rows_ld", fake, 7, 4, 8, fake, fake, nil)
    expect_invalid(lib, "q8_quantize_rows_ld", fake, -1, 4, 8, fake, fake, nil)
    expect_invalid(lib, "q8_quantize_rows_ld", nil, 16, 4, 8, fake, fake, nil)
    expect_invalid(lib, "q8_quantize_rows_ld", fake, 16, 4, 8, fake, nil, nil)
    expect_invalid(lib, "q8_silu_mul_quantize_rows_ld", fake, 7, fake, 8, 4, 8, nil, fake, fake, nil)
    expect_invalid(lib, "q8_silu_mul_quantize_rows_ld", fake, 8, fake, 3, 4, 8, nil, fake, fake, nil)
    expect_invalid(lib, "q8_silu_mul_quantize_rows_ld", fake, 16, nil, 16, 4, 8, nil, fake, fake, nil)
    expect_invalid(lib, "q8_dequantize", fake, lib.Q8_F32, 4, 8, fake, lib.Q8_PER_TENSOR, 0.0,
                   fake, nil)
    expect_invalid(lib, "q8_dequantize", fake, lib.Q8_I8, 4, 8, fake, 9, 0.0, fake, nil)
    expect_invalid(lib, "q8_pack_weight", fake, 4, 8, 2, lib.Q8_PER_CHANNEL, fake, fake, nil)
    expect_invalid(lib, "q8_pack_weight", fake, 4, 8, 0, lib.Q8_PER_TOKEN, fake, fake, nil)
    g = lib.load().q8_gemm
    # bad out_kind, act, epi, mismatched scale modes, null operands
    assert g(fake, fake, 4, 4, 16, 0, 0, fake, 0, fake, 0, 0, 1.0, nil, 0, 7, fake, nil) == 1
    assert g(fake, fake, 4, 4, 16, 0, 0, fake, 0, fake, 0, 0, 1.0, nil, 5, lib.Q8_F32, fake, nil) == 1
    assert g(fake, fake, 4, 4, 16, 0, 0, fake, 0, fake, 0, 9, 1.0, nil, 0, lib.Q8_F32, fake, nil) == 1
    assert g(nil, fake, 4, 4, 16, 0, 0, fake, 0, fake, 0, 1, 0.0, nil, 0, lib.Q8_F32, fake, nil) == 1
    assert g(fake, fake, 4, 4, 16, 0, 0, nil, 1, fake, 2, 1, 0.0, nil, 0, lib.Q8_F32, fake, nil) == 1
    assert g(fake, fake, 4, 4, 16, 0, 0, fake, 2, fake, 2, 1, 0.0, nil, 0, lib.Q8_F32, fake, nil) == 1
    # int32 output takes no bias / activation
    assert g(fake, fake, 4, 4, 16, 0, 0, nil, 0, nil, 0, 0, 0.0, fake, 0, lib.Q8_I32, fake, nil) == 1
    assert g(fake, fake, -1, 4, 16, 0, 0, nil, 0, nil, 0, 0, 0.0, nil, 0, lib.Q8_I32, fake, nil) == 1
    # q8_gemv only takes M <= 16
    gv = lib.load().q8_gemv
    assert gv(fake, fake, 17, 4, 16, fake, 0, fake, 0, 1, 0.0, nil, 0, lib.Q8_F32, fake, nil) == 1


def test_per_tensor_key_needs_an_aligned_scale_slot(lib):
    """Per-tensor reductions keep their running key in the caller's scales
    output (a 64-bit atomic), so that slot must be 8-byte aligned."""
    fake, odd, nil = C.c_void_p(0x1000), C.c_void_p(0x1004), None
    expect_invalid(lib, "q8_quantize_rows", fake, 4, 8, lib.Q8_PER_TENSOR, fake, odd, nil,
                   match="aligned")
    expect_invalid(lib, "q8_pack_weight", fake, 4, 8, 0, lib.Q8_PER_TENSOR, fake, odd, nil,
                   match="aligned")
    expect_invalid(lib, "q8_qlinear_dynamic", fake, 4, 16, lib.Q8_PER_TENSOR, fake, fake,
                   lib.Q8_PER_CHANNEL, 8, nil, 0, fake, fake, odd, nil, match="aligned")


def test_nonzero_zero_points_are_unsupported_not_wrong(lib):
    """q8_gemm (the fused-epilogue GEMM) takes no zero points; the
    reference's quantized_dot with zero points is q8_quantized_dot."""
    fake = C.c_void_p(0x1000)
    rc = lib.load().q8_gemm(fake, fake, 4, 4, 16, 3, 0, None, 0, None, 0, 0, 0.0, None, 0,
                            lib.Q8_I32, fake, None)
    assert rc == lib.Q8_ERR_UNSUPPORTED


def test_quantized_dot_workspace_and_validation(lib):
    """Validation fails before anything is launched."""
    L = lib.load()
    need = C.c_size_t(123)
    # i8 operands without zero points need no workspace
    assert L.q8_quantized_dot_workspace(4, 5, 16, lib.Q8_I8, lib.Q8_I8, 0, 0, C.byref(need)) == lib.Q8_OK
    assert need.value == 0
    # ui8 A: an int8 copy of A (256-aligned) and, for the 128 it shifts by,
    # the row sums of A
    assert L.q8_quantized_dot_workspace(4, 5, 16, lib.Q8_U8, lib.Q8_I8, 0, 0, C.byref(need)) == lib.Q8_OK
    assert need.value == 256 + 256
    # ui8 A with zero point 128: no shift left, only the copy
    assert L.q8_quantized_dot_workspace(4, 5, 16, lib.Q8_U8, lib.Q8_I8, 128, 0, C.byref(need)) == lib.Q8_OK
    assert need.value == 256
    fake = C.c_void_p(0x1000)
    expect_invalid(lib, "q8_quantized_dot_workspace", 4, 5, 16, 7, lib.Q8_I8, 0, 0, C.byref(need))
    expect_invalid(lib, "q8_quantized_dot", fake, 7, fake, lib.Q8_I8, 4, 5, 16, 0, 0, None, 0, fake, None)
    expect_invalid(lib, "q8_quantized_dot", fake, lib.Q8_U8, fake, lib.Q8_I8, 4, 5, 16, 0, 0, fake, 16,
                   fake, None, match="workspace")


def test_python_ops_refuse_cpu_tensors():
    torch = pytest.importorskip("torch")
    from mlfw_amd import ops
    with pytest.raises(ValueError):
        ops.quantize_per_token(torch.zeros(2, 4))
    with pytest.raises(TypeError):
        ops.quantize_per_token(torch.zeros(2, 4, dtype=torch.float64))


def _conv_args(x_shape, w_shape, strides, lo, hi, dil):
    a = lambda v: (C.c_int64 * len(v))(*v)  # noqa: E731
    return a(x_shape), a(w_shape), a(strides), a(lo), a(hi), a(dil)


def test_conv_workspace_query_and_validation(lib):
    L = lib.load()
    need = C.c_size_t(123)
    # the reference's own conv test shape (pass.test.js:255-274): 27-long contraction -> direct kernel
    xs, ws, st, lo, hi, dl = _conv_args([1, 3, 8, 8], [16, 3, 3, 3], [1, 1], [0, 0], [0, 0], [1, 1])
    assert L.q8_quantized_conv_workspace(2, xs, ws, st, lo, hi, dl, 1, C.byref(need)) == lib.Q8_OK
    assert need.value == 0
    # 64 x 3 x 3 contraction -> im2col matrix of 36 positions x 576 bytes
    xs, ws, st, lo, hi, dl = _conv_args([2, 64, 8, 8], [32, 64, 3, 3], [1, 1], [0, 0], [0, 0], [1, 1])
    assert L.q8_quantized_conv_workspace(2, xs, ws, st, lo, hi, dl, 1, C.byref(need)) == lib.Q8_OK
    assert need.value >= 36 * 576
    fake = C.c_void_p(0x1000)
    bad = [
        ([1, 4, 8, 8], [8, 3, 3, 3], 1),      # kernel I != C / groups
        ([1, 4, 8, 8], [6, 2, 3, 3], 4),      # groups does not divide O
        ([1, 4, 2, 2], [8, 4, 3, 3], 1),      # kernel larger than the input
    ]
    for x_shape, w_shape, groups in bad:
        args = _conv_args(x_shape, w_shape, [1, 1], [0, 0], [0, 0], [1, 1])
        expect_invalid(lib, "q8_quantized_conv_workspace", 2, *args, groups, C.byref(need))
        expect_invalid(lib, "q8_quantized_conv", fake, fake, 2, *args, groups, 0, 0, lib.Q8_I32,
                       0.0, fake, 1 << 20, fake, None)
    args = _conv_args([1, 4, 8, 8], [8, 4, 3, 3], [0, 1], [0, 0], [0, 0], [1, 1])   # stride 0
    expect_invalid(lib, "q8_quantized_conv_workspace", 2, *args, 1, C.byref(need))
    args = _conv_args([1, 4, 8, 8], [8, 4, 3, 3], [1, 1], [-1, 0], [0, 0], [1, 1])  # negative pad
    expect_invalid(lib, "q8_quantized_conv_workspace", 2, *args, 1, C.byref(need))
    args = _conv_args([1, 64, 8, 8], [8, 64, 3, 3], [1, 1], [0, 0], [0, 0], [1, 1])
    expect_invalid(lib, "q8_quantized_conv", fake, fake, 2, *args, 1, 0, 0, lib.Q8_I32, 0.0,
                   fake, 16, fake, None, match="workspace")                          # workspace too small
    expect_invalid(lib, "q8_quantized_conv", fake, fake, 4, *args, 1, 0, 0, lib.Q8_I32, 0.0,
                   fake, 1 << 20, fake, None)                                        # rank 4
    expect_invalid(lib, "q8_quantized_conv_ex", fake, 9, fake, lib.Q8_I8, 2, *args, 1, 2, 0, lib.Q8_I32,
                   0.0, fake, 1 << 20, fake, None)                                   # bad operand type


def test_requant_validation(lib):
    fake = C.c_void_p(0x1000)
    L = lib.load()
    # the quantize verifier's scale > 0 (ops/quantization.ts:44-47)
    for s_next in (0.0, -1.0, float("inf"), float("nan")):
        rc = L.q8_gemm_requant(fake, fake, 32, 32, 64, fake, lib.Q8_PER_TOKEN, fake,
                               lib.Q8_PER_CHANNEL, lib.Q8_EPI_ROWCOL, 0.0, None, 0, s_next, fake, None)
        assert rc == lib.Q8_ERR_INVALID, s_next
    rc = L.q8_gemm_requant(fake, fake, 32, 32, 64, None, lib.Q8_PER_TOKEN, fake, lib.Q8_PER_CHANNEL,
                           lib.Q8_EPI_ROWCOL, 0.0, None, 0, 0.1, fake, None)
    assert rc == lib.Q8_ERR_INVALID          # ROWCOL without sA
