"""mlfw_amd -- MI355X (gfx950) int8 quantized-inference path of mlfw.

The compute lives in libq8hip.so (hand-written HIP kernels behind the C ABI
of include/q8hip.h).  This package is its Python host side:
  _lib       ctypes binding of the C ABI (fails loudly if the library is absent)
  ops        the reference's int8 operators on torch device tensors
  build      hipcc build step (gfx950 only)
"""
__all__ = ["ops", "build"]
