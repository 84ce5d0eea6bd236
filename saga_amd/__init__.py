"""saga_amd: SAGA + Atop-N decode attention for AMD Instinct MI355X (gfx950).

Layout:
  csrc/        HIP kernels and the C ABI of libsaga_amd.so (include/saga_amd.h)
  _lib.py      ctypes binding of the library
  ops.py       tensor-level operations (one C-ABI call each)
  attention/   the reference's attention package API (attention.py,
               triton_atopn.py) on top of ops
  build.py     hipcc build of libsaga_amd.so
"""
__version__ = "0.1.0"
