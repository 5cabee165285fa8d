"""MI355X-native EggRoll hot path (HIP kernels for gfx950 behind a C ABI).

Layout:
  csrc/        HIP kernels and the C ABI of libhses.so (include/hses.h)
  _lib.py      ctypes binding (no fallback: calls raise if the library is absent)
  kernels.py   torch-tensor wrappers over the entry points
  noiser.py    the EggRoll noiser API (mirrors hyperscalees-noiser)
  snn.py       SNN-MLP forward and ES step built on the kernels
"""
__version__ = "0.1.0"
