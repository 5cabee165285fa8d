"""MI355X-native EggRoll hot path (HIP kernels for gfx950 behind a C ABI).

Layout:
  csrc/        HIP kernels and the C ABI of libhses.so (include/hses.h)
  _lib.py      ctypes binding (no fallback: calls raise if the library is absent)
  kernels.py   torch-tensor wrappers over the entry points (the noiser and
               kernel-launch surface of hyperscalees-noiser / hyperscalees-kernels)
  snn.py       SNN-MLP forward and ES step built on the kernels
  rwkv.py      RWKV-7 TimeMixing / ChannelMixing compositions
  rwkv_lm.py   RWKV-7 LM population forward and ES step
  snn_attention.py  spiking self-attention transformer population forward and ES step
  verify.py    the K-chunk driver's four-path equivalence check
  data.py      IDX/MNIST reader and the batch sampler
  smoke.py     one small ES step on cuda:0 checked against the CPU oracle
  profile_fc1.py, profile_kernels.py  launch targets for rocprofv3 measurements
  build.py     compiles libhses.so in-tree
"""
__version__ = "0.1.0"
