"""MI355X-native (gfx950) routed MoE experts: the ``*_moe_experts`` ops of aymuos15/cernels.

Layout:
  csrc/            hand-written HIP kernels (route, grouped GEMMs, decode GEMV) + the C ABI
  _native.py       ctypes binding of libcernels_moe.so (include/cernels_moe.h)
  ops.py           torch-facing ops with the reference's op names and schemas
  kops/registry/   drop-in loaders with the reference's kernel()/decode_kernel() signatures
  modeling/swaps   instance-level expert-forward swap, as src/modeling/swaps.py
  configs/         seeded synthetic workloads (the benchmark configurations)
"""

__version__ = "0.1.0"
