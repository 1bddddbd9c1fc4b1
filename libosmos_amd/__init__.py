"""libosmos MI355X: libosmos's quantized-weight matrix products (the lane's int8 expert products, the fp32 decode
matvec, the int8-MFMA expert matmul, the MoE routing plumbing) as HIP kernels for gfx950, behind the reference's own C
kernel-launch ABI (include/osmos/gpu/*.h). The product is libosmos_mi355x.so; this package builds it (build.py),
binds it for Python callers (capi.py) and generates synthetic workloads (synth.py).
"""
from .capi import lib, LIB_PATH  # noqa: F401
