"""qraf_amd -- MI355X (gfx950) decode hot path for QRAF models.

Q8_0/Q4_0 block-dequant matvec and batched GEMM, ragged paged-KV decode
attention and fused per-token elementwise kernels, hand-written in HIP and
exposed through the C ABI in include/qraf_hip.h.  Importing this package
loads libqraf_hip.so and raises if it is missing: there is no CPU fallback.
"""
from ._lib import F16, F32, Q4_0, Q8_0, HipError, LIB_PATH, lib  # noqa: F401
from . import backend  # noqa: F401

__all__ = ["lib", "LIB_PATH", "HipError", "backend", "F32", "F16", "Q8_0", "Q4_0"]
