"""MI355X-native quantized-linear hot path of open_rknpu2_lm_infer.

``libhip_matmul.so`` (built from ``csrc/``) exports the reference's rk_npu_*
C ABI for the dynamic-int8-activation W4/W8 linear, the fused SwiGLU, the
fused FFN and the routed MoE FFN, implemented with hand-written gfx950 HIP
kernels. ``npu`` mirrors the reference's Rust op layer over that ABI.
"""
from . import _ffi  # noqa: F401

__all__ = ["_ffi", "npu", "build"]
