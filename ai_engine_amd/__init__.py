"""MI355X (gfx950) backend for ai_engine's conv-as-GEMM path.

The product is the HIP library libaih_conv.so (sources in csrc/, C ABI in
include/aih_conv.h); `conv` is its host-side mirror of the reference's op
interface (GemmPwSpec / ConvIgemmSpec / ConvDwSpec / lower_op's Conv arm).
"""
from . import conv  # noqa: F401

__all__ = ["conv"]
