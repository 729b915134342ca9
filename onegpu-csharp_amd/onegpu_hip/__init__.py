"""MI355X (gfx950) int8 quantized-matmul path: the reference's Int8Gemm / DynamicQuantizeKernels / DequantizeKernels
API (recursive-ai-oss/onegpu-csharp, src/RecursiveAI.OneGpu.Kernels) over the C-ABI HIP library libonegpu_hip.so.

The compute runs only in the HIP library; importing fails loudly when the built extension is missing.
"""
import os

from .errors import (GpuCommandFailedException, GpuDeviceLostException, GpuException, GpuKernelIndexException,
                     GpuKernelShapeException, GpuOutOfMemoryException, GpuUnsupportedException)

try:
    from ._onegpu_host import (ConvIntegerKernels, ConvProblem, DequantizeKernels, DynamicQuantizeKernels, ElementType,
                               GatherKernels, GpuBuffer,
                               GpuCommandEncoder, GpuComputeCapabilities, GpuDevice, GpuIndexStatus, Int8Gemm,
                               Int8GemmOptions, Int8GemmProblem, Int8Operand, Int8Ranges, Int8Scratch,
                               OG_RANGES_MAX, version)
except ImportError as e:  # pragma: no cover - a build problem, reported as such
    raise ImportError("onegpu_hip: the native extension is not built; run python onegpu-csharp_amd/build.py "
                      f"(or __graft_entry__.build()) first: {e}") from e

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lib", "libonegpu_hip.so")


def padded_bool_length(count: int) -> int:
    """GpuKernelBuffers.PaddedBoolLength (src/RecursiveAI.OneGpu.Kernels/GpuKernelBuffers.cs:25-30)."""
    if count < 0:
        raise ValueError("count")
    return (count + 3) & ~3


def padded_half_length(count: int) -> int:
    """GpuKernelBuffers.PaddedHalfLength (GpuKernelBuffers.cs:12-17)."""
    if count < 0:
        raise ValueError("count")
    return (count + 1) & ~1


__all__ = ["ConvIntegerKernels", "ConvProblem", "DequantizeKernels", "DynamicQuantizeKernels", "ElementType", "GatherKernels", "GpuIndexStatus",
           "GpuKernelIndexException", "GpuBuffer", "GpuCommandEncoder",
           "GpuComputeCapabilities", "GpuDevice", "Int8Gemm", "Int8GemmOptions", "Int8GemmProblem", "Int8Operand",
           "Int8Ranges", "OG_RANGES_MAX", "Int8Scratch", "GpuException", "GpuKernelShapeException", "GpuUnsupportedException", "GpuOutOfMemoryException",
           "GpuDeviceLostException", "GpuCommandFailedException", "padded_bool_length", "padded_half_length", "LIB_PATH",
           "version"]
