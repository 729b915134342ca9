"""The reference's exception types for this path (src/RecursiveAI.OneGpu/GpuDevice.cs:266-396,
src/RecursiveAI.OneGpu.Kernels/GpuKernelShapeException.cs:7-25), raised by the host layer."""


class GpuException(Exception):
    pass


class GpuKernelShapeException(GpuException, ValueError):
    """A shape, stride, offset or size is invalid for the operation; raised before any work is recorded."""

    def __init__(self, operation: str, argument: str, message: str):
        super().__init__(f"{operation}: {argument}: {message}")
        self.Operation = operation
        self.Argument = argument


class GpuUnsupportedException(GpuException):
    def __init__(self, message: str, capability: str = "", expected: str = "", actual: str = ""):
        super().__init__(message)
        self.Capability = capability or None
        self.Expected = expected or None
        self.Actual = actual or None


class GpuOutOfMemoryException(GpuException):
    pass


class GpuDeviceLostException(GpuException):
    pass


class GpuCommandFailedException(GpuException):
    pass


class GpuKernelIndexException(GpuException):
    """An index given to a gather was outside its axis (GpuIndexStatus.cs:66-80)."""

    def __init__(self, operation: str, position: int):
        super().__init__(f"{operation}: the index at position {position} of the indices is outside its axis")
        self.Operation = operation
        self.Position = position
