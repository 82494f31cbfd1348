"""Error types of the MI355X kernel library.

Mirrors the launch/load part of the reference taxonomy
(triton_metal/errors.py:84-103 ``MetalLaunchError(message, kernel_name, grid,
reason)``; driver.py:141-159 raises ``RuntimeError`` for load failures).  Every
class derives from ``RuntimeError`` like the reference's, so callers that catch
``RuntimeError`` keep working.
"""


class HipLaunchError(RuntimeError):
    """A kernel launch (or a typed op) was rejected or failed on the device."""

    def __init__(self, message, kernel_name=None, grid=None, reason=None, code=None):
        self.kernel_name = kernel_name
        self.grid = grid
        self.reason = reason
        self.code = code
        parts = [message]
        if kernel_name:
            parts.append(f"  kernel: {kernel_name}")
        if grid:
            parts.append(f"  grid: {grid}")
        if reason:
            parts.append(f"  reason: {reason}")
        super().__init__("\n".join(parts))


class KernelLoadError(RuntimeError):
    """A code object or kernel could not be loaded (driver.py:141-159)."""

    def __init__(self, message, code=None):
        self.code = code
        super().__init__(message)


class NativeLibraryMissing(KernelLoadError):
    """libtm_hip.so has not been built (run ``triton_metal_amd.build.build()``)."""


class NoDeviceError(RuntimeError):
    """No usable HIP runtime or GPU."""
