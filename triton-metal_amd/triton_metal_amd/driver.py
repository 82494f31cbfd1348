"""Code-object loader and launcher: the HIP counterpart of MetalUtils.

``HipUtils.load_binary`` mirrors ``MetalUtils.load_binary``
(triton_metal/backend/driver.py:114-162): it takes a kernel name and a code
object (bytes or a file path) and returns the 5-tuple
``(module, function, n_regs, n_spills, n_max_threads)``.  ``HipUtils.launch``
mirrors ``MetalUtils.launch`` (driver.py:164-227) but runs asynchronously on a
HIP stream: pass ``sync=True`` to wait like the Metal path does by default.

Kernel arguments are marshalled by value: tensors become device pointers,
Python ints 32-bit ints, Python floats 32-bit floats; a ``(value, ctype)``
pair forces a ctypes type (e.g. ``(n, ctypes.c_int64)``).
"""
from __future__ import annotations

import ctypes as C
import os

from . import _lib
from .errors import HipLaunchError, KernelLoadError


class HipUtils:
    """Load code objects and launch their kernels through libtm_hip.so."""

    def __init__(self):
        self._lib = _lib.lib()
        _lib.check(self._lib.tm_init(), "tm_init")

    def load_binary(self, name, kernel, shared_mem=0, device=None):
        if isinstance(kernel, (bytes, bytearray)):
            data = bytes(kernel)
        elif isinstance(kernel, (str, os.PathLike)):
            with open(kernel, "rb") as f:
                data = f.read()
        else:
            raise TypeError("kernel must be code-object bytes or a path")
        buf = C.create_string_buffer(data, len(data))
        mod = C.c_void_p()
        ctx = _device_ctx(device)
        with ctx:
            rc = self._lib.tm_module_load(buf, len(data), C.byref(mod))
            if rc:
                raise KernelLoadError(f"Failed to load code object: {_lib.last_error()}", code=rc)
            fn = C.c_void_p()
            regs, spills, maxt, shm = C.c_int(), C.c_int(), C.c_int(), C.c_int()
            rc = self._lib.tm_module_get_function(mod, name.encode(), C.byref(fn),
                                                  C.byref(regs), C.byref(spills),
                                                  C.byref(maxt), C.byref(shm))
            if rc:
                self._lib.tm_module_unload(mod)
                raise KernelLoadError(f"Kernel '{name}' not found in code object: "
                                      f"{_lib.last_error()}", code=rc)
        return mod, fn, regs.value, spills.value, maxt.value

    def builtin_function(self, name, device=None):
        """A kernel of the library's embedded code objects by name (resolved
        on ``device`` or the current device), for ``launch``."""
        fn = C.c_void_p()
        with _device_ctx(device):
            rc = self._lib.tm_builtin_get_function(name.encode(), C.byref(fn))
        if rc:
            raise KernelLoadError(f"built-in kernel '{name}': {_lib.last_error()}", code=rc)
        return fn

    def unload(self, module):
        _lib.check(self._lib.tm_module_unload(module), "tm_module_unload")

    def launch(self, function, grid, block, args, shared_mem=0, stream=None, sync=False):
        grid = tuple(grid) + (1,) * (3 - len(grid))
        block = tuple(block) + (1,) * (3 - len(block))
        holders = [_marshal(a) for a in args]
        ptrs = (C.c_void_p * max(1, len(holders)))(
            *[C.cast(C.pointer(h), C.c_void_p) for h in holders])
        if stream is None:
            import torch
            stream = torch.cuda.current_stream().cuda_stream
        rc = self._lib.tm_launch(function, *grid, *block, shared_mem, stream, ptrs)
        if rc:
            raise HipLaunchError("Kernel launch failed", grid=grid, reason=_lib.last_error(),
                                 code=rc)
        if sync:
            _lib.check(self._lib.tm_synchronize(stream), "tm_synchronize")


def _device_ctx(device):
    import contextlib
    if device is None:
        return contextlib.nullcontext()
    import torch
    return torch.cuda.device(device)


def _marshal(a):
    try:
        import torch
        if isinstance(a, torch.Tensor):
            return C.c_void_p(a.data_ptr())
    except ImportError:
        pass
    if isinstance(a, tuple) and len(a) == 2 and isinstance(a[1], type):
        return a[1](a[0])
    if a is None:
        return C.c_void_p(0)
    if isinstance(a, bool):
        return C.c_int(int(a))
    if isinstance(a, int):
        return C.c_int(a)
    if isinstance(a, float):
        return C.c_float(a)
    raise TypeError(f"cannot marshal kernel argument of type {type(a).__name__}")
