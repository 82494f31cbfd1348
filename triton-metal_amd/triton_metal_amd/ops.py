"""Operator surface: the reference's hot-path kernels as calls on torch tensors.

Each ``make_*_kernel`` factory mirrors the reference generator of the same
name in triton_metal/codegen/_msl_templates.py and returns a callable that
takes the buffers in the reference template's buffer order (tensors for
buffers, Python ints/floats for the ``constant`` scalars).  Where the
reference generator returns MSL text to be compiled and dispatched by a
Metal runner, the callable here launches the gfx950 kernel directly on the
current HIP stream of the tensors' device.

All tensors must live on one CUDA (HIP) device.  The native library is the
only execution path: if it is missing or the device is unusable an error is
raised; nothing falls back to the CPU.
"""
from __future__ import annotations

import ctypes as C
import math

import torch

from . import _lib
from ._lib import TM_DT_BF16, TM_DT_F16, TM_DT_F32, TM_DT_NONE, TM_DT_U8

_FLOAT_DT = {torch.float32: TM_DT_F32, torch.float16: TM_DT_F16, torch.bfloat16: TM_DT_BF16}


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def _dt(t: torch.Tensor, what: str) -> int:
    try:
        return _FLOAT_DT[t.dtype]
    except KeyError:
        raise TypeError(f"{what}: unsupported dtype {t.dtype}") from None


def _zdt(z) -> int:
    if z is None:
        return TM_DT_NONE
    if z.dtype == torch.uint8:
        return TM_DT_U8
    return _dt(z, "zeros")


def _device_of(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected a tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise ValueError(f"tensor on {t.device}; the kernels run on a HIP device")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise ValueError("no tensor arguments")
    return dev


def _need_contig(t, what):
    if t is not None and not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")


def _numel_at_least(t, n, what):
    if t.numel() < n:
        raise ValueError(f"{what} holds {t.numel()} elements, needs {n}")


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


class Launch:
    """One validated call of a C-ABI entry point with its arguments bound.

    Calling it launches asynchronously on the stream bound at creation (the
    current stream of the tensors' device then) or on ``stream`` if given.
    The device must be the current HIP device when called."""

    __slots__ = ("_f", "_args", "_what", "dev", "stream", "_keep")

    def __init__(self, f, args, what, dev, stream=None):
        self._f = f
        self._args = args
        self._what = what
        self.dev = dev
        self.stream = _stream(dev) if stream is None else stream
        self._keep = None

    def __call__(self, stream=None):
        rc = self._f(*self._args, self.stream if stream is None else stream)
        if rc:
            _lib.check(rc, self._what, kernel_name=self._what)


def _run(launch: Launch):
    """Launch now, making the tensors' device current if it is not."""
    if launch.dev.index == torch.cuda.current_device():
        launch()
    else:
        with torch.cuda.device(launch.dev):
            launch()


class Kernel:
    """A launched-by-call kernel with the reference template's buffer order."""

    def __init__(self, name, fn, params):
        self.name = name
        self._fn = fn
        self.params = params

    def __call__(self, *args, **kwargs):
        return self._fn(*args, **kwargs)

    def __repr__(self):
        return f"Kernel({self.name}, {self.params})"


# ---------------------------------------------------------------------------
# weight-only quantized matmul (A7, A8)
# ---------------------------------------------------------------------------
def plan_int8_matmul(input, weight, output, scales, zeros, M, N, K, stream=None) -> Launch:
    """Validate and bind an int8_matmul call (see int8_matmul)."""
    if weight.dtype != torch.int8:
        # the kernels read signed bytes (the reference's `device const char*`);
        # uint8 storage of the same bytes must be passed as weight.view(torch.int8)
        raise TypeError(f"weight must be int8, got {weight.dtype}")
    dev = _device_of(input, weight, output, scales, zeros)
    for t, w in ((input, "input"), (weight, "weight"), (output, "output"), (scales, "scales"),
                 (zeros, "zeros")):
        _need_contig(t, w)
    adt = _dt(input, "input")
    if output.dtype != input.dtype:
        raise TypeError("output dtype must equal input dtype")
    _numel_at_least(input, M * K, "input")
    _numel_at_least(weight, N * K, "weight")
    _numel_at_least(output, M * N, "output")
    _numel_at_least(scales, N, "scales")
    if zeros is not None:
        _numel_at_least(zeros, N, "zeros")
    return _wq_launch(8, input, weight, None, output, scales, zeros, M, N, K, 1, adt,
                      _dt(scales, "scales"), _zdt(zeros), "int8_matmul", dev, stream)


def int8_matmul(input, weight, output, scales, zeros, M, N, K):
    """output[M,N] = input[M,K] @ ((weight[N,K] - zeros[N]) * scales[N])^T.

    Buffer order of make_int8_matmul_kernel (_msl_templates.py:2652-2661).
    ``zeros`` may be None (symmetric quantisation)."""
    _run(plan_int8_matmul(input, weight, output, scales, zeros, M, N, K))
    return output


def plan_int4_matmul(input, weight, output, scales, zeros, M, N, K, group_size=128,
                     stream=None) -> Launch:
    """Validate and bind an int4_matmul call (see int4_matmul)."""
    dev = _device_of(input, weight, output, scales, zeros)
    for t, w in ((input, "input"), (weight, "weight"), (output, "output"), (scales, "scales"),
                 (zeros, "zeros")):
        _need_contig(t, w)
    if weight.dtype not in (torch.uint8, torch.int8, torch.int32, torch.uint32):
        raise TypeError(f"weight must hold packed bytes (uint8/int32), got {weight.dtype}")
    if K % 2:
        raise ValueError("K must be even")
    adt = _dt(input, "input")
    if output.dtype != input.dtype:
        raise TypeError("output dtype must equal input dtype")
    ng = (K + group_size - 1) // group_size
    _numel_at_least(input, M * K, "input")
    if weight.numel() * weight.element_size() < N * K // 2:
        raise ValueError("weight holds fewer than N*K/2 bytes")
    _numel_at_least(output, M * N, "output")
    _numel_at_least(scales, N * ng, "scales")
    if zeros is not None:
        _numel_at_least(zeros, N * ng, "zeros")
    return _wq_launch(4, input, weight, None, output, scales, zeros, M, N, K, group_size, adt,
                      _dt(scales, "scales"), _zdt(zeros), "int4_matmul", dev, stream)


def _wq_launch(qbits, input, weight, bias, output, scales, zeros, M, N, K, group_size, adt, sdt,
               zdt, what, dev, stream):
    """Bind a validated weight-only call to tm_wq_matmul_ws with the device
    workspace its plan needs (split-K shapes; none otherwise), allocated here
    from torch's caching allocator and kept alive with the launch."""
    L = _lib.lib()
    ws_bytes = L.tm_wq_workspace_bytes(qbits, _ptr(input), _ptr(weight), _ptr(scales),
                                       _ptr(zeros), M, N, K, group_size, adt, sdt, zdt)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
    args = (qbits, _ptr(input), _ptr(weight), _ptr(bias), _ptr(output), _ptr(scales),
            _ptr(zeros), M, N, K, group_size, adt, sdt, zdt, _ptr(ws), ws_bytes)
    launch = Launch(L.tm_wq_matmul_ws, args, what, dev, stream)
    launch._keep = ws
    return launch


def wq_kernel_for(qbits, M, N, K, group_size=128, act_dtype=torch.float16, scale_dtype=None,
                  zero_dtype=None, align=_lib.TM_WQ_ALIGN_ALL, cu_count=256,
                  max_lds=160 * 1024, with_workspace=True, details=False):
    """Name, grid, block and dynamic LDS bytes of the kernel that an int4 /
    int8 matmul of these sizes and dtypes runs (tm_wq_plan; no device is
    touched).  ``zero_dtype`` is a torch dtype or None (no zero-points);
    ``align`` the TM_WQ_ALIGN_* bits of the call's pointers; the defaults
    describe torch allocations on one MI355X and the Python operators, which
    pass a workspace (``with_workspace=False``: the plain C entry points).
    ``details=True`` returns a dict that adds the split-K slices and the
    workspace bytes."""
    dts = {None: TM_DT_NONE, torch.uint8: _lib.TM_DT_U8, **_FLOAT_DT}
    adt = dts[act_dtype]
    sdt = dts[scale_dtype if scale_dtype is not None else act_dtype]
    name = C.create_string_buffer(64)
    grid, block, lds, splits = C.c_uint(), C.c_uint(), C.c_uint(), C.c_uint()
    ws = C.c_size_t()
    rc = _lib.lib().tm_wq_plan(qbits, M, N, K, group_size, adt, sdt, dts[zero_dtype], align,
                               cu_count, max_lds, int(with_workspace), name, 64, C.byref(grid),
                               C.byref(block), C.byref(lds), C.byref(splits), C.byref(ws))
    _lib.check(rc, "wq_kernel_for")
    if details:
        return dict(name=name.value.decode(), grid=grid.value, block=block.value, lds=lds.value,
                    splits=splits.value, workspace_bytes=ws.value)
    return name.value.decode(), grid.value, block.value, lds.value


def int4_matmul(input, weight, output, scales, zeros, M, N, K, group_size=128):
    """output[M,N] = input[M,K] @ dequant(weight)^T with per-group scale/zero.

    Buffer order of make_int4_matmul_kernel (_msl_templates.py:2704-2713).
    ``weight`` holds [N, K/2] bytes (even k in the low nibble) as uint8, or
    the same bytes as int32/uint32 [N, K/8]; scales/zeros are
    [N, ceil(K/group_size)]; ``zeros`` may be None."""
    _run(plan_int4_matmul(input, weight, output, scales, zeros, M, N, K, group_size))
    return output


def _linear_bias(base, bias, input, N, what, stream):
    """Rebind a validated weight-only matmul launch with a bias (its fused
    nn.Linear form; the bias is argument 3 of tm_wq_matmul_ws)."""
    if bias is not None:
        _device_of(input, bias)
        _need_contig(bias, "bias")
        if bias.dtype != input.dtype:
            raise TypeError("bias dtype must equal input dtype")
        _numel_at_least(bias, N, "bias")
    a = base._args
    launch = Launch(base._f, a[:3] + (_ptr(bias),) + tuple(a[4:]), what, base.dev, stream)
    launch._keep = base._keep
    return launch


def plan_int8_linear(input, weight, bias, output, scales, zeros, M, N, K, stream=None) -> Launch:
    """Validate and bind an int8_linear call (see int8_linear)."""
    base = plan_int8_matmul(input, weight, output, scales, zeros, M, N, K, stream)
    return _linear_bias(base, bias, input, N, "int8_linear", stream)


def int8_linear(input, weight, bias, output, scales, zeros, M, N, K):
    """int8_matmul in nn.Linear form: output = input @ dequant(weight)^T + bias[N].

    The bias (input dtype, None for none) is added to the fp32 sum before the
    output rounding, as make_fused_linear_kernel (_msl_templates.py:4013-4135)
    adds its bias."""
    _run(plan_int8_linear(input, weight, bias, output, scales, zeros, M, N, K))
    return output


def plan_int4_linear(input, weight, bias, output, scales, zeros, M, N, K, group_size=128,
                     stream=None) -> Launch:
    """Validate and bind an int4_linear call (see int4_linear)."""
    base = plan_int4_matmul(input, weight, output, scales, zeros, M, N, K, group_size, stream)
    return _linear_bias(base, bias, input, N, "int4_linear", stream)


def int4_linear(input, weight, bias, output, scales, zeros, M, N, K, group_size=128):
    """int4_matmul in nn.Linear form: output = input @ dequant(weight)^T + bias[N]
    (bias added in fp32 before the output rounding; None for none)."""
    _run(plan_int4_linear(input, weight, bias, output, scales, zeros, M, N, K, group_size))
    return output


def wq_dequant(weight, scales, zeros, N, K, qbits, group_size=128, out_dtype=torch.float16,
               out=None):
    """Dequantised weight tile [N, K] = round((float(q) - z) * s) in out_dtype."""
    dev = _device_of(weight, scales, zeros)
    if out is None:
        out = torch.empty(N, K, dtype=out_dtype, device=dev)
    _need_contig(out, "out")
    args = (_ptr(weight), _ptr(scales), _ptr(zeros), _ptr(out), N, K, group_size, qbits,
            _dt(scales, "scales"), _zdt(zeros), _dt(out, "out"))
    _run(Launch(_lib.lib().tm_wq_dequant, args, "wq_dequant", dev))
    return out


def _repack(awq, qweight, qzeros, scales, group_size, zero_offset, g_idx):
    if qweight.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"qweight must be int32, got {qweight.dtype}")
    if awq:
        K, N = qweight.shape[0], qweight.shape[1] * 8
    else:
        K, N = qweight.shape[0] * 8, qweight.shape[1]
    ng = (K + group_size - 1) // group_size
    if g_idx is not None:
        want = torch.arange(K, device=g_idx.device, dtype=g_idx.dtype) // group_size
        if g_idx.numel() != K or not torch.equal(g_idx, want):
            raise ValueError("act-order checkpoints (a g_idx other than k // group_size) have no "
                             "equivalent in the [N, K/2] layout")
    dev = _device_of(qweight, qzeros, scales)
    for t, w in ((qweight, "qweight"), (qzeros, "qzeros"), (scales, "scales")):
        _need_contig(t, w)
    if qzeros is not None and (qzeros.dtype not in (torch.int32, torch.uint32)
                               or tuple(qzeros.shape) != (ng, N // 8)):
        raise ValueError(f"qzeros must be int32 [{ng}, {N // 8}], got {qzeros.dtype} "
                         f"{tuple(qzeros.shape)}")
    if scales is not None and (scales.element_size() != 2 or tuple(scales.shape) != (ng, N)):
        raise ValueError(f"scales must be 16-bit [{ng}, {N}], got {scales.dtype} "
                         f"{tuple(scales.shape)}")
    weight = torch.empty(N, K // 2, dtype=torch.uint8, device=dev)
    s_out = None if scales is None else torch.empty(N, ng, dtype=scales.dtype, device=dev)
    z_out = None if qzeros is None else torch.empty(N, ng, dtype=torch.uint8, device=dev)
    L = _lib.lib()
    if awq:
        args = (_ptr(qweight), _ptr(qzeros), _ptr(scales), N, K, group_size, _ptr(weight),
                _ptr(s_out), _ptr(z_out))
        _run(Launch(L.tm_wq_repack_awq, args, "wq_repack_awq", dev))
    else:
        args = (_ptr(qweight), _ptr(qzeros), _ptr(scales), N, K, group_size, zero_offset,
                _ptr(weight), _ptr(s_out), _ptr(z_out))
        _run(Launch(L.tm_wq_repack_gptq, args, "wq_repack_gptq", dev))
    return weight, s_out, z_out


def from_gptq(qweight, qzeros, scales, group_size=128, zero_offset=1, g_idx=None):
    """A GPTQ int4 checkpoint (qweight int32 [K/8, N], qzeros int32 [K/G, N/8],
    scales [K/G, N]) in the int4 layout of int4_matmul: returns
    (weight uint8 [N, K/2], scales [N, K/G], zeros uint8 [N, K/G]).
    zero_offset: 1 for the original format (zero-points stored minus one), 0 for
    its v2 variant.  g_idx, if given, must be the trivial k // group_size."""
    return _repack(False, qweight, qzeros, scales, group_size, zero_offset, g_idx)


def from_awq(qweight, qzeros, scales, group_size=128):
    """An AWQ int4 checkpoint (qweight int32 [K, N/8] in AWQ column order,
    qzeros int32 [K/G, N/8], scales [K/G, N]) in the int4 layout of
    int4_matmul: returns (weight uint8 [N, K/2], scales [N, K/G], zeros uint8 [N, K/G])."""
    return _repack(True, qweight, qzeros, scales, group_size, 0, None)


def make_int8_matmul_kernel():
    return Kernel("int8_matmul", int8_matmul, {})


def make_int4_matmul_kernel(group_size=128):
    def run(input, weight, output, scales, zeros, M, N, K):
        return int4_matmul(input, weight, output, scales, zeros, M, N, K, group_size=group_size)
    return Kernel("int4_matmul", run, {"group_size": group_size})


# ---------------------------------------------------------------------------
# dense matmul (A1, A4, fused linear)
# ---------------------------------------------------------------------------
def plan_matmul(A, B, C, M, N, K, stream=None) -> Launch:
    """Validate and bind a matmul call (see matmul)."""
    dev = _device_of(A, B, C)
    for t, w in ((A, "A"), (B, "B"), (C, "C")):
        _need_contig(t, w)
    if A.dtype != B.dtype:
        raise TypeError("A and B must share a dtype")
    _numel_at_least(A, M * K, "A")
    _numel_at_least(B, K * N, "B")
    _numel_at_least(C, M * N, "C")
    idt = _FP8_DT[_TORCH_FP8[A.dtype]] if A.dtype in _TORCH_FP8 else _dt(A, "A")
    args = (_ptr(A), _ptr(B), _ptr(C), M, N, K, K, N, N, idt, _dt(C, "C"))
    return Launch(_lib.lib().tm_matmul, args, "matmul_kernel", dev, stream)


def gemm_kernel_for(M, N, K, lda=None, ldb=None, ldc=None, trans_b=False, bias=False,
                    in_dtype=torch.float16, out_dtype=None, align=_lib.TM_GEMM_ALIGN_ALL):
    """Name, grid and block of the kernel a dense matmul (``trans_b=False``:
    B [K, N], as ``matmul``) or linear (``trans_b=True``: weight [N, K], as
    ``fused_linear``, with or without ``bias``) of these sizes runs
    (tm_gemm_plan; no device is touched).  Leading dimensions default to the
    contiguous ones; ``align`` holds the TM_GEMM_ALIGN_* bits of the call's
    pointers (torch allocations: all)."""
    lda = K if lda is None else lda
    ldb = (K if trans_b else N) if ldb is None else ldb
    ldc = N if ldc is None else ldc
    out_dtype = in_dtype if out_dtype is None else out_dtype
    name = C.create_string_buffer(96)
    grid, block = C.c_uint(), C.c_uint()
    rc = _lib.lib().tm_gemm_plan(M, N, K, lda, ldb, ldc, int(trans_b), int(bias),
                                 _FLOAT_DT[in_dtype], _FLOAT_DT[out_dtype], align, name, 96,
                                 C.byref(grid), C.byref(block))
    _lib.check(rc, "gemm_kernel_for")
    return name.value.decode(), grid.value, block.value


def matmul(A, B, C, M, N, K):
    """C[M,N] = A[M,K] @ B[K,N] (row-major, contiguous), fp32 accumulation.

    Buffer order of make_matmul_kernel (_msl_templates.py:447-585).  The
    output dtype is C's (fp32 output from fp16 inputs gives the
    make_simdgroup_matmul_kernel(dtype="fp16") contract)."""
    _run(plan_matmul(A, B, C, M, N, K))
    return C


_TEMPLATE_DT = {"fp32": torch.float32, "f32": torch.float32, "fp16": torch.float16,
                "f16": torch.float16, "bf16": torch.bfloat16}


def _size_arg(v, dev, what):
    """A size of the device-sizes matmul: a uint32 / int32 device tensor (the
    template's `device const uint*` buffer; its first element is read) or a
    Python int (written to a new one-element device tensor).  Returns the
    tensor and the value when it is known on the host (None otherwise)."""
    if isinstance(v, int):
        if v < 0:
            raise ValueError(f"{what}={v}")
        return torch.tensor([v], dtype=torch.int32, device=dev), v
    if not isinstance(v, torch.Tensor) or v.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"{what} must be an int or a uint32 / int32 device tensor")
    if v.device != dev or v.numel() < 1:
        raise ValueError(f"{what} must be a non-empty tensor on {dev}")
    return v, None


def plan_matmul_device_sizes(A, B, C, M_buf, N_buf, K_buf, max_m=None, max_n=None,
                             group_size=0, stream=None) -> Launch:
    """Validate and bind a matmul whose sizes live in device memory (see
    matmul_device_sizes)."""
    dev = _device_of(A, B, C)
    for t, w in ((A, "A"), (B, "B"), (C, "C")):
        _need_contig(t, w)
    if A.dtype != B.dtype:
        raise TypeError("A and B must share a dtype")
    if C.dtype not in (A.dtype, torch.float32):
        raise TypeError(f"C must be {A.dtype} or float32, got {C.dtype}")
    (mb, m), (nb, n), (kb, k) = (_size_arg(M_buf, dev, "M"), _size_arg(N_buf, dev, "N"),
                                 _size_arg(K_buf, dev, "K"))
    if max_m is None or max_n is None:
        # the capacity is the sizes themselves: read them (a synchronising copy
        # for device tensors)
        m = int(mb[0].item()) if m is None else m
        n = int(nb[0].item()) if n is None else n
        k = int(kb[0].item()) if k is None else k
        max_m = m if max_m is None else max_m
        max_n = n if max_n is None else max_n
    if m is not None and n is not None and k is not None:
        _numel_at_least(A, m * k, "A")
        _numel_at_least(B, k * n, "B")
        _numel_at_least(C, min(m, max_m) * min(n, max_n), "C")
    # the kernel checks the sizes it reads on the device against the buffers'
    # element counts and does nothing when they do not fit
    args = (_ptr(A), _ptr(B), _ptr(C), _ptr(mb), _ptr(nb), _ptr(kb), int(max_m), int(max_n),
            A.numel(), B.numel(), C.numel())
    if group_size:
        f, args = _lib.lib().tm_matmul_swizzled, args + (int(group_size),)
    else:
        f = _lib.lib().tm_matmul_2d
    args += (_dt(A, "A"), _dt(C, "C"))
    launch = Launch(f, args, "matmul_swizzled" if group_size else "matmul_2d", dev, stream)
    launch._keep = (mb, nb, kb)
    return launch


def matmul_device_sizes(A, B, C, M_buf, N_buf, K_buf, max_m=None, max_n=None, group_size=0):
    """C[M,N] = A[M,K] @ B[K,N] with M, N, K read on the device: the buffer
    order of make_matmul_2d_kernel / make_matmul_swizzled_kernel
    (_msl_templates.py:588-781; A, B, C, M_buf, N_buf, K_buf, row-major with
    leading dimensions K, N, N).  The sizes are one-element uint32 / int32
    device tensors or ints.  max_m / max_n bound the launch's grid (M and N
    read on the device are clamped to them); left out, they are the sizes
    themselves, read with one synchronising copy.  Sizes on the device whose
    M K, K N or M N exceed A's, B's or C's elements make the launch do
    nothing.  group_size 0 walks the output tiles on a 2-D grid, > 0 in runs of
    that many tile rows (the swizzled template's grouped order).  fp32
    accumulation; C is A's dtype or float32."""
    _run(plan_matmul_device_sizes(A, B, C, M_buf, N_buf, K_buf, max_m, max_n, group_size))
    return C


def _check_template_dtype(A, dtype):
    want = _TEMPLATE_DT.get(dtype)
    if want is None:
        raise ValueError(f"dtype must be one of {sorted(_TEMPLATE_DT)}, got {dtype!r}")
    if A.dtype != want:
        raise TypeError(f"kernel built for {dtype}, got {A.dtype} inputs")


def make_matmul_2d_kernel(block_m=32, block_n=32, block_k=32, dtype="fp32"):
    """The 2-D-dispatch matmul template (_msl_templates.py:588-679): call with
    (A, B, C, M_buf, N_buf, K_buf[, max_m, max_n]).  Tile sizes are the
    library's; the arguments are kept for the reference signature."""
    def run(A, B, C, M_buf, N_buf, K_buf, max_m=None, max_n=None):
        _check_template_dtype(A, dtype)
        return matmul_device_sizes(A, B, C, M_buf, N_buf, K_buf, max_m, max_n, 0)
    return Kernel("matmul_2d", run, {"dtype": dtype})


def make_matmul_swizzled_kernel(block_m=32, block_n=32, block_k=32, group_size=4,
                                dtype="fp32"):
    """The grouped-order matmul template (_msl_templates.py:682-781): call with
    (A, B, C, M_buf, N_buf, K_buf[, max_m, max_n]); runs of group_size tile
    rows.  Tile sizes are the library's."""
    if group_size <= 0:
        raise ValueError(f"group_size must be positive, got {group_size}")

    def run(A, B, C, M_buf, N_buf, K_buf, max_m=None, max_n=None):
        _check_template_dtype(A, dtype)
        return matmul_device_sizes(A, B, C, M_buf, N_buf, K_buf, max_m, max_n, group_size)
    return Kernel("matmul_swizzled", run, {"dtype": dtype, "group_size": group_size})


def fused_linear(input, weight, C, bias, M, N, K):
    """C[M,N] = input[M,K] @ weight[N,K]^T (+ bias[N]).

    Buffer order of make_fused_linear_kernel (_msl_templates.py:4013-4135)
    with ``bias`` None for has_bias=False."""
    dev = _device_of(input, weight, C, bias)
    for t, w in ((input, "input"), (weight, "weight"), (C, "C"), (bias, "bias")):
        _need_contig(t, w)
    if input.dtype != weight.dtype or (bias is not None and bias.dtype != input.dtype):
        raise TypeError("input, weight and bias must share a dtype")
    _numel_at_least(input, M * K, "input")
    _numel_at_least(weight, N * K, "weight")
    _numel_at_least(C, M * N, "C")
    if bias is not None:
        _numel_at_least(bias, N, "bias")
    args = (_ptr(input), _ptr(weight), _ptr(bias), _ptr(C), M, N, K, _dt(input, "input"),
            _dt(C, "C"))
    _run(Launch(_lib.lib().tm_linear, args, "fused_linear", dev))
    return C


# tl.dot in general form (A2): strides, batches, FP8, epilogues
_FP8_DT = {"fp8e4nv": _lib.TM_DT_FP8_E4M3, "fp8e5": _lib.TM_DT_FP8_E5M2,
           "fp8e4b15": _lib.TM_DT_FP8_E4M3B15, "fp8e4b8": _lib.TM_DT_FP8_E4M3B8,
           "fp8e5b16": _lib.TM_DT_FP8_E5M2B16}
_TORCH_FP8 = {torch.float8_e4m3fn: "fp8e4nv", torch.float8_e5m2: "fp8e5"}
DOT_EPILOGUES = {"none": _lib.TM_EPI_NONE, "add-matrix": _lib.TM_EPI_ADD_MATRIX,
                 "add-rows": _lib.TM_EPI_ADD_ROWS, "add-cols": _lib.TM_EPI_ADD_COLS,
                 "softmax": _lib.TM_EPI_SOFTMAX, "chain-dot": _lib.TM_EPI_CHAIN_DOT}


def _in_dt(t, what, fp8_format):
    """dtype code of a dot operand: float tensors by dtype, torch's FP8 dtypes
    by name, raw uint8 codes by the Triton FP8 format name given."""
    if t.dtype in _FLOAT_DT:
        return _FLOAT_DT[t.dtype]
    if t.dtype in _TORCH_FP8:
        return _FP8_DT[_TORCH_FP8[t.dtype]]
    if t.dtype == torch.uint8 and fp8_format is not None:
        try:
            return _FP8_DT[fp8_format]
        except KeyError:
            raise ValueError(f"unknown FP8 format {fp8_format!r}; one of {sorted(_FP8_DT)}") from None
    raise TypeError(f"{what}: unsupported dtype {t.dtype} (uint8 FP8 codes need fp8_format=)")


def _bmk(t, what):
    """(batch, d0, d1) sizes and element strides of a 2-D or 3-D view."""
    if t.dim() == 2:
        return (1,) + tuple(t.shape), (0,) + tuple(t.stride())
    if t.dim() == 3:
        return tuple(t.shape), tuple(t.stride())
    raise ValueError(f"{what} must be 2-D or 3-D, got {t.dim()}-D")


def plan_dot(a, b, c, epilogue="none", z=None, w=None, fp8_format=None, stream=None) -> Launch:
    """Validate and bind one tl.dot (see dot)."""
    if epilogue not in DOT_EPILOGUES:
        raise ValueError(f"epilogue must be one of {sorted(DOT_EPILOGUES)}, got {epilogue!r}")
    dev = _device_of(a, b, c, z, w)
    (ba, M, K), sa = _bmk(a, "a")
    (bb, K2, N), sb = _bmk(b, "b")
    (bc, Mc, Nc), sc = _bmk(c, "c")
    if K2 != K or Mc != M:
        raise ValueError(f"shapes {tuple(a.shape)} @ {tuple(b.shape)} -> {tuple(c.shape)}")
    batch = max(ba, bb, bc)
    for nb, what in ((ba, "a"), (bb, "b"), (bc, "c")):
        if nb not in (1, batch) or (nb == 1 and what == "c" and batch > 1):
            raise ValueError(f"{what}: batch {nb} does not match {batch}")
    # an operand with batch 1 is broadcast over the batch: its batch stride is
    # zero whether it is a 2-D view or a 3-D [1, ., .] view
    if ba == 1:
        sa = (0,) + sa[1:]
    if bb == 1:
        sb = (0,) + sb[1:]
    idt = _in_dt(a, "a", fp8_format)
    if _in_dt(b, "b", fp8_format) != idt:
        raise TypeError("a and b must share a dtype")
    L = 0
    sw = (0, 0)
    wdt = TM_DT_NONE
    if epilogue == "chain-dot":
        if w is None or w.dim() != 2 or w.shape[0] != N:
            raise ValueError(f"chain-dot needs w [N={N}, L]")
        L = w.shape[1]
        sw = tuple(w.stride())
        wdt = _in_dt(w, "w", fp8_format)
        if Nc != L:
            raise ValueError(f"chain-dot output must be [.., M, L={L}], got {tuple(c.shape)}")
    elif Nc != N:
        raise ValueError(f"c must be [.., {M}, {N}], got {tuple(c.shape)}")
    sz = (0, 0, 0)
    zdt = TM_DT_NONE
    if epilogue.startswith("add-"):
        if z is None:
            raise ValueError(f"{epilogue} needs z")
        (bz, Mz, Nz), sz = _bmk(z, "z")
        need = {"add-matrix": (M, N), "add-rows": (M, 1), "add-cols": (1, N)}[epilogue]
        if Mz < need[0] or Nz < need[1] or bz not in (1, batch):
            raise ValueError(f"z of shape {tuple(z.shape)} too small for {epilogue}")
        if bz == 1:
            sz = (0,) + tuple(sz[1:])
        zdt = _in_dt(z, "z", fp8_format)
    strides = (C.c_longlong * 14)(*sa, *sb, *sc, *sz, *sw)
    args = (_ptr(a), _ptr(b), _ptr(c), _ptr(z), _ptr(w), batch, M, N, K, L, strides,
            DOT_EPILOGUES[epilogue], idt, _dt(c, "c"), zdt, wdt)
    launch = Launch(_lib.lib().tm_dot, args, "dot", dev, stream)
    launch._keep = strides
    return launch


def dot(a, b, c, epilogue="none", z=None, w=None, fp8_format=None):
    """c = epilogue(a @ b) for 2-D ([M, K] @ [K, N]) or batched 3-D views with
    any element strides (transposed and column-major views included), the
    strided tl.dot template of _lowerer_templates.py:1116-1540:
      "none", "add-matrix" (+ z[.., m, n]), "add-rows" (+ z[.., m, 0]),
      "add-cols" (+ z[.., 0, n]), "softmax" (over n), "chain-dot" ((a @ b) @ w,
      w [N, L], c [.., M, L]).
    Inputs fp16 / bf16 / fp32, torch.float8_e4m3fn / float8_e5m2, or uint8
    FP8 codes with fp8_format one of "fp8e4nv", "fp8e5", "fp8e4b15", "fp8e4b8",
    "fp8e5b16"; fp32 accumulation; c's dtype is the output dtype.  z may be c
    itself (the reference reads the bias from the output buffer)."""
    _run(plan_dot(a, b, c, epilogue, z, w, fp8_format))
    return c


def make_matmul_kernel(block_m=32, block_n=32, block_k=32, dtype="fp32"):
    """Tile sizes are chosen by the library; the arguments are kept for the
    reference signature (_msl_templates.py:447)."""
    return Kernel("matmul_kernel", matmul, {"dtype": dtype})


def make_simdgroup_matmul_kernel(dtype="fp32"):
    if dtype not in ("fp32", "f32", "fp16", "f16"):
        raise ValueError(f"simdgroup_matmul supports fp32 and fp16, got {dtype}")
    return Kernel("simdgroup_matmul", matmul, {"dtype": dtype})


def make_fused_linear_kernel(has_bias=True):
    if has_bias:
        return Kernel("fused_linear", fused_linear, {"has_bias": True})

    def run(input, weight, C, M, N, K):
        return fused_linear(input, weight, C, None, M, N, K)
    return Kernel("fused_linear", run, {"has_bias": False})


# ---------------------------------------------------------------------------
# flash attention forward (A9, A10)
# ---------------------------------------------------------------------------
def _bhsd_strides(t, what):
    if t.dim() != 4:
        raise ValueError(f"{what} must be [B, H, S, D]")
    if t.stride(3) != 1:
        raise ValueError(f"{what}: the head dimension must be contiguous")
    return list(t.stride()[:3])


def plan_flash_attention(q, k, v, o, lse=None, causal=False, scale=None,
                         stream=None) -> Launch:
    """Validate and bind a flash attention forward on [B, H, S, D] views.

    ``lse`` (optional) is fp32 [B, H, S] contiguous.  ``scale`` defaults to
    1/sqrt(D)."""
    dev = _device_of(q, k, v, o, lse)
    if not (q.shape == k.shape == v.shape == o.shape):
        raise ValueError(f"shape mismatch: {q.shape} {k.shape} {v.shape} {o.shape}")
    if not (q.dtype == k.dtype == v.dtype == o.dtype):
        raise TypeError("q, k, v and o must share a dtype")
    B, H, S, D = q.shape
    if lse is not None:
        if lse.dtype != torch.float32 or not lse.is_contiguous() or lse.numel() < B * H * S:
            raise ValueError("lse must be a contiguous fp32 tensor of B*H*S elements")
    st = (_bhsd_strides(q, "q") + _bhsd_strides(k, "k") + _bhsd_strides(v, "v")
          + _bhsd_strides(o, "o"))
    strides = (C.c_longlong * 12)(*st)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), B, H, S, D, strides, float(scale),
            1 if causal else 0, _dt(q, "q"))
    launch = Launch(_lib.lib().tm_flash_attention, args, "flash_attention", dev, stream)
    launch._keep = strides
    return launch


def attention(q, k, v, causal=False, scale=None, return_lse=False):
    """Allocate O (and LSE) and run flash attention on [B, H, S, D] tensors."""
    o = torch.empty_like(q, memory_format=torch.contiguous_format)
    lse = None
    if return_lse:
        B, H, S, _ = q.shape
        lse = torch.empty(B, H, S, dtype=torch.float32, device=q.device)
    _run(plan_flash_attention(q, k, v, o, lse, causal, scale))
    return (o, lse) if return_lse else o


def flash_attention(Q, K, V, O, seq_len, scale, causal=False, lse=None):
    """Buffer order of make_flash_attention_kernel (_msl_templates.py:1624-1634):
    Q, K, V, O are [n_heads * seq_len, head_dim] contiguous."""
    D = Q.shape[-1]
    views = [t.reshape(1, -1, seq_len, D) for t in (Q, K, V, O)]
    _run(plan_flash_attention(*views, lse=lse, causal=causal, scale=scale))
    return O


def flash_attn_fwd(Q, K, V, Out,
                   stride_qz, stride_qh, stride_qm, stride_qk,
                   stride_kz, stride_kh, stride_kn, stride_kk,
                   stride_vz, stride_vh, stride_vn, stride_vk,
                   stride_oz, stride_oh, stride_om, stride_ok,
                   Z, H, N_CTX, BLOCK_M=None, BLOCK_N=None, HEAD_DIM=None, IS_CAUSAL=False,
                   lse=None):
    """The signature of the @triton.jit _flash_attn_fwd kernel
    (tests/test_flash_attention.py:24-33); softmax scale 1/sqrt(HEAD_DIM)
    (line 54).  BLOCK_M / BLOCK_N are accepted for signature compatibility;
    the library picks its own tiles."""
    D = HEAD_DIM if HEAD_DIM is not None else Q.shape[-1]

    def view(t, sz, sh, sm, sk):
        return torch.as_strided(t, (Z, H, N_CTX, D), (sz, sh, sm, sk), t.storage_offset())

    q = view(Q, stride_qz, stride_qh, stride_qm, stride_qk)
    k = view(K, stride_kz, stride_kh, stride_kn, stride_kk)
    v = view(V, stride_vz, stride_vh, stride_vn, stride_vk)
    o = view(Out, stride_oz, stride_oh, stride_om, stride_ok)
    _attention_any_strides(q, k, v, o, 1.0 / math.sqrt(D), IS_CAUSAL, lse)
    return Out


def _attention_any_strides(q, k, v, o, scale, causal, lse=None):
    """Flash attention on [B, H, S, D] views whose head dimension may be
    strided: the kernels read rows of contiguous head elements, so a view with
    a head-dimension stride other than 1 goes through a contiguous device
    copy (and the output comes back through a strided device copy)."""
    qc, kc, vc = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
    if o.stride(-1) == 1:
        _run(plan_flash_attention(qc, kc, vc, o, lse=lse, causal=causal, scale=scale))
    else:
        oc = torch.empty(o.shape, dtype=o.dtype, device=o.device)
        _run(plan_flash_attention(qc, kc, vc, oc, lse=lse, causal=causal, scale=scale))
        o.copy_(oc)
    return o


def fa_fwd_strided(Q, K, V, Out, stride_qm, stride_qk, stride_kn, stride_kk, stride_vn,
                   stride_vk, stride_om, stride_ok, sm_scale, N_CTX, HEAD_DIM, BLOCK_M=None,
                   BLOCK_N=None):
    """The signature of the reference's second FlashAttention kernel,
    _fa_fwd_strided_kernel (tests/test_cpp_backend.py:567-576): one head of
    N_CTX queries and keys, [N_CTX, HEAD_DIM] with a row and a head-dimension
    stride per tensor, softmax scale sm_scale, no causal mask.  BLOCK_M /
    BLOCK_N are accepted for the signature; the library picks its own tiles."""
    D = HEAD_DIM

    def view(t, sm, sk):
        return torch.as_strided(t, (1, 1, N_CTX, D), (0, 0, sm, sk), t.storage_offset())

    _attention_any_strides(view(Q, stride_qm, stride_qk), view(K, stride_kn, stride_kk),
                           view(V, stride_vn, stride_vk), view(Out, stride_om, stride_ok),
                           float(sm_scale), False)
    return Out


def make_flash_attention_kernel(head_dim=64, Br=16, Bc=16, block_size=256, causal=False):
    """Returns a callable with the template's buffer order (Q, K, V, O,
    seq_len, scale); Br/Bc/block_size are accepted for the reference
    signature (_msl_templates.py:1568), the library chooses its own tiles."""
    def run(Q, K, V, O, seq_len, scale, lse=None):
        if Q.shape[-1] != head_dim:
            raise ValueError(f"kernel built for head_dim={head_dim}, got {Q.shape[-1]}")
        return flash_attention(Q, K, V, O, seq_len, scale, causal=causal, lse=lse)
    return Kernel("flash_attention", run, {"head_dim": head_dim, "causal": causal})


# ---------------------------------------------------------------------------
# decode attention (one query token per head over a KV cache)
# ---------------------------------------------------------------------------
def plan_decode_attention(q, k_cache, v_cache, o, seq_lens=None, seq_len=None, page_table=None,
                          scale=None, lse=None, workspace=None, stream=None) -> Launch:
    """Validate and bind one decode-attention call (see decode_attention)."""
    dev = _device_of(q, k_cache, v_cache, o, seq_lens, page_table, lse, workspace)
    if q.dim() != 3 or o.shape != q.shape:
        raise ValueError(f"q and o must be [B, Hq, D]: {tuple(q.shape)} {tuple(o.shape)}")
    B, Hq, D = q.shape
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must share shape and strides")
    if k_cache.dtype != v_cache.dtype:
        raise TypeError("k_cache and v_cache must share a dtype")
    if k_cache.dim() != 4 or k_cache.shape[-1] != D or k_cache.stride(-1) != 1:
        raise ValueError("the cache must be 4-D with a contiguous head dim equal to q's")
    for t, w in ((q, "q"), (o, "o"), (seq_lens, "seq_lens"), (page_table, "page_table"),
                 (lse, "lse")):
        _need_contig(t, w)
    if page_table is not None:
        # [pages, page_size, Hkv, D]
        npages, page_size, Hkv = k_cache.shape[:3]
        if page_table.dtype != torch.int32 or page_table.dim() != 2 or page_table.shape[0] != B:
            raise ValueError("page_table must be int32 [B, max_pages]")
        max_pages = page_table.shape[1]
        strides = (k_cache.stride(0), k_cache.stride(2), k_cache.stride(1))
        cap = page_size * max_pages
    else:
        # [B, Hkv, S, D]
        if k_cache.shape[0] != B:
            raise ValueError(f"cache batch {k_cache.shape[0]} != q batch {B}")
        Hkv, cap = k_cache.shape[1], k_cache.shape[2]
        page_size, max_pages = 0, 0
        strides = (k_cache.stride(0), k_cache.stride(1), k_cache.stride(2))
    if Hq % Hkv:
        raise ValueError(f"q heads {Hq} not a multiple of kv heads {Hkv}")
    if seq_len is None:
        seq_len = cap
    if seq_len > cap:
        raise ValueError(f"seq_len {seq_len} exceeds the cache's {cap} positions")
    if seq_lens is not None and (seq_lens.dtype != torch.int32 or seq_lens.shape != (B,)):
        raise ValueError("seq_lens must be int32 [B]")
    if lse is not None and (lse.dtype != torch.float32 or lse.shape != (B, Hq)):
        raise ValueError("lse must be fp32 [B, Hq]")
    if scale is None:
        scale = D ** -0.5
    need = _lib.lib().tm_decode_attention_workspace_size(B, Hq, Hkv, D, seq_len,
                                                         page_size if page_table is not None else 0)
    if workspace is None and need > 0:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    wbytes = 0 if workspace is None else workspace.numel() * workspace.element_size()
    st = (C.c_longlong * 3)(*strides)
    args = (_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(o), _ptr(lse), B, Hq, Hkv, D,
            _ptr(seq_lens), int(seq_len), st, _ptr(page_table), page_size, max_pages,
            float(scale), _dt(q, "q"), _dt(k_cache, "k_cache"), _dt(o, "o"), _ptr(workspace),
            wbytes)
    launch = Launch(_lib.lib().tm_decode_attention, args, "decode_attention", dev, stream)
    launch._keep = (st, workspace)
    return launch


def decode_attention(q, k_cache, v_cache, seq_lens=None, seq_len=None, page_table=None,
                     scale=None, o=None, lse=None):
    """Attention of one query token per (batch, head) over a KV cache.

    q [B, Hq, D]; cache [B, Hkv, S, D] (any strides, contiguous D), or paged
    [pages, page_size, Hkv, D] with page_table int32 [B, max_pages];
    seq_lens int32 [B] (positions per batch entry) or None for seq_len (default:
    the cache's capacity) everywhere.  Query head h reads KV head
    h // (Hq // Hkv).  scale defaults to D**-0.5.  Returns o (q's dtype unless
    given)."""
    if o is None:
        o = torch.empty_like(q)
    _run(plan_decode_attention(q, k_cache, v_cache, o, seq_lens=seq_lens, seq_len=seq_len,
                               page_table=page_table, scale=scale, lse=lse))
    return o


# Wrappers with the buffer orders of the reference's decode templates.
def kv_cache_attention(Q, K_cache, V_cache, O, seq_len, scale):
    """make_kv_cache_attention_kernel (_msl_templates.py:1949-2048): Q, O
    [n_heads, D]; K_cache, V_cache hold [n_heads, seq_len, D] in their first
    n_heads * seq_len * D elements: head h starts at element h * seq_len * D
    (head_offset_kv = pid * seq_len * D, line 1988), whatever capacity the
    buffers have beyond that."""
    H, D = Q.shape
    n = H * seq_len * D
    kc = K_cache.reshape(-1)[:n].view(1, H, seq_len, D)
    vc = V_cache.reshape(-1)[:n].view(1, H, seq_len, D)
    decode_attention(Q.unsqueeze(0), kc, vc, seq_len=seq_len, scale=scale, o=O.view(1, H, D))
    return O


def gqa_attention(Q, K_cache, V_cache, O, seq_len, scale, n_q_per_kv):
    """make_gqa_attention_kernel (_msl_templates.py:2049-2160): Q, O
    [n_q_heads, D]; K_cache, V_cache hold [n_kv_heads, seq_len, D] in their
    first elements, n_kv_heads = n_q_heads / n_q_per_kv (KV head h starts at
    element h * seq_len * D); query head h reads KV head h // n_q_per_kv."""
    Hq, D = Q.shape
    if n_q_per_kv <= 0 or Hq % n_q_per_kv:
        raise ValueError(f"n_q_per_kv={n_q_per_kv} does not divide {Hq} query heads")
    Hkv = Hq // n_q_per_kv
    n = Hkv * seq_len * D
    kc = K_cache.reshape(-1)[:n].view(1, Hkv, seq_len, D)
    vc = V_cache.reshape(-1)[:n].view(1, Hkv, seq_len, D)
    decode_attention(Q.unsqueeze(0), kc, vc, seq_len=seq_len, scale=scale, o=O.view(1, Hq, D))
    return O


def batched_kv_decode(Q, K_cache, V_cache, O, seq_lens, max_seq_len, batch_size=None):
    """make_batched_kv_decode_kernel (_msl_templates.py:2161-2278): Q, O
    [batch, n_heads, D]; caches [batch, n_heads, max_seq_len, D]; seq_lens
    int32 [batch]; scale 1/sqrt(D)."""
    B, H, D = Q.shape
    if batch_size is not None and batch_size != B:
        raise ValueError(f"batch_size={batch_size} but Q has {B} entries")
    kc = K_cache.reshape(B, H, max_seq_len, D)
    vc = V_cache.reshape(B, H, max_seq_len, D)
    decode_attention(Q, kc, vc, seq_lens=seq_lens.to(torch.int32), seq_len=max_seq_len,
                     scale=D ** -0.5, o=O)
    return O


def multi_head_paged_attention(Q, K_pages, V_pages, page_table, O, seq_len, n_pages,
                               page_size=16):
    """make_multi_head_paged_attention_kernel (_msl_templates.py:2405-2532):
    Q, O [n_heads, D]; pages [n_physical_pages, page_size, n_heads, D];
    page_table [>= n_pages] (logical -> physical); scale 1/sqrt(D)."""
    H, D = Q.shape
    kp = K_pages.reshape(-1, page_size, H, D)
    vp = V_pages.reshape(-1, page_size, H, D)
    pt = page_table[:n_pages].to(torch.int32).reshape(1, n_pages).contiguous()
    decode_attention(Q.unsqueeze(0), kp, vp, seq_len=seq_len, page_table=pt, scale=D ** -0.5,
                     o=O.view(1, H, D))
    return O


def paged_attention(Q, K_pages, V_pages, page_table, O, seq_len, n_pages, page_size=16):
    """make_paged_attention_kernel (_msl_templates.py:2279-2404): one head;
    Q, O [D]; pages [n_physical_pages, page_size, D]."""
    D = Q.shape[-1]
    multi_head_paged_attention(Q.reshape(1, D), K_pages.reshape(-1, page_size, 1, D),
                               V_pages.reshape(-1, page_size, 1, D), page_table,
                               O.view(1, D), seq_len, n_pages, page_size)
    return O


def fp16_kv_attention(Q, K_cache, V_cache, O, seq_len):
    """make_fp16_kv_attention_kernel (_msl_templates.py:2533-2629): Q, O fp32
    [D]; K_cache, V_cache fp16 [>= seq_len, D]; scale 1/sqrt(D)."""
    D = Q.shape[-1]
    kc = K_cache.reshape(1, 1, -1, D)
    vc = V_cache.reshape(1, 1, -1, D)
    decode_attention(Q.reshape(1, 1, D), kc, vc, seq_len=seq_len, scale=D ** -0.5,
                     o=O.view(1, 1, D))
    return O


def make_kv_cache_attention_kernel(head_dim=64, block_size=256):
    def run(Q, K_cache, V_cache, O, seq_len, scale):
        return kv_cache_attention(Q, K_cache, V_cache, O, seq_len, scale)
    return Kernel("kv_cache_attention", run, {"head_dim": head_dim})


def make_gqa_attention_kernel(head_dim=64, n_q_per_kv=4, block_size=256):
    def run(Q, K_cache, V_cache, O, seq_len, scale):
        return gqa_attention(Q, K_cache, V_cache, O, seq_len, scale, n_q_per_kv)
    return Kernel("gqa_attention", run, {"head_dim": head_dim, "n_q_per_kv": n_q_per_kv})


def make_batched_kv_decode_kernel(n_heads=8, head_dim=64, block_size=256):
    def run(Q, K_cache, V_cache, O, seq_lens, max_seq_len, batch_size):
        return batched_kv_decode(Q, K_cache, V_cache, O, seq_lens, max_seq_len, batch_size)
    return Kernel("batched_kv_decode", run, {"n_heads": n_heads, "head_dim": head_dim})


def make_paged_attention_kernel(head_dim=64, page_size=16, block_size=256):
    def run(Q, K_pages, V_pages, page_table, O, seq_len, n_pages):
        return paged_attention(Q, K_pages, V_pages, page_table, O, seq_len, n_pages, page_size)
    return Kernel("paged_attention", run, {"head_dim": head_dim, "page_size": page_size})


def make_multi_head_paged_attention_kernel(n_heads=8, head_dim=64, page_size=16, block_size=256):
    def run(Q, K_pages, V_pages, page_table, O, seq_len, n_pages):
        return multi_head_paged_attention(Q, K_pages, V_pages, page_table, O, seq_len, n_pages,
                                          page_size)
    return Kernel("multi_head_paged_attention", run,
                  {"n_heads": n_heads, "head_dim": head_dim, "page_size": page_size})


def make_fp16_kv_attention_kernel(head_dim=64, block_size=256):
    def run(Q, K_cache, V_cache, O, seq_len):
        return fp16_kv_attention(Q, K_cache, V_cache, O, seq_len)
    return Kernel("fp16_kv_attention", run, {"head_dim": head_dim})


# ---------------------------------------------------------------------------
# KDA chunked forward (no counterpart in the reference)
# ---------------------------------------------------------------------------
KDA_KEY_DIM = KDA_VALUE_DIM = 128
KDA_CHUNK = 64


def kda_workspace_size(batch, seq_len, heads, key_dim=KDA_KEY_DIM, value_dim=KDA_VALUE_DIM,
                       chunk_size=KDA_CHUNK) -> int:
    """Bytes of device workspace tm_kda_chunk_fwd needs (0 = unsupported shape)."""
    return int(_lib.lib().tm_kda_workspace_size(batch, seq_len, heads, key_dim, value_dim,
                                                chunk_size))


def _kda_check(q, k, v, g, beta, o, initial_state, final_state, extra=None):
    """Shared argument checks of the KDA operators; returns (dev, B, T, H, K, V)."""
    dev = _device_of(q, k, v, g, beta, o, initial_state, final_state, extra)
    if q.dim() != 4 or k.shape != q.shape or g.shape != q.shape:
        raise ValueError(f"q, k, g must share a [B, T, H, K] shape: {q.shape} {k.shape} {g.shape}")
    B, T, H, Dk = q.shape
    if v.dim() != 4 or v.shape[:3] != q.shape[:3] or o.shape != v.shape:
        raise ValueError(f"v and o must be [B, T, H, V]: {v.shape} {o.shape}")
    Dv = v.shape[3]
    if beta.shape != (B, T, H):
        raise ValueError(f"beta must be [B, T, H], got {tuple(beta.shape)}")
    for t, name in ((q, "q"), (k, "k"), (v, "v"), (o, "o")):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
    if g.dtype != torch.float32:
        raise TypeError(f"g must be float32, got {g.dtype}")
    if beta.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"beta must be float32 or bfloat16, got {beta.dtype}")
    for t, name in ((initial_state, "initial_state"), (final_state, "final_state")):
        if t is not None and (t.dtype != torch.float32 or tuple(t.shape) != (B, H, Dk, Dv)):
            raise ValueError(f"{name} must be fp32 [B, H, K, V] = {(B, H, Dk, Dv)}")
    for t, name in ((q, "q"), (k, "k"), (v, "v"), (g, "g"), (beta, "beta"), (o, "o"),
                    (initial_state, "initial_state"), (final_state, "final_state")):
        _need_contig(t, name)
    return dev, B, T, H, Dk, Dv


def plan_chunk_kda(q, k, v, g, beta, o, scale=None, initial_state=None, final_state=None,
                   workspace=None, chunk_size=KDA_CHUNK, stream=None) -> Launch:
    """Validate and bind one KDA chunked forward.

    q, k: bf16 [B, T, H, 128]; v, o: bf16 [B, T, H, 128]; g: fp32 [B, T, H, 128]
    (log decay); beta: fp32 or bf16 [B, T, H]; initial_state / final_state:
    fp32 [B, H, 128, 128] or None; workspace: a uint8 device tensor of at least
    kda_workspace_size(B, T, H) bytes (allocated here when None)."""
    dev, B, T, H, Dk, Dv = _kda_check(q, k, v, g, beta, o, initial_state, final_state,
                                      workspace)
    need = _lib.lib().tm_kda_workspace_size(B, T, H, Dk, Dv, chunk_size)
    if need == 0 and B * T * H > 0:
        raise ValueError(f"unsupported KDA shape: key_dim={Dk} value_dim={Dv} "
                         f"chunk_size={chunk_size} (supported: 128, 128, 64)")
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} "
                         f"bytes, needs {need}")
    if scale is None:
        scale = Dk ** -0.5
    bdt = TM_DT_BF16 if beta.dtype == torch.bfloat16 else TM_DT_F32
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(initial_state), _ptr(o),
            _ptr(final_state), B, T, H, Dk, Dv, chunk_size, float(scale), bdt, _ptr(workspace),
            workspace.numel() * workspace.element_size())
    launch = Launch(_lib.lib().tm_kda_chunk_fwd, args, "kda_chunk_fwd", dev, stream)
    launch._keep = workspace
    return launch


def plan_fused_recurrent_kda(q, k, v, g, beta, o, scale=None, initial_state=None,
                             final_state=None, stream=None) -> Launch:
    """Validate and bind one token-by-token KDA forward (see fused_recurrent_kda).
    Tensors as plan_chunk_kda; no workspace.  initial_state and final_state
    may be the same tensor (in-place state update)."""
    dev, B, T, H, Dk, Dv = _kda_check(q, k, v, g, beta, o, initial_state, final_state)
    if (Dk, Dv) != (128, 128) and B * H > 0:
        raise ValueError(f"unsupported KDA shape: key_dim={Dk} value_dim={Dv} (supported: 128, 128)")
    if scale is None:
        scale = Dk ** -0.5
    bdt = TM_DT_BF16 if beta.dtype == torch.bfloat16 else TM_DT_F32
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(initial_state), _ptr(o),
            _ptr(final_state), B, T, H, Dk, Dv, float(scale), bdt)
    return Launch(_lib.lib().tm_kda_recurrent_fwd, args, "kda_recurrent_fwd", dev, stream)


def fused_recurrent_kda(q, k, v, g, beta, scale=None, initial_state=None,
                        output_final_state=False):
    """Kimi Delta Attention, token by token, in the calling convention of the
    published ``fused_recurrent_kda`` operator (the decoding counterpart of
    chunk_kda): same tensors, same rule, one step per token.

    Returns (o [B, T, H, V] bf16, final_state fp32 [B, H, K, V] or None)."""
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    o = torch.empty(B, T, H, Dv, dtype=torch.bfloat16, device=q.device)
    st = (torch.empty(B, H, Dk, Dv, dtype=torch.float32, device=q.device)
          if output_final_state else None)
    _run(plan_fused_recurrent_kda(q, k, v, g, beta, o, scale=scale, initial_state=initial_state,
                                  final_state=st))
    return o, st


def chunk_kda(q, k, v, g, beta, scale=None, initial_state=None, output_final_state=False,
              chunk_size=KDA_CHUNK):
    """Kimi Delta Attention, chunked forward, in the calling convention of the
    published ``chunk_kda`` operator: [B, T, H, D] tensors, g the per-channel
    log decay, beta the per-step write strength, scale default K**-0.5.

    Returns (o [B, T, H, V] bf16, final_state fp32 [B, H, K, V] or None)."""
    B, T, H, Dk = q.shape
    Dv = v.shape[-1]
    o = torch.empty(B, T, H, Dv, dtype=torch.bfloat16, device=q.device)
    st = (torch.empty(B, H, Dk, Dv, dtype=torch.float32, device=q.device)
          if output_final_state else None)
    _run(plan_chunk_kda(q, k, v, g, beta, o, scale=scale, initial_state=initial_state,
                        final_state=st, chunk_size=chunk_size))
    return o, st
