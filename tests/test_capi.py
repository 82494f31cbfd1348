"""The C ABI library loads and exports what include/tm_hip.h declares (CPU only).

No compute is launched: only symbol presence, metadata calls and argument
validation that fails before any HIP call.
"""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))
LIB = ROOT / "triton-metal_amd" / "triton_metal_amd" / "libtm_hip.so"


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(tm_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_functions()
    for n in ["tm_init", "tm_last_error", "tm_module_load", "tm_launch", "tm_int4_matmul",
              "tm_int8_matmul", "tm_int4_linear", "tm_int8_linear", "tm_matmul", "tm_linear",
              "tm_wq_dequant"]:
        assert n in names


def test_library_exports_every_declared_symbol():
    assert LIB.exists(), "libtm_hip.so not built (run __graft_entry__.build())"
    lib = ctypes.CDLL(str(LIB))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    import triton_metal_amd._lib as L
    assert set(declared_functions()) <= set(L.SIGNATURES)


def test_metadata_calls_without_gpu():
    import triton_metal_amd._lib as L
    lib = L.lib()
    assert b"gfx950" in lib.tm_version()
    assert lib.tm_num_builtin_modules() >= 2
    names = {lib.tm_builtin_module_name(i).decode() for i in range(lib.tm_num_builtin_modules())}
    assert {"wq_gemm", "gemm"} <= names
    assert lib.tm_builtin_module_name(99) is None


def test_argument_validation_before_any_hip_call():
    import triton_metal_amd._lib as L
    lib = L.lib()
    p = ctypes.c_void_p(16)
    # odd K for int4
    rc = lib.tm_int4_matmul(p, p, p, p, None, 1, 16, 7, 128, L.TM_DT_F16, L.TM_DT_F16,
                            L.TM_DT_NONE, None)
    assert rc == L.TM_ERR_INVALID_ARG and "even" in L.last_error()
    # bad dtype
    rc = lib.tm_int8_matmul(p, p, p, p, None, 1, 16, 64, 7, L.TM_DT_F16, L.TM_DT_NONE, None)
    assert rc == L.TM_ERR_INVALID_ARG
    # zeros dtype given but NULL pointer
    rc = lib.tm_int8_matmul(p, p, p, p, None, 1, 16, 64, L.TM_DT_F16, L.TM_DT_F16,
                            L.TM_DT_F16, None)
    assert rc == L.TM_ERR_INVALID_ARG and "zeros" in L.last_error()
    # leading dimension too small
    rc = lib.tm_matmul(p, p, p, 4, 4, 4, 2, 4, 4, L.TM_DT_F16, L.TM_DT_F16, None)
    assert rc == L.TM_ERR_INVALID_ARG
    # empty problems are a no-op success
    assert lib.tm_matmul(p, p, p, 0, 4, 4, 4, 4, 4, L.TM_DT_F16, L.TM_DT_F16, None) == 0
    with pytest.raises(RuntimeError):
        L.check(L.TM_ERR_INVALID_ARG, "probe")


def test_kda_workspace_and_validation():
    import triton_metal_amd._lib as L
    lib = L.lib()
    # 74240 bytes per (batch*head, 64-step chunk); C5 = 1 x 16 heads x 128 chunks
    assert lib.tm_kda_workspace_size(1, 8192, 16, 128, 128, 64) == 16 * 128 * 74240
    assert lib.tm_kda_workspace_size(2, 65, 3, 128, 128, 64) == 2 * 3 * 2 * 74240
    assert lib.tm_kda_workspace_size(1, 64, 1, 64, 128, 64) == 0        # unsupported dims
    assert lib.tm_kda_workspace_size(1, 64, 1, 128, 128, 32) == 0
    p = ctypes.c_void_p(16)
    args = [p, p, p, p, p, None, p, None]
    rc = lib.tm_kda_chunk_fwd(*args, 1, 64, 1, 64, 128, 64, 0.1, L.TM_DT_F32, p, 1 << 20, None)
    assert rc == L.TM_ERR_UNSUPPORTED and "key_dim" in L.last_error()
    rc = lib.tm_kda_chunk_fwd(*args, 1, 64, 1, 128, 128, 64, 0.1, L.TM_DT_F16, p, 1 << 20, None)
    assert rc == L.TM_ERR_INVALID_ARG and "beta_dtype" in L.last_error()
    rc = lib.tm_kda_chunk_fwd(*args, 1, 64, 1, 128, 128, 64, 0.1, L.TM_DT_F32, p, 100, None)
    assert rc == L.TM_ERR_INVALID_ARG and "workspace" in L.last_error()
    rc = lib.tm_kda_chunk_fwd(*args, -1, 64, 1, 128, 128, 64, 0.1, L.TM_DT_F32, p, 0, None)
    assert rc == L.TM_ERR_INVALID_ARG
    # no heads: nothing to do
    assert lib.tm_kda_chunk_fwd(*args, 1, 64, 0, 128, 128, 64, 0.1, L.TM_DT_F32, p, 0,
                                None) == 0


def test_int8_matmul_rejects_uint8_weights():
    """The kernels read the weight bytes as signed int8 (the reference's
    `device const char*`); uint8 storage is refused rather than misread."""
    import torch
    import triton_metal_amd as tm
    x = torch.zeros(1, 64, dtype=torch.float16)
    w = torch.zeros(16, 64, dtype=torch.uint8)
    with pytest.raises(TypeError, match="int8"):
        tm.int8_matmul(x, w, torch.zeros(1, 16, dtype=torch.float16),
                       torch.ones(16, dtype=torch.float16), None, 1, 16, 64)


def test_dot_validation_before_any_hip_call():
    import triton_metal_amd._lib as L
    lib = L.lib()
    p = ctypes.c_void_p(16)
    st = (ctypes.c_longlong * 14)(0, 8, 1, 0, 8, 1, 0, 8, 1, 0, 0, 0, 0, 0)
    args = (p, p, p, None, None, 1, 8, 8, 8, 0, st)
    # unknown epilogue, bad dtype, add epilogue without Z, negative stride
    assert lib.tm_dot(*args, 9, L.TM_DT_F16, L.TM_DT_F16, L.TM_DT_NONE, L.TM_DT_NONE,
                      None) == L.TM_ERR_INVALID_ARG
    assert lib.tm_dot(*args, 0, 42, L.TM_DT_F16, L.TM_DT_NONE, L.TM_DT_NONE,
                      None) == L.TM_ERR_INVALID_ARG
    assert lib.tm_dot(*args, L.TM_EPI_ADD_ROWS, L.TM_DT_F16, L.TM_DT_F16, L.TM_DT_NONE,
                      L.TM_DT_NONE, None) == L.TM_ERR_INVALID_ARG
    assert "Z" in L.last_error()
    neg = (ctypes.c_longlong * 14)(0, 8, -1, 0, 8, 1, 0, 8, 1, 0, 0, 0, 0, 0)
    assert lib.tm_dot(p, p, p, None, None, 1, 8, 8, 8, 0, neg, 0, L.TM_DT_F16, L.TM_DT_F16,
                      L.TM_DT_NONE, L.TM_DT_NONE, None) == L.TM_ERR_INVALID_ARG
    # softmax rows beyond what a workgroup keeps on chip
    assert lib.tm_dot(p, p, p, None, None, 1, 8, 9000, 8, 0, st, L.TM_EPI_SOFTMAX,
                      L.TM_DT_F16, L.TM_DT_F32, L.TM_DT_NONE, L.TM_DT_NONE,
                      None) == L.TM_ERR_UNSUPPORTED
    # empty problems succeed without touching the device
    assert lib.tm_dot(p, p, p, None, None, 0, 8, 8, 8, 0, st, 0, L.TM_DT_F16, L.TM_DT_F16,
                      L.TM_DT_NONE, L.TM_DT_NONE, None) == 0
