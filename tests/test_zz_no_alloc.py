"""tm_decode_attention_noalloc (the allocation-free decode-attention entry)
against tm_decode_attention with a caller workspace, through the C ABI.

Both entry points plan the same slices and run the same kernels, so the
outputs are bit-identical.  Two calls in a row on the shared scratch, the
second with a smaller input; and a plan needing more scratch than the static
array holds is refused before anything is launched.
"""
import ctypes as C

import pytest
import torch

pytestmark = pytest.mark.gpu


def _problem(B, Hq, Hkv, D, S, seed, dt=torch.float16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, D, generator=g).to(dt)
    k = torch.randn(B, Hkv, S, D, generator=g).to(dt)
    v = torch.randn(B, Hkv, S, D, generator=g).to(dt)
    return q, k, v


def _call(L, noalloc, dev, q, k, v, lens, dt_code):
    from triton_metal_amd import _lib
    B, Hq, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    o = torch.full((B, Hq, D), float("nan"), dtype=q.dtype, device=dev)
    lse = torch.full((B, Hq), float("nan"), dtype=torch.float32, device=dev)
    sl = torch.tensor(lens, dtype=torch.int32, device=dev)
    strides = (C.c_longlong * 3)(k.stride(0), k.stride(1), k.stride(2))
    stream = torch.cuda.current_stream(dev).cuda_stream
    common = (C.c_void_p(q.data_ptr()), C.c_void_p(k.data_ptr()), C.c_void_p(v.data_ptr()),
              C.c_void_p(o.data_ptr()), C.c_void_p(lse.data_ptr()), B, Hq, Hkv, D,
              C.c_void_p(sl.data_ptr()), S, strides, None, 0, 0, D ** -0.5, dt_code, dt_code,
              dt_code)
    ws = None
    if noalloc:
        rc = L.tm_decode_attention_noalloc(*common, stream)
    else:
        need = L.tm_decode_attention_workspace_size(B, Hq, Hkv, D, S, 0)
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
        rc = L.tm_decode_attention(*common, C.c_void_p(ws.data_ptr()), ws.numel(), stream)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return o, lse


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_noalloc_matches_workspace_entry_twice(dev, dt):
    from triton_metal_amd import _lib
    L = _lib.lib()
    code = _lib.TM_DT_F16 if dt == torch.float16 else _lib.TM_DT_BF16
    # first call: many slices (long sequence, few heads); second: smaller
    for (B, Hq, Hkv, D, S, lens, seed) in [(2, 16, 4, 128, 9000, [9000, 4321], 1),
                                           (1, 8, 2, 64, 1500, [1500], 2)]:
        q, k, v = (t.to(dev) for t in _problem(B, Hq, Hkv, D, S, seed, dt))
        need = L.tm_decode_attention_workspace_size(B, Hq, Hkv, D, S, 0)
        assert need > 0  # the scratch is used, not bypassed
        print(f"[noalloc] B={B} Hq={Hq} Hkv={Hkv} D={D} S={S} scratch {need} B", flush=True)
        o_ref, l_ref = _call(L, False, dev, q, k, v, lens, code)
        o_na, l_na = _call(L, True, dev, q, k, v, lens, code)
        assert torch.equal(o_na, o_ref)
        assert torch.equal(l_na, l_ref)


def test_noalloc_rejects_plans_beyond_the_scratch(dev):
    """A plan needing more than TM_DECODE_SCRATCH_BYTES fails with
    TM_ERR_INVALID_ARG before any launch (the output stays untouched)."""
    from triton_metal_amd import _lib
    L = _lib.lib()
    limit = 8 << 20
    # paged caches cap a slice at 64 pages, so a long paged sequence needs many slices
    B, Hq, Hkv, D, ps = 1, 64, 4, 128, 16
    S = 1 << 20
    need = L.tm_decode_attention_workspace_size(B, Hq, Hkv, D, S, ps)
    assert need > limit
    q = torch.zeros(B, Hq, D, dtype=torch.float16, device=dev)
    o = torch.full_like(q, 7.0)
    cache = torch.zeros(16, ps, Hkv, D, dtype=torch.float16, device=dev)  # never read
    table = torch.zeros(B, S // ps, dtype=torch.int32, device=dev)
    rc = L.tm_decode_attention_noalloc(
        C.c_void_p(q.data_ptr()), C.c_void_p(cache.data_ptr()), C.c_void_p(cache.data_ptr()),
        C.c_void_p(o.data_ptr()), None, B, Hq, Hkv, D, None, S, None,
        C.c_void_p(table.data_ptr()), ps, S // ps, D ** -0.5, _lib.TM_DT_F16, _lib.TM_DT_F16,
        _lib.TM_DT_F16, torch.cuda.current_stream(dev).cuda_stream)
    assert rc == _lib.TM_ERR_INVALID_ARG
    assert "scratch" in _lib.last_error()
    torch.cuda.synchronize()
    assert (o == 7.0).all()
