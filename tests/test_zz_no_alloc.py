"""qflash_hip_scales_noalloc (the workspace in static device memory) against
qflash_hip_scales (a caller workspace), through the C ABI.

Two calls in a row, the second on smaller inputs, so that whatever the first
call left in the shared static array cannot leak into the second; both must
give the scales of the workspace entry point bit for bit, and those equal
torch's own absmax / 127 on the GPU.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _geo(q, k, v):
    return (ctypes.c_int64 * 24)(*q.shape, *q.stride(), *k.shape, *k.stride(), *v.shape, *v.stride())


def _scales(L, fn, q, k, v, code, ws=None):
    out = torch.full((4,), float("nan"), dtype=q.dtype, device=q.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ptrs = [ctypes.c_void_p(x.data_ptr()) for x in (q, k, v)]
    if ws is None:
        rc = fn(*ptrs, code, _geo(q, k, v), ctypes.c_void_p(out.data_ptr()), stream)
    else:
        rc = fn(*ptrs, code, _geo(q, k, v), ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()),
                ws.numel(), stream)
    assert rc == 0, L.qflash_hip_last_error()
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_noalloc_scales_equal_workspace_scales(dtype):
    from qflash_amd import _lib
    L = _lib.load()
    code = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}[dtype]
    ws = torch.zeros(_lib.SCALES_WORKSPACE, dtype=torch.int32, device=DEV)
    g = torch.Generator().manual_seed(11)
    # first call: large inputs with large maxima; second: smaller inputs whose
    # maxima are below the first call's, so stale slots would show
    shapes = [((4, 6, 197, 64), 30.0), ((2, 3, 49, 32), 0.5)]
    for shape, amp in shapes:
        print(f"[case] dtype={dtype} shape={shape} amp={amp}", flush=True)
        q, k, v = ((torch.randn(*shape, generator=g) * amp).to(DEV, dtype) for _ in range(3))
        k = k.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)  # token-major view
        want = _scales(L, L.qflash_hip_scales, q, k, v, code, ws)
        got = _scales(L, L.qflash_hip_scales_noalloc, q, k, v, code)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16 if dtype != torch.float32 else torch.int32),
                           want.view(torch.int16 if dtype != torch.float32 else torch.int32)), (got, want)
        ref = torch.stack([x.abs().amax() / 127 for x in (q, k, v)])
        assert torch.equal(got[:3], ref)
        assert torch.equal(got[3], got[0] * got[1])


def test_noalloc_scales_rejects_null_arguments():
    from qflash_amd import _lib
    L = _lib.load()
    geo = (ctypes.c_int64 * 24)(*([1] * 24))
    assert L.qflash_hip_scales_noalloc(None, None, None, _lib.F32, geo, None, None) == -1
    assert b"null" in L.qflash_hip_last_error()
