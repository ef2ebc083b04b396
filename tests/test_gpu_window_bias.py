"""qflash_hip_window_bias against the torch ops it replaces (GPU).

The reference builds QWindowAttention's int32 bias with torch ops on the
device (qflash/attention.py:68-74, then qflash/kernel.py:327-336);
`bias_values` restates them op for op.  The fused kernel must give the same
int32 for every element: random tables and masks, values on both sides of the
-100 threshold, and products near half-integers, where the order of the fp32
roundings decides the result.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from qflash_amd.kernel import bias_values, window_bias

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _torch_bias(rel, mask, sm):
    H, N = rel.shape[-3], rel.shape[-1]
    x = rel.reshape(1, H, N, N) if mask is None else rel + mask.view(mask.shape[0], 1, N, N)
    return bias_values(x, sm).contiguous()


@pytest.mark.parametrize("sm", [0.1767766952966369 * 1.4426950408889634, 0.05, 1 / 57.3, 0.9, 3.7])
@pytest.mark.parametrize("with_mask", [False, True])
def test_window_bias_matches_torch_ops(sm, with_mask):
    print(f"[case] sm={sm} with_mask={with_mask}", flush=True)
    g = np.random.default_rng(int(sm * 1e4) + with_mask)
    H, N, nW = 3, 49, 16
    rel = torch.from_numpy((g.standard_normal((1, H, N, N)) * 0.02).astype(np.float32)).to(DEV)
    mask = None
    if with_mask:
        m = np.zeros((nW, N, N), np.float32)
        m[g.random((nW, N, N)) < 0.3] = -100.0
        edge = g.random((nW, N, N))
        m[edge < 0.05] = np.float32(-99.99999)
        m[(edge >= 0.05) & (edge < 0.1)] = np.float32(-100.00001)
        m[(edge >= 0.1) & (edge < 0.15)] = -1e9
        mask = torch.from_numpy(m).to(DEV)
    got = window_bias(rel, mask, sm)
    want = _torch_bias(rel, mask, sm)
    torch.cuda.synchronize()
    assert got.shape == want.shape and got.dtype == torch.int32
    assert int((got != want).sum()) == 0


@pytest.mark.parametrize("sm", [0.05, 1 / 57.3, 0.3])
def test_window_bias_at_rounding_boundaries(sm):
    """x * LOG2E / sm_scale within a few ulp of k + 1/2 for many k."""
    print(f"[case] sm={sm}", flush=True)
    H, N = 2, 64
    k = np.arange(-2000, 2000, dtype=np.float64)
    target = (k + 0.5) * sm / 1.44269504
    x = np.concatenate([np.nextafter(target.astype(np.float32), np.float32(np.inf)),
                        target.astype(np.float32),
                        np.nextafter(target.astype(np.float32), np.float32(-np.inf))])
    x = x[np.abs(x) < 90.0]
    flat = np.resize(x, H * N * N).astype(np.float32)
    rel = torch.from_numpy(flat.reshape(1, H, N, N)).to(DEV)
    for mask in (None, torch.zeros((4, N, N), dtype=torch.float32, device=DEV)):
        got = window_bias(rel, mask, sm)
        want = _torch_bias(rel, mask, sm)
        torch.cuda.synchronize()
        assert int((got != want).sum()) == 0


@pytest.mark.parametrize("shape", [(49, 49), (1, 3, 49, 49), (8, 3, 49, 49)])
def test_mask_bias_matches_torch_ops(shape):
    """qflash_hip_mask_bias (mask_to_bias on an fp32 device mask) against
    bias_values' torch ops, with values at and around the -100 threshold."""
    from qflash_amd.kernel import mask_to_bias
    print(f"[case] shape={shape}", flush=True)
    g = np.random.default_rng(len(shape) * 100 + shape[0])
    m = (g.standard_normal(shape) * 3).astype(np.float32)
    sel = g.random(shape)
    m[sel < 0.2] = -100.0
    m[(sel >= 0.2) & (sel < 0.25)] = np.float32(-99.99999)
    m[(sel >= 0.25) & (sel < 0.3)] = -1e30
    mask = torch.from_numpy(m).to(DEV)
    sm = 0.1767766952966369 * 1.4426950408889634
    Z, H, N = 8, 3, 49
    got = mask_to_bias(mask, sm, Z, H, N, materialize=True)
    want = bias_values(mask, sm).expand(Z, H, N, N).contiguous()
    torch.cuda.synchronize()
    assert int((got != want).sum()) == 0


def test_mask_bias_unaligned_and_ragged():
    """A mask whose data starts 4 bytes into its buffer (scalar path) and
    sizes that are not multiples of 4 (the last partial group)."""
    import ctypes

    from qflash_amd.kernel import _lib as lib, _stream_ptr
    g = np.random.default_rng(5)
    base = torch.from_numpy((g.standard_normal(1 + 7 * 49) * 40).astype(np.float32)).to(DEV)
    mask = base[1:].view(7, 49)                   # 4-byte offset into the allocation
    assert mask.data_ptr() % 16 != 0 and mask.is_contiguous()
    sm = 0.3
    for m in (mask, base[:343].view(7, 49), base[:341]):
        out = torch.empty(m.shape, dtype=torch.int32, device=DEV)
        rc = lib.load().qflash_hip_mask_bias(ctypes.c_void_p(m.data_ptr()), m.numel(), sm,
                                             ctypes.c_void_p(out.data_ptr()), _stream_ptr(m))
        lib.check(rc, "qflash_hip_mask_bias")
        want = bias_values(m, sm)
        torch.cuda.synchronize()
        assert int((out != want).sum()) == 0
