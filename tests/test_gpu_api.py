"""GPU: the drop-in modules run the gfx950 kernels, and what the kernels return
equals the C oracle's codes on the inputs the modules handed over.

The real ``qflash.forward`` is wrapped (not replaced) to record its inputs and
output; the check recomputes the host constants, int8 codes and bias on the CPU
from the recorded fp tensors and runs the C oracle on them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import oracle_c
from oracle.qflash_oracle import Consts, Flags

pytestmark = pytest.mark.gpu
DEV = "cuda"


class _Tap:
    def __init__(self, fn):
        self.fn, self.calls = fn, []

    def __call__(self, q, k, v, attn_mask=None, scale=None, return_mode="output"):
        out = self.fn(q, k, v, attn_mask=attn_mask, scale=scale, return_mode=return_mode)
        self.calls.append((q, k, v, attn_mask, out))
        return out


def _expected(q, k, v, mask):
    from qflash_amd.kernel import LOG2E, fixed_point_constants, mask_to_bias, quantize
    q, k, v = q.cpu(), k.cpu(), v.cpu()
    Z, H, N, D = q.shape
    qs, ks, vs = (x.abs().amax() / 127 for x in (q, k, v))
    sm = (1.0 / math.sqrt(D)) * LOG2E * (qs * ks).item()
    c = Consts(*fixed_point_constants(sm, 30, 30))
    bias = None if mask is None else mask_to_bias(mask.cpu(), sm, Z, H, N, materialize=True)
    codes = oracle_c.attention_codes(quantize(q, qs), quantize(k, ks), quantize(v, vs), c, Flags(), bias, threads=8)
    return torch.from_numpy(codes) * vs


def test_qattention_runs_the_kernel_bit_exactly(monkeypatch):
    from qflash_amd import QAttention
    from qflash_amd import attention as A
    tap = _Tap(A.qflash.forward)
    monkeypatch.setattr(A.qflash, "forward", tap)
    torch.manual_seed(0)
    m = QAttention(384, 6).to(DEV)
    x = torch.randn(4, 197, 384, device=DEV)
    with torch.no_grad():
        y = m(x)
    torch.cuda.synchronize()
    q, k, v, mask, out = tap.calls[0]
    assert mask is None and not q.is_contiguous()
    assert torch.equal(out.cpu(), _expected(q, k, v, None))
    assert y.shape == x.shape and torch.isfinite(y).all()


@pytest.mark.parametrize("shifted", [False, True])
def test_window_attention_runs_the_masked_kernel_bit_exactly(monkeypatch, shifted):
    from qflash_amd import QWindowAttention
    from qflash_amd import attention as A
    tap = _Tap(A.qflash.forward)
    monkeypatch.setattr(A.qflash, "forward", tap)
    torch.manual_seed(1)
    m = QWindowAttention(96, 3, 7).to(DEV)
    nW, B = 16, 2
    x = torch.randn(B * nW, 49, 96, device=DEV)
    mask = None
    if shifted:
        ys, xs = torch.meshgrid(torch.arange(7), torch.arange(7), indexing="ij")
        region = (ys.flatten() >= 4).long() * 2 + (xs.flatten() >= 4).long()
        m4 = (region[:, None] != region[None, :]).float() * -100.0
        mask = torch.zeros(nW, 49, 49)
        mask[nW // 2:] = m4
        mask = mask.to(DEV)
    with torch.no_grad():
        y = m(x, mask)
    torch.cuda.synchronize()
    q, k, v, am, out = tap.calls[0]
    assert am is not None
    assert torch.equal(out.cpu(), _expected(q, k, v, am))
    assert y.shape == x.shape and torch.isfinite(y).all()


def test_forward_latency_mode_returns_milliseconds():
    from qflash_amd import qflash
    g = torch.Generator().manual_seed(2)
    q = torch.randn(2, 3, 197, 64, generator=g).to(DEV)
    ms = qflash.forward(q, q, q, return_mode="latency")
    assert isinstance(ms, float) and 0 < ms < 100


def test_forward_keeps_input_dtype_and_stream():
    from qflash_amd import qflash
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(2, 2, 70, 32, generator=g).half().to(DEV) for _ in range(3))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        out = qflash.forward(q, k, v)
    s.synchronize()
    assert out.dtype == torch.float16
    want = _expected(q, k, v, None).half()
    assert torch.equal(out.cpu(), want)
    np.asarray(out.cpu())
