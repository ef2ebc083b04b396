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


class _WindowTap:
    """Wraps qflash_forward_window; records the reference-composed (B_, H, N, N) mask."""

    def __init__(self, fn):
        self.fn, self.calls = fn, []

    def __call__(self, q, k, v, rel_bias, mask=None, scale=None):
        out = self.fn(q, k, v, rel_bias, mask, scale)
        full = rel_bias
        if mask is not None:
            B_, H, N = q.shape[0], q.shape[1], q.shape[2]
            nw = mask.shape[0]
            full = rel_bias + mask.view(1, nw, 1, N, N).expand(B_ // nw, -1, H, -1, -1).reshape(-1, H, N, N)
        self.calls.append((q, k, v, full, out))
        return out


@pytest.mark.parametrize("shifted", [False, True])
def test_window_attention_runs_the_masked_kernel_bit_exactly(monkeypatch, shifted):
    from qflash_amd import QWindowAttention
    from qflash_amd import attention as A
    tap = _WindowTap(A.qflash_forward_window)
    monkeypatch.setattr(A, "qflash_forward_window", tap)
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


def test_window_forward_matches_reference_golden_swin():
    """qflash_forward_window on the golden Swin case's parts (rel bias = window 0
    of the composed mask, shift mask rebuilt from the region ids) reproduces the
    reference's dequantised output."""
    from golden_io import load_cases
    from qflash_amd.kernel import qflash_forward_window
    c = load_cases()["swin_N49_D32"]
    full = torch.from_numpy(c["mask"])
    ys, xs = torch.meshgrid(torch.arange(7), torch.arange(7), indexing="ij")
    region = (ys.flatten() >= 4).long() * 2 + (xs.flatten() >= 4).long()
    shift = torch.zeros(2, 49, 49)
    shift[1] = (region[:, None] != region[None, :]).float() * -100.0
    q, k, v = (torch.from_numpy(c[n]).to(DEV) for n in ("q_fp", "k_fp", "v_fp"))
    out = qflash_forward_window(q, k, v, full[0:1].to(DEV), shift.to(DEV))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), c["out_fp"])


@pytest.mark.parametrize("seed", [0, 1])
def test_window_kernel_equals_masked_kernel_on_cfg4(seed):
    """cfg4 (4096 windows): the window-periodic launch and the masked launch on the
    materialised bias give identical codes, and both match the C oracle."""
    from qflash_amd.kernel import (LOG2E, bias_values, fixed_point_constants, mask_to_bias, qflash_masked_kernel,
                                   qflash_window_kernel, quantize)
    from qflash_amd.workloads import CONFIGS, make_inputs, make_window_parts
    cfg = CONFIGS["cfg4"]
    q, k, v, mask = make_inputs(cfg, seed)
    rel, shift = make_window_parts(cfg, seed)
    composed = rel + shift.view(1, cfg.windows, 1, cfg.N, cfg.N).expand(cfg.images, -1, cfg.H, -1, -1).reshape(
        -1, cfg.H, cfg.N, cfg.N)
    assert torch.equal(composed, mask)
    qs, ks, vs = (x.abs().amax() / 127 for x in (q, k, v))
    sm = (1.0 / cfg.D ** 0.5) * LOG2E * (qs * ks).item()
    consts = fixed_point_constants(sm, 30, 30)
    q8, k8, v8 = (quantize(x, s).to(DEV) for x, s in ((q, qs), (k, ks), (v, vs)))
    dense = mask_to_bias(mask, sm, cfg.Z, cfg.H, cfg.N, materialize=True)
    compact = bias_values(rel + shift.view(cfg.windows, 1, cfg.N, cfg.N), sm).contiguous()
    flags = dict(EXP_USE_SHIFT=True, L_USE_SHIFT=True, ACC_USE_SHIFT=True, L_SHIFT=30, ACC_SHIFT=30)
    o1, o2 = torch.empty_like(v8), torch.empty_like(v8)
    bd = dense.to(DEV)
    qflash_masked_kernel[None](q8, k8, v8, o1, bd, *consts, *q8.stride(), *k8.stride(), *v8.stride(), *o1.stride(),
                               *bd.stride(), cfg.Z, cfg.H, N_CTX=cfg.N, HEAD_DIM=cfg.D, **flags)
    qflash_window_kernel(q8, k8, v8, o2, compact.to(DEV), consts, cfg.windows, flags)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    want = oracle_c.attention_codes(q8.cpu(), k8.cpu(), v8.cpu(), Consts(*consts), Flags(), bias=dense, threads=16)
    np.testing.assert_array_equal(o2.cpu().numpy(), want)


def test_masked_kernel_strided_bias_columns():
    """A bias whose key stride is not 1 (a transposed view) takes the element-wise
    bias loads; codes equal the contiguous bias's."""
    from qflash_amd.kernel import fixed_point_constants, qflash_masked_kernel
    g = np.random.default_rng(9)
    Z, H, N, D = 2, 2, 70, 64
    q8, k8, v8 = (torch.from_numpy(g.integers(-128, 128, (Z, H, N, D)).astype(np.int8)).to(DEV) for _ in range(3))
    bias = torch.from_numpy(g.integers(-3000, 3000, (Z, H, N, N)).astype(np.int32))
    bias_t = bias.transpose(-1, -2).contiguous().transpose(-1, -2)          # same values, key stride N
    consts = fixed_point_constants(0.0123, 30, 30)
    flags = dict(EXP_USE_SHIFT=True, L_USE_SHIFT=True, ACC_USE_SHIFT=True, L_SHIFT=30, ACC_SHIFT=30)
    outs = []
    for b in (bias, bias_t):
        bd = b.to(DEV)
        o = torch.empty_like(v8)
        qflash_masked_kernel[None](q8, k8, v8, o, bd, *consts, *q8.stride(), *k8.stride(), *v8.stride(),
                                   *o.stride(), *bd.stride(), Z, H, N_CTX=N, HEAD_DIM=D, **flags)
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    want = oracle_c.attention_codes(q8.cpu(), k8.cpu(), v8.cpu(), Consts(*consts), Flags(), bias=bias, threads=8)
    np.testing.assert_array_equal(outs[0].cpu().numpy(), want)


def test_patch_attention_model_runs_the_kernels_bit_exactly(monkeypatch):
    """patch_attention (qflash/attention.py:89-108) on a small model built from
    timm-like stand-ins: every swapped module runs on the GPU and each
    attention call returns the oracle's codes times o_scale for the inputs the
    module handed over; the model output equals a second, unpatched run of the
    same modules through the recorded outputs."""
    from torch import nn

    from qflash_amd import QAttention, QWindowAttention, patch_attention
    from qflash_amd import attention as A
    from test_api import TimmLikeAttention, TimmLikeWindowAttention

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.norm = nn.LayerNorm(192)
            self.attn = TimmLikeAttention(192, 3)

        def forward(self, x):
            return x + self.attn(self.norm(x))

    class WinStage(nn.Module):
        def __init__(self):
            super().__init__()
            self.wattn = TimmLikeWindowAttention(96, 3, 7)

        def forward(self, x, mask):
            return x + self.wattn(x, mask)

    class Model(nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = nn.Sequential(Block(), Block())
            self.win = WinStage()

        def forward(self, x, xw, mask):
            return self.blocks(x), self.win(xw, mask)

    torch.manual_seed(4)
    model = Model()
    counts = patch_attention(model, attn_types=[TimmLikeAttention], window_attn_types=[TimmLikeWindowAttention])
    assert counts == {"attn": 2, "wattn": 1}
    assert isinstance(model.blocks[0].attn, QAttention) and isinstance(model.win.wattn, QWindowAttention)
    model = model.to(DEV)
    tap, wtap = _Tap(A.qflash.forward), _WindowTap(A.qflash_forward_window)
    monkeypatch.setattr(A.qflash, "forward", tap)
    monkeypatch.setattr(A, "qflash_forward_window", wtap)
    x = torch.randn(2, 197, 192, device=DEV)
    nW = 4
    xw = torch.randn(2 * nW, 49, 96, device=DEV)
    ys, xs = torch.meshgrid(torch.arange(7), torch.arange(7), indexing="ij")
    region = (ys.flatten() >= 4).long() * 2 + (xs.flatten() >= 4).long()
    mask = torch.zeros(nW, 49, 49)
    mask[nW // 2:] = (region[:, None] != region[None, :]).float() * -100.0
    with torch.no_grad():
        y, yw = model(x, xw, mask.to(DEV))
    torch.cuda.synchronize()
    assert len(tap.calls) == 2 and len(wtap.calls) == 1
    for q, k, v, m, out in tap.calls:
        assert m is None
        assert torch.equal(out.cpu(), _expected(q, k, v, None))
    q, k, v, am, out = wtap.calls[0]
    assert torch.equal(out.cpu(), _expected(q, k, v, am))
    assert torch.isfinite(y).all() and torch.isfinite(yw).all()
