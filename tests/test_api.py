"""The drop-in module API (qflash_amd.attention) on the CPU.

Structure and host logic only: parameter names, state_dict keys, weight
transfer, in-place patching and the masks handed to ``qflash.forward``
(mirroring qflash/attention.py:12-108).  The attention op itself is replaced
by a recorder here; on the GPU the real op runs (test_gpu_api.py).
"""
from __future__ import annotations

import pytest
import torch
from torch import nn

import qflash_amd
from qflash_amd import QAttention, QWindowAttention, patch_attention
from qflash_amd import attention as A
from qflash_amd.attention import get_relative_position_index


class TimmLikeAttention(nn.Module):
    """Stands in for timm.layers.attention.Attention (same submodule names)."""

    def __init__(self, dim, num_heads, qkv_bias=True):
        super().__init__()
        self.num_heads = num_heads
        self.qkv = nn.Linear(dim, dim * 3, bias=qkv_bias)
        self.proj = nn.Linear(dim, dim)


class TimmLikeWindowAttention(nn.Module):
    """Stands in for timm.models.swin_transformer.WindowAttention."""

    def __init__(self, dim, num_heads, window_size, qkv_bias=True):
        super().__init__()
        self.dim, self.num_heads, self.window_size = dim, num_heads, (window_size, window_size)
        self.relative_position_bias_table = nn.Parameter(torch.randn((2 * window_size - 1) ** 2, num_heads))
        self.register_buffer("relative_position_index", get_relative_position_index(window_size, window_size),
                             persistent=False)
        self.qkv = nn.Linear(dim, dim * 3, bias=qkv_bias)
        self.proj = nn.Linear(dim, dim)


class Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.norm = nn.LayerNorm(64)
        self.attn = TimmLikeAttention(64, 2)


class Stage(nn.Module):
    def __init__(self):
        super().__init__()
        self.blocks = nn.Sequential(Block(), Block())
        self.wattn = TimmLikeWindowAttention(48, 3, 7, qkv_bias=False)


def test_package_exports_the_reference_names():
    assert set(qflash_amd.__all__) == {"qflash", "QAttention", "QWindowAttention", "patch_attention"}
    assert callable(qflash_amd.qflash.forward) and len(qflash_amd.qflash.kernel) == 2


def test_qattention_state_dict_keys():
    m = QAttention(192, 3)
    assert list(m.state_dict()) == ["qkv.weight", "qkv.bias", "proj.weight", "proj.bias"]
    assert m.head_dim == 64 and m.num_heads == 3
    assert list(QAttention(64, 2, qkv_bias=False).state_dict()) == ["qkv.weight", "proj.weight", "proj.bias"]


def test_window_attention_state_dict_and_buffers():
    m = QWindowAttention(96, 3, 7)
    assert list(m.state_dict()) == ["relative_position_bias_table", "qkv.weight", "qkv.bias", "proj.weight",
                                    "proj.bias"]
    assert m.relative_position_bias_table.shape == (169, 3)
    assert m.window_size == (7, 7) and m.window_area == 49
    assert "relative_position_index" in dict(m.named_buffers())
    t = m.relative_position_bias_table
    assert t.abs().max() <= 2.0 and 0.01 < t.std() < 0.03   # trunc_normal_(std=.02), absolute cut at +-2


@pytest.mark.parametrize("hw", [(7, 7), (3, 5), (1, 4)])
def test_relative_position_index_brute_force(hw):
    h, w = hw
    idx = get_relative_position_index(h, w)
    pos = [(y, x) for y in range(h) for x in range(w)]
    want = torch.tensor([[(yi - yj + h - 1) * (2 * w - 1) + (xi - xj + w - 1) for (yj, xj) in pos]
                         for (yi, xi) in pos])
    assert torch.equal(idx, want)
    assert idx.min() == 0 and idx.max() == (2 * h - 1) * (2 * w - 1) - 1


def test_from_orig_copies_weights_dtype_and_device():
    src = TimmLikeAttention(64, 2).to(torch.float64)
    new = QAttention.from_orig(src)
    assert new.qkv.weight.dtype == torch.float64
    for a, b in zip(src.state_dict().values(), new.state_dict().values()):
        assert torch.equal(a, b)
    wsrc = TimmLikeWindowAttention(48, 3, 7, qkv_bias=False)
    wnew = QWindowAttention.from_orig(wsrc)
    assert wnew.qkv.bias is None
    assert torch.equal(wnew.relative_position_bias_table, wsrc.relative_position_bias_table)


def test_patch_attention_in_place_with_named_types():
    model = nn.Sequential(Stage(), Stage())
    before = {k: v.clone() for k, v in model.state_dict().items()}
    counts = patch_attention(model, attn_types=[TimmLikeAttention], window_attn_types=[TimmLikeWindowAttention])
    assert counts == {"attn": 4, "wattn": 2}
    assert isinstance(model[0].blocks[1].attn, QAttention)
    assert isinstance(model[1].wattn, QWindowAttention)
    after = model.state_dict()
    assert list(after) == list(before)
    assert all(torch.equal(before[k], after[k]) for k in before)
    # patching again finds nothing
    assert patch_attention(model, [TimmLikeAttention], [TimmLikeWindowAttention]) == {"attn": 0, "wattn": 0}


def test_patch_attention_without_timm_needs_named_types():
    try:
        import timm  # noqa: F401
        pytest.skip("timm is installed")
    except ImportError:
        pass
    with pytest.raises(ImportError):
        patch_attention(nn.Sequential(Block()))


class _Recorder:
    """Replaces qflash.forward: records its arguments, returns fp32 softmax attention."""

    def __init__(self):
        self.calls = []

    def __call__(self, q, k, v, attn_mask=None, scale=None):
        self.calls.append((q, k, v, attn_mask))
        s = (q @ k.transpose(-1, -2)) / q.shape[-1] ** 0.5
        if attn_mask is not None:
            s = s + attn_mask
        return torch.softmax(s, -1) @ v


def _timm_window_reference(m, x, mask):
    """WindowAttention.forward of timm in plain fp32 (the contract QWindowAttention keeps)."""
    B_, N, C = x.shape
    H = m.num_heads
    qkv = m.qkv(x).reshape(B_, N, 3, H, C // H).permute(2, 0, 3, 1, 4)
    q, k, v = qkv.unbind(0)
    attn = (q * (C // H) ** -0.5) @ k.transpose(-2, -1)
    bias = m.relative_position_bias_table[m.relative_position_index.view(-1)].view(N, N, -1).permute(2, 0, 1)
    attn = attn + bias.unsqueeze(0)
    if mask is not None:
        nW = mask.shape[0]
        attn = attn.view(-1, nW, H, N, N) + mask.unsqueeze(1).unsqueeze(0)
        attn = attn.view(-1, H, N, N)
    attn = attn.softmax(-1)
    return m.proj((attn @ v).transpose(1, 2).reshape(B_, N, -1))


class _WindowRecorder(_Recorder):
    """Replaces qflash_forward_window: composes the (B_, H, N, N) mask exactly as
    the reference module does (attention.py:68-72) and records it."""

    def __call__(self, q, k, v, rel_bias, mask=None, scale=None):
        attn_mask = rel_bias
        if mask is not None:
            B_, H, N = q.shape[0], q.shape[1], q.shape[2]
            nw = mask.shape[0]
            attn_mask = rel_bias + mask.view(1, nw, 1, N, N).expand(B_ // nw, -1, H, -1, -1).reshape(-1, H, N, N)
        return super().__call__(q, k, v, attn_mask=attn_mask)


def test_window_attention_mask_composition(monkeypatch):
    rec = _WindowRecorder()
    monkeypatch.setattr(A, "qflash_forward_window", rec)
    torch.manual_seed(0)
    m = QWindowAttention(48, 3, 7)
    nW, B = 4, 2
    x = torch.randn(B * nW, 49, 48)
    shift = torch.zeros(nW, 49, 49)
    shift[2:, :20, 20:] = -100.0
    with torch.no_grad():
        got = m(x, shift)
        want = _timm_window_reference(m, x, shift)
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    q, k, v, am = rec.calls[0]
    assert q.shape == (B * nW, 3, 49, 16) and am.shape == (B * nW, 3, 49, 49)
    assert not q.is_contiguous()                      # token-major views go straight to the op
    with torch.no_grad():
        got0 = m(x)
    assert rec.calls[1][3].shape == (1, 3, 49, 49)    # no shift mask: the (1,H,N,N) bias broadcasts
    torch.testing.assert_close(got0, _timm_window_reference(m, x, None), rtol=1e-5, atol=1e-5)


def test_qattention_forward_contract(monkeypatch):
    rec = _Recorder()
    monkeypatch.setattr(A.qflash, "forward", rec)
    torch.manual_seed(1)
    m = QAttention(64, 2)
    x = torch.randn(3, 10, 64)
    with torch.no_grad():
        got = m(x)
        qkv = m.qkv(x).reshape(3, 10, 3, 2, 32).permute(2, 0, 3, 1, 4)
        q, k, v = qkv.unbind(0)
        ref = torch.softmax(q @ k.transpose(-1, -2) / 32 ** 0.5, -1) @ v
        want = m.proj(ref.transpose(1, 2).reshape(3, 10, 64))
    torch.testing.assert_close(got, want, rtol=1e-5, atol=1e-5)
    mask = torch.ones(10, 10, dtype=torch.bool)
    with torch.no_grad():
        m(x, attn_mask=mask)
    assert rec.calls[-1][3] is mask


def test_modules_on_cpu_raise_instead_of_falling_back():
    x = torch.randn(2, 49, 96)
    with pytest.raises(ValueError, match="GPU"):
        QWindowAttention(96, 3, 7)(x)
    with pytest.raises(ValueError, match="GPU"):
        QAttention(96, 3)(x)
