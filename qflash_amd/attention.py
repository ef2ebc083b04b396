"""Drop-in attention modules, mirroring qflash/attention.py of the reference.

``QAttention`` replaces timm's ``Attention`` and ``QWindowAttention`` replaces
timm's ``WindowAttention`` (same constructor arguments, parameter names and
state_dict keys, same forward contracts); ``patch_attention`` swaps them into
a model in place.  The attention itself runs through ``qflash.forward`` on the
gfx950 HIP kernels.

timm is optional: when it is importable its helpers are used; otherwise the
three small helpers it provides here (``to_2tuple``, ``trunc_normal_``,
``get_relative_position_index``) are restated below.  ``patch_attention``
needs the timm classes it looks for, unless the caller names them.
"""
from __future__ import annotations

import collections.abc
from typing import Dict, Iterable, Optional

import torch
from torch import nn

from .kernel import LOG2E, forward_codes, int8_weights, qflash, qflash_forward_window, qkv_int8

try:  # pragma: no cover - timm is absent in the build image
    from timm.layers import to_2tuple, trunc_normal_
    from timm.models.swin_transformer import get_relative_position_index
except ImportError:
    def to_2tuple(x):
        """timm.layers.to_2tuple: pass iterables through, repeat scalars."""
        if isinstance(x, collections.abc.Iterable) and not isinstance(x, str):
            return tuple(x)
        return (x, x)

    def trunc_normal_(tensor, mean=0.0, std=1.0, a=-2.0, b=2.0):
        """timm.layers.trunc_normal_ (same defaults as torch's)."""
        return nn.init.trunc_normal_(tensor, mean=mean, std=std, a=a, b=b)

    def get_relative_position_index(win_h: int, win_w: int) -> torch.Tensor:
        """(win_h*win_w)^2 index into the (2*win_h-1)*(2*win_w-1) bias table.

        For window positions i=(yi,xi) and j=(yj,xj):
        index = (yi - yj + win_h - 1) * (2*win_w - 1) + (xi - xj + win_w - 1).
        """
        ys, xs = torch.meshgrid(torch.arange(win_h), torch.arange(win_w), indexing="ij")
        coords = torch.stack((ys.flatten(), xs.flatten()))        # (2, N)
        rel = coords[:, :, None] - coords[:, None, :]              # (2, N, N)
        return (rel[0] + win_h - 1) * (2 * win_w - 1) + (rel[1] + win_w - 1)


class QAttention(nn.Module):
    """timm ``Attention`` drop-in (attention.py:12-36 of the reference)."""

    def __init__(self, dim: int, num_heads: int, qkv_bias: bool = True):
        super().__init__()
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.qkv = nn.Linear(dim, dim * 3, bias=qkv_bias)
        self.proj = nn.Linear(dim, dim)
        self.int8_proj = False  # set_int8_proj: the qkv projection on int8 MFMA (not in the reference)

    def set_int8_proj(self, enabled: bool = True) -> "QAttention":
        """Opt in to the int8 QKV projection fused with the quantiser
        (qkv_int8): the qkv weight as per-channel int8 codes (taken from the
        weight now; call again after changing it), the activations quantised
        per tensor, the projection on int8 MFMA, the attention's int8 codes
        straight from its epilogue.  An approximation of the fp32 projection
        the reference computes; off by default.  Needs fp32 CUDA activations
        with C and 3C multiples of 32 and 96; other inputs take the fp32 path."""
        self.int8_proj = enabled
        if enabled:
            w8, w_scale = int8_weights(self.qkv.weight)
            self.register_buffer("qkv_w8", w8, persistent=False)
            self.register_buffer("qkv_w_scale", w_scale, persistent=False)
        return self

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None,
                is_causal: bool = False) -> torch.Tensor:
        B, N, C = x.shape
        if self.int8_proj and x.is_cuda and x.dtype == torch.float32 and C % 32 == 0 \
                and self.qkv.weight.device == x.device:
            q8, k8, v8, scales = qkv_int8(x, self.qkv_w8, self.qkv_w_scale,
                                          None if self.qkv.bias is None else self.qkv.bias.detach(), self.num_heads)
            x = forward_codes(q8, k8, v8, scales, attn_mask, (1.0 / self.head_dim ** 0.5) * LOG2E)
            return self.proj(x.transpose(1, 2).reshape(B, N, C))
        qkv = self.qkv(x).reshape(B, N, 3, self.num_heads, self.head_dim).permute(2, 0, 3, 1, 4)
        q, k, v = qkv.unbind(0)           # (B, H, N, hd) views, token-major in memory
        x = qflash.forward(q, k, v, attn_mask=attn_mask)
        return self.proj(x.transpose(1, 2).reshape(B, N, C))

    @classmethod
    def from_orig(cls, src: nn.Module) -> "QAttention":
        new = cls(dim=src.qkv.in_features, num_heads=src.num_heads, qkv_bias=src.qkv.bias is not None)
        new = new.to(device=src.qkv.weight.device, dtype=src.qkv.weight.dtype)
        new.load_state_dict(src.state_dict())
        return new


class QWindowAttention(nn.Module):
    """timm ``WindowAttention`` drop-in (attention.py:39-86 of the reference)."""

    def __init__(self, dim: int, num_heads: int, window_size, qkv_bias: bool = True):
        super().__init__()
        self.dim = dim
        self.num_heads = num_heads
        self.window_size = to_2tuple(window_size)
        win_h, win_w = self.window_size
        self.window_area = win_h * win_w
        self.relative_position_bias_table = nn.Parameter(torch.empty((2 * win_h - 1) * (2 * win_w - 1), num_heads))
        self.register_buffer("relative_position_index", get_relative_position_index(win_h, win_w), persistent=False)
        self.qkv = nn.Linear(dim, dim * 3, bias=qkv_bias)
        self.proj = nn.Linear(dim, dim)
        trunc_normal_(self.relative_position_bias_table, std=.02)

    def _get_rel_pos_bias(self) -> torch.Tensor:
        bias = self.relative_position_bias_table[self.relative_position_index.view(-1)]
        bias = bias.view(self.window_area, self.window_area, -1).permute(2, 0, 1).contiguous()
        return bias.unsqueeze(0)         # (1, H, N, N)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        B_, N, C = x.shape
        qkv = self.qkv(x).reshape(B_, N, 3, self.num_heads, -1).permute(2, 0, 3, 1, 4)
        q, k, v = qkv.unbind(0)
        # The reference adds the (nW, N, N) shift mask to the (1, H, N, N) bias
        # as a materialised (B_, H, N, N) tensor; its values repeat every nW
        # windows, and qflash_forward_window gives the same codes from the nW
        # distinct slices.
        x = qflash_forward_window(q, k, v, self._get_rel_pos_bias(), mask)
        return self.proj(x.transpose(1, 2).reshape(B_, N, -1))

    @classmethod
    def from_orig(cls, src: nn.Module) -> "QWindowAttention":
        new = cls(dim=src.dim, num_heads=src.num_heads, window_size=src.window_size,
                  qkv_bias=src.qkv.bias is not None)
        new = new.to(device=src.qkv.weight.device, dtype=src.qkv.weight.dtype)
        new.load_state_dict(src.state_dict())
        return new


def patch_attention(model: nn.Module, attn_types: Optional[Iterable[type]] = None,
                    window_attn_types: Optional[Iterable[type]] = None) -> Dict[str, int]:
    """Replace timm Attention / WindowAttention modules in place (attention.py:89-108).

    Returns {"attn": n, "wattn": m}.  By default the classes are timm's
    (``timm.layers.attention.Attention``, ``timm.models.swin_transformer.
    WindowAttention``), which requires timm; ``attn_types`` /
    ``window_attn_types`` let a caller name other classes with the same
    structure.
    """
    if attn_types is None or window_attn_types is None:
        import timm.layers.attention as _ta
        import timm.models.swin_transformer as _ts
        attn_types = (_ta.Attention,) if attn_types is None else attn_types
        window_attn_types = (_ts.WindowAttention,) if window_attn_types is None else window_attn_types
    attn_types, window_attn_types = tuple(attn_types), tuple(window_attn_types)

    targets = []
    for name, module in model.named_modules():
        if isinstance(module, attn_types):
            targets.append((name, "attn"))
        elif isinstance(module, window_attn_types):
            targets.append((name, "wattn"))

    counts = {"attn": 0, "wattn": 0}
    for name, kind in targets:
        parent_name, _, child_name = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        src = getattr(parent, child_name)
        new = (QAttention if kind == "attn" else QWindowAttention).from_orig(src)
        setattr(parent, child_name, new)
        counts[kind] += 1
    return counts
