"""Synthetic workloads of the benchmark configurations (cfg1-cfg5).

Inputs follow the benchmark definition: per tensor, fp32 N(0, 1) drawn
token-major as (B, N, H*D) from a seeded CPU generator, round(0.02*H*D)
(at least 1) channels picked by randperm and scaled x8, then viewed as
(B, H, N, D).  cfg4 (Swin-T windows) adds a (13*13, H) relative-position
bias table ~ N(0, 0.02) and a 4-region shift mask (-100 between regions) on
windows 32..63 of each image, combined as QWindowAttention does it
(qflash/attention.py:68-72).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Config:
    name: str
    Z: int            # batch (or windows for Swin)
    H: int
    N: int
    D: int
    dtype: torch.dtype = torch.float32
    swin: bool = False
    images: int = 0   # Swin: images; Z = images * windows
    windows: int = 0
    window: int = 7

    @property
    def ops(self) -> int:
        """Algorithmic int8 ops per call: two N x N x D GEMMs, 2 ops per MAC."""
        return 4 * self.Z * self.H * self.N * self.N * self.D

    @property
    def bytes_min(self) -> int:
        """Q, K, V and O int8 codes (+ the unique Swin bias entries)."""
        b = 4 * self.Z * self.H * self.N * self.D
        if self.swin:
            b += self.windows * self.H * self.N * self.N * 4
        return b


CONFIGS = {
    "cfg1": Config("DeiT-T B8 H3 N197 d64", 8, 3, 197, 64),
    "cfg2": Config("ViT-S B64 H6 N197 d64 (fp16)", 64, 6, 197, 64, dtype=torch.float16),
    "cfg3": Config("ViT-B/384 B64 H12 N577 d64", 64, 12, 577, 64),
    "cfg4": Config("Swin-T 7x7 windows 64x64 H3 N49 d32", 4096, 3, 49, 32, swin=True, images=64, windows=64),
    "cfg5": Config("long B8 H16 N4096 d64", 8, 16, 4096, 64),
}
HEADLINE = "cfg3"


def outlier_tensor(g: torch.Generator, B: int, H: int, N: int, D: int, frac: float = 0.02,
                   factor: float = 8.0) -> torch.Tensor:
    x = torch.randn(B, N, H * D, generator=g)
    n_out = max(1, int(round(frac * H * D)))
    ch = torch.randperm(H * D, generator=g)[:n_out]
    x[:, :, ch] *= factor
    return x.view(B, N, H, D).permute(0, 2, 1, 3)


def relative_position_index(ws: int) -> torch.Tensor:
    ys, xs = torch.meshgrid(torch.arange(ws), torch.arange(ws), indexing="ij")
    c = torch.stack((ys.flatten(), xs.flatten()))
    rel = c[:, :, None] - c[:, None, :]
    return (rel[0] + ws - 1) * (2 * ws - 1) + (rel[1] + ws - 1)


def swin_parts(g: torch.Generator, H: int, ws: int, windows: int):
    """QWindowAttention's two mask inputs: the (1, H, N, N) relative-position
    bias gathered from a (2ws-1)^2 x H table ~ N(0, 0.02), and the (windows, N, N)
    shift mask (-100 between the 4 regions on the second half of the windows)."""
    N = ws * ws
    table = torch.randn((2 * ws - 1) ** 2, H, generator=g) * 0.02
    bias = table[relative_position_index(ws).view(-1)].view(N, N, H).permute(2, 0, 1).contiguous().unsqueeze(0)
    ys, xs = torch.meshgrid(torch.arange(ws), torch.arange(ws), indexing="ij")
    split = ws - ws // 2  # shift = ws // 2 -> regions split at row / column ws - shift
    region = ((ys.flatten() >= split).long() * 2 + (xs.flatten() >= split).long())
    m4 = (region[:, None] != region[None, :]).float() * -100.0
    mask = torch.zeros(windows, N, N)
    mask[windows // 2:] = m4
    return bias, mask


def swin_attn_mask(g: torch.Generator, H: int, ws: int, images: int, windows: int) -> torch.Tensor:
    """(images*windows, H, N, N) fp32 mask = rel-pos bias + shift mask, composed
    as QWindowAttention does (qflash/attention.py:68-72)."""
    N = ws * ws
    bias, mask = swin_parts(g, H, ws, windows)
    mask = mask.view(1, windows, 1, N, N).expand(images, -1, H, -1, -1)
    return bias + mask.reshape(-1, H, N, N)


def make_window_parts(cfg: Config, seed: int):
    """(rel_bias, shift_mask) of a Swin config, drawn exactly as make_inputs draws
    the composed mask (same generator sequence after Q, K, V)."""
    g = torch.Generator().manual_seed(seed)
    for _ in range(3):
        outlier_tensor(g, cfg.Z, cfg.H, cfg.N, cfg.D)
    return swin_parts(g, cfg.H, cfg.window, cfg.windows)


def make_inputs(cfg: Config, seed: int, token_major: bool = True):
    """fp Q, K, V (B, H, N, D) in cfg.dtype (token-major views) and the fp32 mask or None."""
    g = torch.Generator().manual_seed(seed)
    q, k, v = (outlier_tensor(g, cfg.Z, cfg.H, cfg.N, cfg.D) for _ in range(3))
    if not token_major:
        q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    mask = swin_attn_mask(g, cfg.H, cfg.window, cfg.images, cfg.windows) if cfg.swin else None
    if cfg.dtype != torch.float32:
        q, k, v = q.to(cfg.dtype), k.to(cfg.dtype), v.to(cfg.dtype)
    return q, k, v, mask
