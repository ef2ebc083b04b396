"""GPU: the device absmax / quantisation passes (qflash_hip_scales, qflash_hip_quantize)
against torch's own GPU ops, bit for bit (qflash/kernel.py:294-311)."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _torch_ref(q, k, v):
    qs, ks, vs = (x.abs().amax() / 127 for x in (q, k, v))
    codes = [torch.clamp(torch.round(x / s), -128, 127).to(torch.int8) for x, s in ((q, qs), (k, ks), (v, vs))]
    return torch.stack([qs, ks, vs, qs * ks]), codes


def _layouts(B, H, N, D, dtype, g):
    """Contiguous (B,H,N,D), token-major views of one qkv buffer (the module
    path), and a layout with a non-unit head-dim stride."""
    x = (torch.randn(B, N, 3 * H * D, generator=g) * 3).to(dtype).to(DEV)
    x[..., :7] *= 8
    qkv = x.view(B, N, 3, H, D).permute(2, 0, 3, 1, 4)
    yield "token-major", tuple(qkv.unbind(0))
    yield "contiguous", tuple(t.contiguous() for t in qkv.unbind(0))
    t = (torch.randn(B, H, D, N, generator=g)).to(dtype).to(DEV).transpose(-1, -2)
    yield "column-strided", (t, t * 2, t - 1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 3, 197, 64), (1, 4, 577, 64), (3, 2, 49, 32), (1, 2, 33, 128)])
def test_scales_and_codes_match_torch(dtype, shape):
    from qflash_amd.kernel import quantize_qkv
    g = torch.Generator().manual_seed(sum(shape))
    for name, (q, k, v) in _layouts(*shape, dtype, g):
        want_scales, want_codes = _torch_ref(q, k, v)
        scales, finish = quantize_qkv(q, k, v)
        codes = finish()
        torch.cuda.synchronize()
        assert scales.dtype == dtype
        assert torch.equal(scales, want_scales), (name, scales, want_scales)
        for c, w, x in zip(codes, want_codes, (q, k, v)):
            assert c.stride() == w.stride() == torch.empty_like(x, dtype=torch.int8).stride(), name
            assert torch.equal(c, w), name


def test_scale_of_a_constant_tensor_and_ties():
    """Values that land exactly on .5 after the division round half to even."""
    from qflash_amd.kernel import quantize_qkv
    q = torch.full((1, 1, 32, 32), 127.0, device=DEV)
    q[0, 0, 0, :8] = torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -127.5])
    k = torch.arange(32 * 32, dtype=torch.float32, device=DEV).view(1, 1, 32, 32) - 500
    scales, finish = quantize_qkv(q, k, q)
    want_scales, want_codes = _torch_ref(q, k, q)
    codes = finish()
    assert torch.equal(scales, want_scales)
    for c, w in zip(codes, want_codes):
        assert torch.equal(c, w)


def test_forward_uses_the_device_passes_and_matches_torch_sequence():
    """qflash.forward (device quantiser) == the attention kernel fed with torch's codes."""
    from qflash_amd import qflash
    from qflash_amd.kernel import LOG2E, fixed_point_constants, qflash_kernel
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 197, 3 * 6 * 64, generator=g).to(DEV)
    q, k, v = x.view(2, 197, 3, 6, 64).permute(2, 0, 3, 1, 4).unbind(0)
    out = qflash.forward(q, k, v)
    (qs, ks, vs, qk), (q8, k8, v8) = _torch_ref(q, k, v)
    consts = fixed_point_constants((1 / 8) * LOG2E * qk.item())
    o = torch.empty_like(v8)
    qflash_kernel[None](q8, k8, v8, o, *consts, *q8.stride(), *k8.stride(), *v8.stride(), *o.stride(), 2, 6,
                        N_CTX=197, HEAD_DIM=64, L_SHIFT=30, ACC_SHIFT=30)
    torch.cuda.synchronize()
    assert torch.equal(out, o * vs)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("masked", [False, True])
def test_fused_dequantisation_equals_codes_times_scale(dtype, masked):
    """The kernel's fused `o * o_scale` (fp32 / fp16 / bf16 stores) equals torch's
    product of the int8 codes with the scale, for the fast and general kernels."""
    from qflash_amd.kernel import (LOG2E, fixed_point_constants, launch_forward, mask_to_bias, quantize_qkv)
    g = torch.Generator().manual_seed(8)
    Z, H, N, D = 2, 3, 100, 64
    q, k, v = ((torch.randn(Z, N, H, D, generator=g) * 2).to(dtype).to(DEV).permute(0, 2, 1, 3) for _ in range(3))
    scales, finish = quantize_qkv(q, k, v)
    consts = fixed_point_constants((1 / 8) * LOG2E * scales[3].item())
    q8, k8, v8 = finish()
    bias = None
    if masked:
        m = torch.rand(N, N, generator=g) > 0.2
        bias = mask_to_bias(m.to(DEV), 0.01, Z, H, N)
    flags = dict(EXP_USE_SHIFT=True, L_USE_SHIFT=True, ACC_USE_SHIFT=True, L_SHIFT=30, ACC_SHIFT=30)
    from qflash_amd import _lib
    for general in (False, True):
        prev = _lib.set_test_hooks(*(("FORCE_GENERAL",) if general else ()))
        try:
            o8 = torch.empty_like(v8)
            launch_forward(q8, k8, v8, o8, consts, flags, bias)
            out = torch.empty_like(v8, dtype=dtype)
            launch_forward(q8, k8, v8, out, consts, flags, bias, o_scale=scales[2])
        finally:
            _lib.load().qflash_hip_set_test_hooks(prev)
        torch.cuda.synchronize()
        want = o8 * scales[2]
        assert want.dtype == dtype and want.stride() == out.stride()
        assert torch.equal(out, want), (dtype, masked, general)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_codes_near_half_integers_match_torch(seed):
    """fp32 quantisation goes through the reciprocal of the scale except near
    half-integer quotients: values on, just above and just below (k + 1/2)*s
    for every k, and their float neighbours, must round as torch's division."""
    from qflash_amd.kernel import quantize_qkv
    g = torch.Generator().manual_seed(seed)
    amax = float(torch.empty(1).uniform_(0.5, 40.0, generator=g))
    s = torch.tensor(amax) / 127  # the scale the device computes from amax
    ks = torch.arange(-129, 129, dtype=torch.float32) + 0.5
    base = (ks * s).to(torch.float32)
    up = torch.nextafter(base, torch.tensor(float("inf")))
    dn = torch.nextafter(base, torch.tensor(float("-inf")))
    vals = torch.cat([base, up, dn, torch.nextafter(up, torch.tensor(float("inf"))),
                      torch.nextafter(dn, torch.tensor(float("-inf")))])
    vals = vals.clamp(-amax, amax)
    n = 32 * 64
    q = torch.empty(n).uniform_(-amax, amax, generator=g)
    q[: vals.numel()] = vals
    q[-1] = amax  # fixes the absmax
    q = q.view(1, 1, 32, 64).to(DEV)
    k = (torch.randn(1, 1, 32, 64, generator=g) * 5).to(DEV)
    want_scales, want_codes = _torch_ref(q, k, q)
    scales, finish = quantize_qkv(q, k, q)
    codes = finish()
    assert torch.equal(scales, want_scales)
    for c, w in zip(codes, want_codes):
        assert torch.equal(c, w)
