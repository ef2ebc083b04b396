"""GPU parity of the int8 QKV projection fused with the quantiser
(qflash_hip_qkv_int8, QAttention.set_int8_proj): no counterpart in the
reference; checked against oracle.qkv_int8_ref and, at the ViT-B/384 shape,
against the materialised projection through the device quantiser."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle.qflash_oracle import qkv_int8_ref, sqnr_db

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _fused(x8: torch.Tensor, w8, w_scale, bias, x_scale: torch.Tensor):
    """The C entry on device operands: (codes (M, Nc) int8, scales (4,) fp32)."""
    from qflash_amd import _lib
    from qflash_amd.kernel import _scales_workspace, _stream_ptr
    M, K = x8.shape
    Nc = w8.shape[0]
    codes = torch.empty((M, Nc), dtype=torch.int8, device=DEV)
    scales = torch.empty(4, dtype=torch.float32, device=DEV)
    ws = _scales_workspace(x8.device)
    vp = ctypes.c_void_p
    rc = _lib.load().qflash_hip_qkv_int8(vp(x8.data_ptr()), vp(w8.data_ptr()), vp(w_scale.data_ptr()),
                                         vp(0 if bias is None else bias.data_ptr()), vp(x_scale.data_ptr()), M, K,
                                         Nc, vp(scales.data_ptr()), vp(codes.data_ptr()), vp(ws.data_ptr()),
                                         ws.numel(), _stream_ptr(x8))
    _lib.check(rc, "qflash_hip_qkv_int8")
    torch.cuda.synchronize()
    return codes, scales


@pytest.mark.parametrize("M,K,C", [(1, 32, 32), (77, 64, 32), (300, 96, 96), (129, 768, 256), (640, 192, 64)])
@pytest.mark.parametrize("bias", [True, False])
def test_fused_projection_vs_oracle(M, K, C, bias):
    print(f"[case] M={M} K={K} C={C} bias={bias}", flush=True)
    g = np.random.default_rng(M + K + C + bias)
    x8 = g.integers(-128, 128, (M, K)).astype(np.int8)
    w8 = g.integers(-128, 128, (3 * C, K)).astype(np.int8)
    x_scale = np.float32(g.uniform(0.005, 0.05))
    w_scale = g.uniform(1e-4, 3e-3, 3 * C).astype(np.float32)
    b = g.normal(0, 2.0, 3 * C).astype(np.float32) if bias else None
    want_codes, want_scales = qkv_int8_ref(x8, w8, x_scale, w_scale, b)
    codes, scales = _fused(torch.from_numpy(x8).to(DEV), torch.from_numpy(w8).to(DEV),
                           torch.from_numpy(w_scale).to(DEV), None if b is None else torch.from_numpy(b).to(DEV),
                           torch.tensor([x_scale], device=DEV))
    np.testing.assert_array_equal(scales.cpu().numpy(), want_scales)
    np.testing.assert_array_equal(codes.cpu().numpy(), want_codes)


def test_fused_projection_zero_columns():
    """A third whose weights are all zero and no bias: scale 0, codes 0 (0 / 0)."""
    g = np.random.default_rng(3)
    M, K, C = 100, 64, 32
    x8 = g.integers(-128, 128, (M, K)).astype(np.int8)
    w8 = g.integers(-128, 128, (3 * C, K)).astype(np.int8)
    w8[C:2 * C] = 0
    w_scale = np.full(3 * C, 1e-3, np.float32)
    want_codes, want_scales = qkv_int8_ref(x8, w8, np.float32(0.01), w_scale)
    assert want_scales[1] == 0
    codes, scales = _fused(torch.from_numpy(x8).to(DEV), torch.from_numpy(w8).to(DEV),
                           torch.from_numpy(w_scale).to(DEV), None, torch.tensor([0.01], device=DEV))
    np.testing.assert_array_equal(scales.cpu().numpy(), want_scales)
    np.testing.assert_array_equal(codes.cpu().numpy(), want_codes)


def test_qkv_int8_vit_b_shape_vs_materialised_projection():
    """B=64, N=577, C=768, H=12 (cfg3's projection): the fused codes and scales
    equal quantize_qkv applied to the projection materialised with torch ops
    (the int32 products through an exact float64 matmul, then the same two
    fp32 roundings)."""
    from qflash_amd.kernel import int8_weights, qkv_int8, quantize_qkv
    torch.manual_seed(0)
    B, N, C, H = 64, 577, 768, 12
    x = torch.randn(B, N, C, device=DEV)
    x[..., ::50] *= 8
    w = torch.randn(3 * C, C, device=DEV) * 0.03
    bias = torch.randn(3 * C, device=DEV) * 0.1
    w8, w_scale = int8_weights(w)
    q8, k8, v8, scales = qkv_int8(x, w8, w_scale, bias, H)
    # materialised: the activations' codes as qkv_int8 forms them, then y, then the quantiser
    x4 = x.reshape(1, 1, B * N, C)
    one = x4.reshape(-1)[:1].view(1, 1, 1, 1)
    xs, fin = quantize_qkv(x4, one, one)
    x8 = fin()[0].reshape(B * N, C)
    acc = x8.double() @ w8.double().t()
    y = (acc.float() * (xs[0] * w_scale)) + bias
    y = y.reshape(B, N, 3, H, C // H).permute(2, 0, 3, 1, 4)
    ref_scales, ref_fin = quantize_qkv(y[0], y[1], y[2])
    rq, rk, rv = ref_fin()
    torch.cuda.synchronize()
    assert torch.equal(scales.cpu(), ref_scales.cpu())
    for a, r in ((q8, rq), (k8, rk), (v8, rv)):
        assert torch.equal(a.cpu(), r.cpu())


def test_qattention_int8_projection_runs_and_tracks_fp32():
    """QAttention with the int8 projection against the same module in fp32:
    an approximation, so only its SQNR is checked (and that the codes path,
    not the fp32 one, ran: the outputs differ)."""
    from qflash_amd.attention import QAttention
    torch.manual_seed(1)
    m = QAttention(384, 6).to(DEV)
    x = torch.randn(8, 197, 384, device=DEV)
    with torch.no_grad():
        ref = m(x)
        m.set_int8_proj(True)
        out = m(x)
    torch.cuda.synchronize()
    assert not torch.equal(ref, out)
    db = sqnr_db(ref.double().cpu().numpy(), out.double().cpu().numpy())
    print(f"[case] int8 projection SQNR vs fp32 projection: {db:.2f} dB", flush=True)
    assert db > 3.0
