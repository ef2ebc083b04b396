"""GPU: the fixed-point constants formed on the device (qflash_hip_constants)
equal the host's Python arithmetic (qflash/kernel.py:297-307) value for value,
raise where it raises, and make a whole forward capturable in a HIP graph."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from qflash_amd import _lib
from qflash_amd.kernel import LOG2E, device_constants, fixed_point_constants, qflash, raise_status

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _host(sm):
    """fixed_point_constants, or the exception type and the int32 range check."""
    try:
        c = fixed_point_constants(sm, 30, 30)
    except (ZeroDivisionError, ValueError, OverflowError) as e:
        return type(e), str(e)
    if any(not (-(1 << 31) <= x < (1 << 31)) for x in c):
        return _lib.QFlashLibraryError, "int32"
    return c


def _device(qk, dtype, scale=1.0, N=577, D=64, masked=False):
    scales = torch.tensor([1.0, 1.0, 1.0, qk], dtype=dtype, device=DEV)
    p = device_constants(scales, scale, N, D, masked).cpu().tolist()
    if p[0]:
        try:
            raise_status(p[0])
        except Exception as e:  # noqa: BLE001 - the mapping under test
            return type(e), str(e)
    return tuple(p[1:6])


SWEEP = ([2.5 / 65536, 3.5 / 65536, 0.4, 2.0, 1.9, 0.0, float("nan"), float("inf"), 1e-38, 3.0]
         + list(np.random.default_rng(0).uniform(1e-5, 2e-3, 40)) + list(np.geomspace(1e-6, 4.0, 60)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_device_constants_equal_host_arithmetic(dtype):
    """Every value of the sweep (half-to-even ties -2.5 / -3.5 / 444.5, 1/sm_scale
    = 0.5 -> sm_rscale 0, sm_scale 0, NaN, inf, tiny, > 2, random and
    geometric scales, both `scale` forms) gives the host's constants or its
    exception, through the input dtype's rounding of q_scale * k_scale."""
    for qk in SWEEP:
        q = torch.tensor(qk, dtype=dtype).item()  # the value the dtype holds, as the host reads it
        for scale in (1.0, (1.0 / math.sqrt(64)) * LOG2E):
            want = _host(scale * q)
            got = _device(qk, dtype, scale)
            if isinstance(want[0], type):
                assert isinstance(got[0], type) and got[0] is want[0], (qk, scale, got, want)
            else:
                assert got == tuple(want), (qk, scale, got, want)


def test_device_constants_ties_are_half_to_even():
    assert _device(2.5 / 65536, torch.float32)[1:3] == (-2, 318)
    assert _device(3.5 / 65536, torch.float32)[1:3] == (-4, 444)
    assert _device(2.0, torch.float32)[0] is ZeroDivisionError  # round(0.5) = 0, then 2^30 / 0


@pytest.mark.parametrize("masked", [False, True])
def test_planned_forward_equals_host_constant_forward(masked):
    """qflash.forward (device constants) equals the launch on host constants, code
    for code, through both kernels (table and general)."""
    from qflash_amd.kernel import fixed_point_constants, launch_forward, mask_to_bias, quantize
    g = torch.Generator().manual_seed(5 + masked)
    Z, H, N, D = 2, 3, 197, 64
    q, k, v = (torch.randn(Z, H, N, D, generator=g) for _ in range(3))
    mask = None
    if masked:
        mask = torch.where(torch.rand(N, N, generator=g) < 0.1, -200.0, torch.randn(N, N, generator=g))
    out = qflash.forward(q.to(DEV), k.to(DEV), v.to(DEV), attn_mask=None if mask is None else mask.to(DEV))
    qs, ks, vs = (x.abs().amax() / 127 for x in (q, k, v))
    sm = (1.0 / math.sqrt(D)) * LOG2E * (qs * ks).item()
    c = fixed_point_constants(sm, 30, 30)
    q8, k8, v8 = (quantize(x, s).to(DEV) for x, s in ((q, qs), (k, ks), (v, vs)))
    bias = None if mask is None else mask_to_bias(mask.to(DEV), sm, Z, H, N)
    o = torch.empty_like(v8)
    flags = dict(EXP_USE_SHIFT=True, L_USE_SHIFT=True, ACC_USE_SHIFT=True, L_SHIFT=30, ACC_SHIFT=30)
    launch_forward(q8, k8, v8, o, c, flags, bias)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), o.cpu().float() * vs)


@pytest.mark.parametrize("plan", ["exp_idiv", "l_idiv", "acc_idiv", "dynamic_bound", "long_rows"])
def test_planned_forward_on_every_plan(monkeypatch, hip_hooks, plan):
    """The planned attention is two launches, each of which runs only when the
    device plan selects it: fwd_fast_planned (the fast path with the identity
    proof of the rescale) and fwd_planned_rest (the per-row bound variant or
    the general path).  Plans that send the work to the second one: the idiv
    variants of kernel.py:30-36 (general path), the dynamic-bound hook (per-row
    bound) and rows of 4096 keys (where the identity proof usually fails);
    qflash.forward must equal the launch on host constants code for code."""
    from qflash_amd import kernel as K
    from qflash_amd.kernel import fixed_point_constants, launch_forward, quantize
    N = 4096 if plan == "long_rows" else 197
    flags = dict(EXP_USE_SHIFT=True, L_USE_SHIFT=True, ACC_USE_SHIFT=True, L_SHIFT=30, ACC_SHIFT=30)
    name = {"exp_idiv": "EXP_USE_SHIFT", "l_idiv": "L_USE_SHIFT", "acc_idiv": "ACC_USE_SHIFT"}.get(plan)
    if name:
        monkeypatch.setattr(K, name, False)
        flags[name] = False
    if plan == "dynamic_bound":
        hip_hooks("FORCE_DYNAMIC_BOUND")
    g = torch.Generator().manual_seed(21)
    Z, H, D = (1, 2, 64) if plan == "long_rows" else (2, 3, 64)
    q, k, v = (torch.randn(Z, H, N, D, generator=g) for _ in range(3))
    out = qflash.forward(q.to(DEV), k.to(DEV), v.to(DEV))
    qs, ks, vs = (x.abs().amax() / 127 for x in (q, k, v))
    sm = (1.0 / math.sqrt(D)) * LOG2E * (qs * ks).item()
    c = fixed_point_constants(sm, 30, 30)
    q8, k8, v8 = (quantize(x, s).to(DEV) for x, s in ((q, qs), (k, ks), (v, vs)))
    o = torch.empty_like(v8)
    launch_forward(q8, k8, v8, o, c, flags)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), o.cpu().float() * vs)


def test_forward_raises_where_the_reference_raises():
    z = torch.zeros(1, 2, 40, 32, device=DEV)
    x = torch.randn(1, 2, 40, 32, device=DEV)
    with pytest.raises(ZeroDivisionError):
        qflash.forward(z, x, x)  # q_scale = 0 -> sm_scale = 0
    with pytest.raises(ValueError):
        qflash.forward(x * float("nan"), x, x)


def test_forward_in_a_captured_graph():
    """qflash.forward captured in a HIP graph: every replay equals the eager call
    on the same inputs, also after the inputs change in place between replays
    (the scales workspace clears itself; the graph holds no memset)."""
    g = torch.Generator().manual_seed(11)
    Z, H, N, D = 2, 6, 197, 64
    q, k, v = (torch.randn(Z, H, N, D, generator=g).to(DEV) for _ in range(3))
    eager = qflash.forward(q, k, v)  # warm-up: workspaces, occupancy caches
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        qflash.forward(q, k, v)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = qflash.forward(q, k, v)
    for rep in range(4):
        if rep >= 2:  # new contents of the same buffers
            for x in (q, k, v):
                x.copy_(torch.randn(Z, H, N, D, generator=g).to(DEV) * (1 + rep))
            eager = qflash.forward(q, k, v)
            torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
        _ = (q.sum() + 1).item()  # eager work between replays


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("masked", [False, True])
def test_scales_constants_equal_the_two_calls(dtype, masked):
    """qflash_hip_scales_constants (one kernel for the scales and the constants)
    writes the scales and parameter block that qflash_hip_scales followed by
    qflash_hip_constants write, and leaves its workspace zero, over inputs whose
    products q_scale * k_scale land on different constants (and a zero tensor:
    sm_scale 0, the ZeroDivisionError status)."""
    import ctypes

    from qflash_amd.kernel import _DT_CODE, _flags, quantize_qkv

    L = _lib.load()
    g = torch.Generator().manual_seed(7)
    for trial, amp in enumerate((1.0, 3.7, 0.02, 40.0, 0.0)):
        Z, H, N, D = 2, 3, 70 + 31 * trial, 64
        q, k, v = ((torch.randn(Z, H, N, D, generator=g) * amp).to(dtype).to(DEV) for _ in range(3))
        scale = (1.0 / math.sqrt(D)) * LOG2E
        scales_a, _ = quantize_qkv(q, k, v)
        params_a = device_constants(scales_a, scale, N, D, masked)
        geo = (ctypes.c_int64 * 24)(*q.shape, *q.stride(), *k.shape, *k.stride(), *v.shape, *v.stride())
        ws = torch.zeros(_lib.SCALES_WORKSPACE, dtype=torch.int32, device=DEV)
        scales_b = torch.empty(4, dtype=dtype, device=DEV)
        params_b = torch.empty(_lib.PARAMS_WORDS, dtype=torch.int32, device=DEV)
        vp = ctypes.c_void_p
        rc = L.qflash_hip_scales_constants(vp(q.data_ptr()), vp(k.data_ptr()), vp(v.data_ptr()), _DT_CODE[dtype],
                                           geo, vp(scales_b.data_ptr()), vp(ws.data_ptr()), ws.numel(), scale, N, D,
                                           int(masked), ctypes.byref(_flags()), vp(params_b.data_ptr()),
                                           vp(torch.cuda.current_stream().cuda_stream))
        assert rc == 0, L.qflash_hip_last_error()
        torch.cuda.synchronize()
        assert torch.equal(scales_a.cpu().view(torch.int16 if dtype != torch.float32 else torch.int32),
                           scales_b.cpu().view(torch.int16 if dtype != torch.float32 else torch.int32)), trial
        assert params_a.cpu().tolist() == params_b.cpu().tolist(), trial
        assert int(ws.abs().sum()) == 0
        if amp == 0.0:
            assert params_b[0].item() == _lib.STATUS_ZERODIV_SCALE
