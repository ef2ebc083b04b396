"""Host logic of qflash_amd.kernel against the reference's own launch records (CPU).

Every golden case recorded what the reference's ``qflash_forward`` handed to its
kernel (qflash/kernel.py:275-346): int8 operands, the five fixed-point constants
and the int32 bias.  The product's host code must produce the same values from
the same fp inputs, and raise where the reference raises.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from golden_io import load_cases
from qflash_amd import _lib
from qflash_amd.kernel import (INT8_MAX, LOG2E, NEG_INF, bias_values, fixed_point_constants, mask_to_bias, qflash,
                               qflash_forward, qflash_kernel, qflash_masked_kernel, quantize)

CASES = load_cases()
FP = sorted(n for n, c in CASES.items() if c.has_fp)


def _host_side(c):
    """The product's host computation on the case's recorded fp inputs."""
    q, k, v = (torch.from_numpy(np.ascontiguousarray(c[n])) for n in ("q_fp", "k_fp", "v_fp"))
    D = q.shape[-1]
    scale = float(c["scale_arg"])
    scale = (1.0 / D ** 0.5 if math.isnan(scale) else scale) * LOG2E
    qs, ks, vs = (x.abs().amax() / INT8_MAX for x in (q, k, v))
    sm_scale = scale * (qs * ks).item()
    f = c.flags
    consts = fixed_point_constants(sm_scale, f.l_shift, f.acc_shift)
    return q, k, v, (qs, ks, vs), sm_scale, consts


@pytest.mark.parametrize("name", FP)
def test_constants_and_quantisation_match_reference_launch(name):
    c = CASES[name]
    q, k, v, (qs, ks, vs), sm_scale, consts = _host_side(c)
    assert list(consts) == [int(x) for x in c["consts"]]
    for x, s, key in ((q, qs, "q_i8"), (k, ks, "k_i8"), (v, vs, "v_i8")):
        np.testing.assert_array_equal(quantize(x, s).numpy(), c[key])
    if c.masked:
        Z, H, N = q.shape[:3]
        mask = torch.from_numpy(np.ascontiguousarray(c["mask"]))
        bias = mask_to_bias(mask, sm_scale, Z, H, N)
        np.testing.assert_array_equal(bias.contiguous().numpy(), c["bias_i32"])
        assert bias.shape == (Z, H, N, N)


def test_fp16_inputs_keep_their_dtype_through_quantisation():
    names = [n for n in FP if str(CASES[n]["in_dtype"]) == "torch.float16"]
    assert names, "no fp16 golden case"
    c = CASES[names[0]]
    assert c["q_fp"].dtype == np.float16
    q, _, _, (qs, _, _), _, _ = _host_side(c)
    assert q.dtype == torch.float16 and qs.dtype == torch.float16
    np.testing.assert_array_equal(quantize(q, qs).numpy(), c["q_i8"])


def test_broadcast_bias_is_a_strided_view():
    """A (1,1,N,N) mask becomes a stride-0 view of (Z,H,N,N): no materialised copy."""
    m = torch.rand(1, 1, 9, 9) > 0.3
    b = mask_to_bias(m, 0.01, 4, 3, 9)
    assert b.shape == (4, 3, 9, 9) and b.stride()[:2] == (0, 0)
    assert (b[2, 1][~m[0, 0]] == NEG_INF).all() and (b[2, 1][m[0, 0]] == 0).all()
    dense = mask_to_bias(m, 0.01, 4, 3, 9, materialize=True)
    assert dense.is_contiguous() and torch.equal(dense, b)


def test_float_mask_threshold_and_rounding():
    """Values < -1e2 are masked to NEG_INF; others become round(x*log2e/sm_scale)."""
    m = torch.tensor([[-100.0, -100.5, 0.25, -0.3, 1e-3]]).view(1, 1, 1, 5)
    sm = 0.05
    b = mask_to_bias(m, sm, 1, 1, 5)[0, 0, 3].tolist()
    want = [round(-100.0 * LOG2E / sm), NEG_INF, round(0.25 * LOG2E / sm), round(-0.3 * LOG2E / sm), 0]
    assert b == want


@pytest.mark.parametrize("sm_scale,exc", [(0.0, ZeroDivisionError), (float("nan"), ValueError),
                                          (float("inf"), OverflowError)])
def test_constants_raise_like_the_reference(sm_scale, exc):
    """int(round(1/sm_scale)) raises for 0, NaN and inf (kernel.py:300)."""
    with pytest.raises(exc):
        fixed_point_constants(sm_scale)


def test_constants_closed_form():
    s = 0.0123
    rs, eM, rM, lM, aM = fixed_point_constants(s, 30, 24)
    assert rs == 81 and eM == round(-s * 65536) and rM == round(s * 127 * 65536)
    assert lM == round(2 ** 30 / 81) and aM == round(2 ** 24 / 81)
    # half-to-even: 1/0.4 = 2.5 -> 2
    assert fixed_point_constants(0.4)[0] == 2
    # sm_scale > 2 gives sm_rscale = 0 -> l_M raises ZeroDivisionError like the reference
    with pytest.raises(ZeroDivisionError):
        fixed_point_constants(2.5)


def test_forward_rejects_head_dims_like_the_reference():
    x = torch.zeros(1, 1, 4, 48)
    with pytest.raises(AssertionError):
        qflash_forward(x, x, x)
    with pytest.raises(AssertionError):
        qflash_forward(torch.zeros(1, 1, 4, 32), torch.zeros(1, 1, 4, 64), torch.zeros(1, 1, 4, 64))


def test_forward_on_cpu_tensors_raises_not_falls_back():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 2, 40, 32, generator=g)
    with pytest.raises(ValueError, match="GPU"):
        qflash_forward(x, x, x)
    with pytest.raises(ValueError, match="GPU"):
        qflash_forward(x, x, x, attn_mask=torch.ones(40, 40, dtype=torch.bool))


def test_launcher_checks_argument_count_and_int32_range():
    t = torch.zeros(1, 1, 32, 32, dtype=torch.int8)
    with pytest.raises(TypeError, match="positional"):
        qflash_kernel[None](t, t, t, t, 1, 2, 3, N_CTX=32, HEAD_DIM=32)
    args = [t, t, t, t, 1, -1, 1, 1, 1] + [0] * 16 + [1, 1]
    with pytest.raises(ValueError, match="GPU"):
        qflash_kernel[None](*args, N_CTX=32, HEAD_DIM=32)
    args_m = [t, t, t, t, t.int(), 1 << 31, -1, 1, 1, 1] + [0] * 20 + [1, 1]
    with pytest.raises(ValueError, match="GPU"):
        qflash_masked_kernel[(1, 1)](*args_m, N_CTX=32, HEAD_DIM=32)
    with pytest.raises(_lib.QFlashLibraryError, match="int32"):
        _int32_check_only(sm_rscale=1 << 31)


def _int32_check_only(**kw):
    from qflash_amd.kernel import _check_i32
    _check_i32(**kw)


def test_op_namespace_matches_reference():
    """class qflash: kernel = [unmasked, masked], forward = qflash_forward (kernel.py:354-356)."""
    assert qflash.forward is qflash_forward
    assert qflash.kernel == [qflash_kernel, qflash_masked_kernel]
    import qflash_amd
    assert qflash_amd.qflash is qflash


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setenv("QFLASH_HIP_LIB", str(tmp_path / "absent.so"))
    with pytest.raises(_lib.QFlashLibraryError, match="not built"):
        _lib.load()


def test_environment_flags_are_read_at_import():
    """QFLASH_* arithmetic switches (kernel.py:30-36) are module constants read once
    at import (checked in a child process so this one keeps its defaults)."""
    import os
    import subprocess
    import sys

    code = ("import qflash_amd.kernel as K; "
            "print(K.EXP_USE_SHIFT, K.L_USE_SHIFT, K.ACC_USE_SHIFT, K.L_SHIFT, K.ACC_SHIFT)")
    env = dict(os.environ, QFLASH_EXP_USE_SHIFT="0", QFLASH_L_SHIFT="20")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = subprocess.run([sys.executable, "-c", code], env=env, cwd=root, capture_output=True, text=True,
                         check=True).stdout.split()
    assert out == ["False", "True", "True", "20", "30"]
    import qflash_amd.kernel as K
    assert (K.EXP_USE_SHIFT, K.L_SHIFT, K.ACC_SHIFT) == (True, 30, 30)


def _shift_mask(ws=7):
    ys, xs = torch.meshgrid(torch.arange(ws), torch.arange(ws), indexing="ij")
    region = (ys.flatten() >= ws - ws // 2).long() * 2 + (xs.flatten() >= ws - ws // 2).long()
    return (region[:, None] != region[None, :]).float() * -100.0


@pytest.mark.parametrize("sm_scale", [0.0123, 0.09, 0.5])
def test_window_bias_equals_materialised_bias(sm_scale):
    """The window path's (nW, H, N, N) bias, indexed by z % nW, equals the bias of
    the reference's materialised (B_, H, N, N) mask element for element."""
    g = torch.Generator().manual_seed(4)
    H, N, nW, B = 3, 49, 4, 3
    rel = torch.randn(1, H, N, N, generator=g) * 0.02
    rel[0, 0, :3, :3] = -100.0                       # sums exactly at / beyond the -1e2 boundary
    rel[0, 1, :3, :3] = 100.0
    shift = torch.zeros(nW, N, N)
    shift[nW // 2:] = _shift_mask()
    shift[1, 5, :] = torch.randn(N, generator=g)     # arbitrary float mask values too
    full = rel + shift.view(1, nW, 1, N, N).expand(B, -1, H, -1, -1).reshape(-1, H, N, N)
    want = mask_to_bias(full, sm_scale, B * nW, H, N, materialize=True)
    compact = bias_values(rel + shift.view(nW, 1, N, N), sm_scale)
    assert compact.shape == (nW, H, N, N)
    for z in range(B * nW):
        assert torch.equal(compact[z % nW], want[z]), z


def test_swin_golden_mask_decomposes_into_window_parts():
    """The golden Swin case's (4, 3, 49, 49) mask is rel_bias + shift mask of 2
    windows (window 0 unshifted), exactly: the window path sees the same sums."""
    c = CASES["swin_N49_D32"]
    full = torch.from_numpy(c["mask"])
    rel = full[0:1].clone()
    shift = torch.zeros(2, 49, 49)
    shift[1] = _shift_mask()
    composed = rel + shift.view(1, 2, 1, 49, 49).expand(2, -1, 3, -1, -1).reshape(-1, 3, 49, 49)
    assert torch.equal(composed, full)


def test_status_words_raise_the_reference_exceptions():
    """The status of qflash_hip_constants maps to the exception the reference's
    host raises for the same value (kernel.py:302-307), in its order."""
    from qflash_amd.kernel import raise_status
    raise_status(0)
    for code, exc, value in ((_lib.STATUS_ZERODIV_SCALE, ZeroDivisionError, 0.0),
                             (_lib.STATUS_NAN, ValueError, float("nan")),
                             (_lib.STATUS_INF, OverflowError, float("inf")),
                             (_lib.STATUS_ZERODIV_RSCALE, ZeroDivisionError, 2.0)):
        with pytest.raises(exc):
            raise_status(code)
        with pytest.raises(exc):  # the host arithmetic on a value that produces it
            fixed_point_constants(value, 30, 30)
    with pytest.raises(_lib.QFlashLibraryError):
        raise_status(_lib.STATUS_RANGE)
