"""The fast kernel's exp2 + requantisation table (qflash_hip_lut_bounds), on the CPU.

The kernel reads p(u) = int8(requant(exp2(-u))) (qflash/kernel.py:40-64) from
a table that holds the computed values for u < lut_n and 0 from there on up
to its size; a step whose u exceed lut_lim (or the table) falls back to
arithmetic.
These tests check that claim against the numpy oracle by brute force over
[0, lut_lim] (capped where lut_lim is very large; the cap is stated), over a
sweep of scales covering both signs of kappa = |exp_M| * sm_rscale - 2^16.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from oracle.qflash_oracle import Consts, exp2_i32, requantize
from qflash_amd import _build, _lib
from qflash_amd.kernel import fixed_point_constants

KLUT_MAX = 4096          # bytes of LDS the kernel reserves for the table
BRUTE_CAP = 1 << 22      # brute-force range per constant set


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_build.LIB_PATH):
        pytest.fail(f"{_build.LIB_PATH} is not built (run __graft_entry__.build())")
    return _lib.load()


def _bounds(lib, c: Consts):
    n, lim = ctypes.c_int32(-1), ctypes.c_int32(-1)
    assert lib.qflash_hip_lut_bounds(c.sm_rscale, c.exp_M, c.req_M, ctypes.byref(n), ctypes.byref(lim)) == 0
    return n.value, lim.value


def _p(u, c: Consts):
    return requantize(exp2_i32(-np.asarray(u, dtype=np.int64), c), c)


SCALES = sorted(set(float(x) for x in np.geomspace(1.5e-4, 1.9, 97)) | {1 / 3.4, 1 / 2.6, 1 / 57.3, 1 / 94.2})


@pytest.mark.parametrize("sm_scale", SCALES)
def test_table_and_zero_range_match_oracle(lib, sm_scale):
    c = Consts(*fixed_point_constants(sm_scale, 30, 30))
    n, lim = _bounds(lib, c)
    if n == 0:
        # no table: the kernel computes p arithmetically.  That happens only when
        # the table would not fit or the bound does not apply.
        A, rs = -c.exp_M, c.sm_rscale
        kap = A * rs - 65536
        u0 = ((rs.bit_length() + 3) * 65536 + A - 1) // A if A > 0 else None
        assert A <= 0 or kap > 2 * A or u0 >= KLUT_MAX or u0 > min((2 ** 31 - 1) // A,
                                                                     rs * 65536 // -kap if kap < 0 else 2 ** 31)
        return
    assert 1 <= n <= KLUT_MAX and lim >= n - 1
    hi = min(lim, BRUTE_CAP)
    p = _p(np.arange(hi + 1), c)
    assert p[n - 1] == 0
    assert np.all(p[n - 1:] == 0), f"p(u) != 0 at u = {n - 1 + int(np.argmax(p[n - 1:] != 0))}"
    if n >= 2:
        assert p[n - 2] != 0  # the table is as short as it can be


def test_sweep_reaches_both_signs_of_kappa_and_small_limits(lib):
    kinds = set()
    for sm in SCALES:
        c = Consts(*fixed_point_constants(sm, 30, 30))
        n, lim = _bounds(lib, c)
        if n:
            kinds.add(("neg" if -c.exp_M * c.sm_rscale < 65536 else "nonneg", lim < 10 ** 5))
    assert ("neg", True) in kinds and ("nonneg", False) in kinds


def test_negative_kappa_limit_is_needed():
    """For kappa < 0 the zero range really ends: past rs*2^16/|kappa| (about
    twice that) p turns negative, so a table clamped without the per-step
    check would be wrong there."""
    hits = 0
    for sm in SCALES:
        c = Consts(*fixed_point_constants(sm, 30, 30))
        A, rs = -c.exp_M, c.sm_rscale
        kap = A * rs - 65536
        if A <= 0 or kap >= 0:
            continue
        lim = rs * 65536 // -kap
        top = min(4 * lim + 4 * rs, (2 ** 31 - 1) // A, BRUTE_CAP)
        if top <= lim:
            continue
        p = _p(np.arange(lim + 1, top + 1), c)
        hits += bool(np.any(p != 0))
    assert hits > 0


def test_rejects_null_outputs(lib):
    assert lib.qflash_hip_lut_bounds(57, -1146, 145571, None, None) == -1  # QFLASH_HIP_EINVAL


def _far(lib, c: Consts):
    lo, hi, p = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    assert lib.qflash_hip_far_bounds(c.sm_rscale, c.exp_M, c.req_M, ctypes.byref(lo), ctypes.byref(hi),
                                     ctypes.byref(p)) == 0
    return lo.value, hi.value, p.value


FAR_EDGE = 1 << 20       # brute-force span at each end of a far range


@pytest.mark.parametrize("sm_scale", SCALES)
def test_far_range_is_constant(lib, sm_scale):
    """The masked table path gives every column with a negative biased score
    the one value p_far, relying on p(u) = p_far for all u in [u_lo, u_hi]
    (qflash_hip_far_bounds).  Checked by brute force over FAR_EDGE values at
    each end of the range and 2^16 random ones between; the table itself
    (lut_n > 0) is the precondition of the range's use."""
    c = Consts(*fixed_point_constants(sm_scale, 30, 30))
    n, _ = _bounds(lib, c)
    lo, hi, p_far = _far(lib, c)
    if n == 0 or hi < lo:
        return
    assert hi <= min((2 ** 31 - 1) // -c.exp_M, 2 ** 30)
    rng = np.random.default_rng(int(sm_scale * 1e6))
    us = np.unique(np.concatenate([np.arange(lo, min(hi, lo + FAR_EDGE) + 1),
                                   np.arange(max(lo, hi - FAR_EDGE), hi + 1),
                                   rng.integers(lo, hi + 1, 1 << 16)]))
    p = _p(us, c)
    bad = us[p != p_far]
    assert bad.size == 0, f"p(u) != {p_far} at u = {bad[:5]}"


def test_far_constant_takes_both_values():
    """Across the sweep the far constant is 0 (kappa >= 0) and requant(-1) < 0
    (kappa < 0), and the ranges of the Swin-like scales (sm_scale ~ 0.02-0.03)
    reach -2^20 - 2^19 below a row maximum of 2^19 (biased)."""
    lib = _lib.load()
    vals, reach = set(), 0
    for sm in SCALES:
        c = Consts(*fixed_point_constants(sm, 30, 30))
        n, _ = _bounds(lib, c)
        lo, hi, p_far = _far(lib, c)
        if n and hi >= lo:
            vals.add(p_far < 0)
            if 0.015 < sm < 0.035:
                reach += lo <= (1 << 19) and hi >= (1 << 19) + (1 << 20) + (1 << 19)
    assert vals == {True, False}
    assert reach > 0


def test_far_bounds_rejects_null_outputs(lib):
    assert lib.qflash_hip_far_bounds(57, -1146, 145571, None, None, None) == -1
