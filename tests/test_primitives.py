"""Integer primitives (CPU): C vs numpy sweeps, closed-form properties, and the
algebra the gfx950 fast path relies on, checked exhaustively over its domain."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle.qflash_oracle as O
from golden_io import load_cases
from oracle import oracle_c

CASES = load_cases()
# distinct constant sets (shift variants), sorted for determinism
CONSTS = sorted({c.consts for c in CASES.values() if c.flags.exp_use_shift},
                key=lambda k: (k.sm_rscale, k.exp_M))


def _pick(pred):
    return [k for k in CONSTS if pred(k)][:2]


SWEEP = (_pick(lambda k: abs(k.exp_M) * k.sm_rscale > 65536)
         + _pick(lambda k: abs(k.exp_M) * k.sm_rscale < 65536)
         + _pick(lambda k: k.sm_rscale < 10))


@pytest.mark.parametrize("k", SWEEP, ids=lambda k: f"rs{k.sm_rscale}_eM{k.exp_M}")
def test_c_and_numpy_primitives_agree_exhaustively(k):
    """E and requant over x in [-2^22, 2^10] (every reachable real-column x for
    D <= 64, plus positive and overflow-regime values)."""
    x = np.arange(-(1 << 22), 1 << 10, dtype=np.int64)
    e_np = O.exp2_i32(x, k)
    p_np = O.requantize(e_np, k)
    e_c, p_c = oracle_c.exp2_requant(x, k)
    np.testing.assert_array_equal(e_c, e_np)
    np.testing.assert_array_equal(p_c, p_np)
    f = O.Flags(exp_use_shift=False)
    e_np2 = O.exp2_i32(x[::7], k, f)
    e_c2, _ = oracle_c.exp2_requant(x[::7], k, f)
    np.testing.assert_array_equal(e_c2, e_np2)


@pytest.mark.parametrize("k", CONSTS[:12], ids=lambda k: f"rs{k.sm_rscale}_eM{k.exp_M}")
def test_exp_closed_form_properties(k):
    rs = k.sm_rscale
    assert int(O.exp2_i32(np.array([0]), k)[0]) == rs                 # E(0) = rs
    # E(x) ~ rs * 2^(x * s) with s = -eM / 2^16: piecewise-linear 2^t in each octave
    s = -k.exp_M / 65536.0
    x = np.arange(-8 * rs, 1, dtype=np.int64)
    e = O.exp2_i32(x, k).astype(np.float64)
    ideal = rs * np.power(2.0, x * s)
    assert np.all(np.abs(e - ideal) <= 0.09 * ideal + 2.0), "exp2 approximation off"
    # requant(E(0)) = round-half-up(rs * rM / 2^16) ~ 127 (wraps as int8)
    want = ((rs * k.req_M + (1 << 15)) >> 16) & 0xFF
    want = want - 256 if want >= 128 else want
    assert int(O.requantize(np.array([rs]), k)[0]) == want


@pytest.mark.parametrize("k", CONSTS[:12], ids=lambda k: f"rs{k.sm_rscale}_eM{k.exp_M}")
def test_release_identity_and_rounding(k):
    """scale_release by alpha = rs is x * (1 + e/2^30) rounded: the identity while
    |x*e| < 2^29 (the kernel's skip rule); alpha = 0 gives 0."""
    e = k.sm_rscale * k.acc_M - (1 << 30)
    bound = (1 << 29) // max(1, abs(e)) - 1
    xs = np.array([0, 1, -1, bound, -bound, 12345, -987654], dtype=np.int64)
    xs = xs[np.abs(xs) <= bound]
    r = O.scale_release(xs, k.sm_rscale, k.acc_M, 30, True, k.sm_rscale)
    np.testing.assert_array_equal(r, xs)
    z = O.scale_release(np.array([5, -5, 1 << 20]), 0, k.acc_M, 30, True, k.sm_rscale)
    np.testing.assert_array_equal(z, [0, 0, 0])
    # C agrees on random x, alpha
    rng = np.random.default_rng(k.sm_rscale)
    x = rng.integers(-(1 << 31), 1 << 31, 4000, dtype=np.int64)
    a = rng.integers(-(1 << 31), 1 << 31, 4000, dtype=np.int64)
    for M, sh, mode in ((k.acc_M, 30, True), (k.l_M, 20, True), (k.acc_M, 30, False)):
        np.testing.assert_array_equal(oracle_c.release(x, a, M, sh, mode, k.sm_rscale),
                                      O.scale_release(x, a, M, sh, mode, k.sm_rscale))


def test_clamped_shift_semantics():
    a = np.array([5, -5, 5, -5, 5, -5, 1 << 30], dtype=np.int64)
    b = np.array([31, 31, 32, 32, -1, -1, 40], dtype=np.int64)
    np.testing.assert_array_equal(O.ashr32(a, b), [0, -1, 0, -1, 0, -1, 0])
    assert O.trunc_div(np.array([-7]), np.array([2]))[0] == -3
    assert O.cvt_i32_x86(np.float32("nan")) == O.INT_MIN
    assert O.cvt_i32_x86(np.float32(3e9)) == O.INT_MIN
    assert O.cvt_i32_x86(np.float32(-2.5)) == -2


# --- the fast path's algebra (qflash_amd/csrc/qflash_fwd.hip, fwd_fast) -----------

def _mul24(a, b):
    """v_mul_i32_i24: low 32 bits of sext24(a) * sext24(b)."""
    def sext24(v):
        v = np.asarray(v, dtype=np.int64) & 0xFFFFFF
        return np.where(v >= (1 << 23), v - (1 << 24), v)
    return O.wrap32(sext24(a) * sext24(b))


def _fast_p(s, mn, k):
    """The six-op sequence of fwd_fast for scores s and row max mn."""
    c1 = O.wrap32(O.wrap32(-mn * k.exp_M) + (1 << 16))
    c3 = O.wrap32(k.sm_rscale - mn)
    t = O.wrap32(_mul24(s, k.exp_M) + c1)
    q1 = t >> 16
    a = O.wrap32(s + _mul24(q1, k.sm_rscale) + c3)
    E = a >> np.minimum(q1 & 0xFFFFFFFF, 31)
    y = O.wrap32(_mul24(E, k.req_M) + (1 << 15))
    return O.i8(y >> 16)


def _fast_domain(k, D=64):
    """Largest |x| the kernel's guards admit for these constants (X*|eM| and |a| bounds)."""
    aem, rs = -k.exp_M, k.sm_rscale
    lim = (1 << 31) - (1 << 17)
    eps = abs(aem * rs - 65536)
    X = lim // aem if aem else 1 << 22
    X = min(X, 1 << 22, (((1 << 22) - 2 * rs - 2) * 65536) // max(eps, 1))
    return X


GUARDED = [k for k in CONSTS if -k.exp_M * k.sm_rscale < (1 << 17) and k.req_M < (1 << 23)
           and abs(-k.exp_M * k.sm_rscale - 65536) <= 2 * -k.exp_M][:8]


@pytest.mark.parametrize("k", GUARDED, ids=lambda k: f"rs{k.sm_rscale}_eM{k.exp_M}")
def test_fast_exp_sequence_equals_reference_on_its_domain(k):
    """For every x in [-X, 0] the 24-bit sequence gives the reference p(x); it is
    evaluated at several row maxima (the per-row constants c1, c3 fold m')."""
    X = _fast_domain(k)
    x = np.arange(-X, 1, dtype=np.int64)
    want = O.requantize(O.exp2_i32(x, k), k)
    for mn in (0, 1234, -70000, 1 << 21, O.NEG_INF):
        s = x + mn
        keep = np.abs(s) < (1 << 23)           # the guards keep s inside 24 bits
        got = _fast_p(s[keep], mn, k)
        np.testing.assert_array_equal(got, want[keep])


@pytest.mark.parametrize("k", GUARDED, ids=lambda k: f"rs{k.sm_rscale}_eM{k.exp_M}")
def test_alpha_stays_in_range_without_overflow(k):
    """E(x) in [-1, rs] for every x <= 0 with x*eM inside int32 (|rs - 2^16/|eM|| <= 2):
    the fast kernel's multipliers alpha*acc_M then fit int32."""
    xmax = ((1 << 31) - 1) // -k.exp_M
    x = np.arange(-xmax, 1, dtype=np.int64)
    e = O.exp2_i32(x, k)
    assert e.min() >= -1 and e.max() == k.sm_rscale


def test_sad_u8_l1_norm_identity():
    """sum |b| over signed bytes = sum | (b xor 0x80) - 0x80 | over unsigned bytes."""
    b = np.arange(-128, 128, dtype=np.int64)
    assert np.array_equal(np.abs(b), np.abs(((b & 0xFF) ^ 0x80) - 0x80))


def test_unsigned_dot_bounds_abs_sum():
    """sum of bytes read as unsigned >= sum |p| for int8 p (the dynamic acc bound)."""
    p = np.arange(-128, 128, dtype=np.int64)
    assert np.all((p & 0xFF) >= np.abs(p))


def test_identity_bound_holds_on_real_accumulators():
    """The static bound |acc| <= T*(2^19+1)*2 used to skip rescales holds along the
    oracle's own trajectory (acc tracked step by step on a golden case)."""
    c = CASES["outlier_N197_D64"]
    k, f = c.consts, c.flags
    q, kk, v = (c[n].astype(np.float64) for n in ("q_i8", "k_i8", "v_i8"))
    N = q.shape[2]
    T = math.ceil(N / 32)
    m = np.full(q.shape[:3], O.NEG_INF, dtype=np.int64)
    acc = np.zeros(q.shape, dtype=np.int64)
    worst = 0
    for st in range(0, N, 32):
        nv = min(32, N - st)
        kt = np.zeros(q.shape[:2] + (32, q.shape[3]))
        vt = np.zeros_like(kt)
        kt[:, :, :nv] = kk[:, :, st:st + nv]
        vt[:, :, :nv] = v[:, :, st:st + nv]
        s = np.rint(q @ kt.transpose(0, 1, 3, 2)).astype(np.int64)
        if nv < 32:
            s[..., nv:] = O.NEG_INF
        mn = np.maximum(m, s.max(-1))
        p = O.requantize(O.exp2_i32(O.wrap32(s - mn[..., None]), k, f), k)
        alpha = O.exp2_i32(O.wrap32(m - mn), k, f)
        acc = O.scale_release(acc, alpha[..., None], k.acc_M, 30, True, k.sm_rscale)
        acc = O.wrap32(acc + np.rint(p.astype(np.float64) @ vt).astype(np.int64))
        m = mn
        worst = max(worst, int(np.abs(acc).max()))
    assert worst <= T * ((1 << 19) + 1) * 2


def test_division_through_double_reciprocal_is_ieee_single():
    """fwd_fast's epilogue: RN_f32(fp64(a) * RN_f64(1/fp64(b))) == RN_f32(a / b) for
    float a = fp32(acc), |b| = |fp32(l)| >= 2 (random int32 pairs, dense small
    ranges and near-midpoint families)."""
    rng = np.random.default_rng(11)

    def check(acc, l):
        a = acc.astype(np.float32)
        b = l.astype(np.float32)
        keep = np.abs(b) >= 2
        a, b = a[keep], b[keep]
        want = a / b                                         # IEEE single division
        got = (a.astype(np.float64) * (1.0 / b.astype(np.float64))).astype(np.float32)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, f"{bad.size} mismatches, e.g. a={a[bad[0]]!r} b={b[bad[0]]!r}"
        # and truncation of the in-range quotient equals x86 cvt (|q| < 2^30)
        assert np.all(np.abs(want) < 2 ** 30)

    for _ in range(4):
        check(rng.integers(-(1 << 31), 1 << 31, 2_000_000), rng.integers(-(1 << 31), 1 << 31, 2_000_000))
        check(rng.integers(-(1 << 31), 1 << 31, 2_000_000), rng.integers(-4096, 4096, 2_000_000))
        check(rng.integers(-(1 << 20), 1 << 20, 2_000_000), rng.integers(2, 1 << 16, 2_000_000))
    a, b = np.meshgrid(np.arange(-3000, 3000), np.arange(2, 700))
    check(a.ravel(), b.ravel())
    # quotients close to midpoints: a = b*(2m+1)/2 +- small, large b
    b = rng.integers(1 << 20, 1 << 24, 1_000_000)
    m = rng.integers(1, 1 << 7, 1_000_000)
    check(b * m + b // 2 + rng.integers(-2, 3, 1_000_000), b)
