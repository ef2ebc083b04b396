"""The CPU oracle against the reference's own outputs (CPU only).

The golden vectors were written by the reference kernel itself (qflash/kernel.py
run under the Triton interpreter, tests/golden/make_golden.py).  Three
independent restatements must reproduce every case bit for bit, and each
plausible mistake planted in the oracle must be caught by at least one case.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest

import oracle.qflash_oracle as O
from golden_io import load_cases
from oracle import oracle_c

CASES = load_cases()
NAMES = sorted(CASES)


def _bias(c):
    return c["bias_i32"] if c.masked else None


@pytest.mark.parametrize("name", NAMES)
def test_numpy_oracle_matches_reference(name):
    c = CASES[name]
    got = O.attention_codes(c["q_i8"], c["k_i8"], c["v_i8"], c.consts, c.flags, _bias(c))
    np.testing.assert_array_equal(got, c["o_i8"])


@pytest.mark.parametrize("name", NAMES)
def test_c_oracle_matches_reference(name):
    c = CASES[name]
    got = oracle_c.attention_codes(c["q_i8"], c["k_i8"], c["v_i8"], c.consts, c.flags, _bias(c), threads=2)
    np.testing.assert_array_equal(got, c["o_i8"])


SMALL = [n for n in NAMES if CASES[n]["q_i8"].shape[2] <= 70 and CASES[n]["q_i8"].size <= 2 * 3 * 70 * 64][:14]


@pytest.mark.parametrize("name", SMALL)
def test_scalar_oracle_matches_reference(name):
    c = CASES[name]
    got = O.attention_codes_scalar(c["q_i8"], c["k_i8"], c["v_i8"], c.consts, c.flags, _bias(c))
    np.testing.assert_array_equal(got, c["o_i8"])


def test_c_oracle_strided_and_head_range():
    """Token-major (strided) operands and a head sub-range give the same codes."""
    c = CASES["tokenmajor_N97_D64"]

    def tm(a):
        return np.ascontiguousarray(a.transpose(0, 2, 1, 3)).transpose(0, 2, 1, 3)

    q, k, v = tm(c["q_i8"]), tm(c["k_i8"]), tm(c["v_i8"])
    assert not q.flags["C_CONTIGUOUS"]
    got = oracle_c.attention_codes(q, k, v, c.consts, c.flags, threads=3)
    np.testing.assert_array_equal(got, c["o_i8"])
    Z, H = q.shape[:2]
    part = oracle_c.attention_codes(q, k, v, c.consts, c.flags, threads=1, zh_range=(1, Z * H - 1))
    flat = part.reshape(Z * H, *part.shape[2:])
    want = c["o_i8"].reshape(Z * H, *part.shape[2:])
    np.testing.assert_array_equal(flat[1:-1], want[1:-1])
    assert not flat[0].any() and not flat[-1].any()


def test_fixture_covers_hazard_regimes():
    """The fixtures exercise the reference's degenerate regimes (wrap, negative tails,
    clamped shifts, every flag variant, masks, padding, D in {32..256})."""
    p0, tails, flags, Ds, Ns = set(), set(), set(), set(), set()
    for c in CASES.values():
        k = c.consts
        p0.add(int(O.requantize(O.exp2_i32(np.array([0]), k, c.flags), k)[0]))
        tails.add(int(O.requantize(O.exp2_i32(np.array([O.NEG_INF - 5000]), k, c.flags), k)[0]))
        flags.add(tuple(int(x) for x in c["flags"]))
        Ds.add(c["q_i8"].shape[3])
        Ns.add(c["q_i8"].shape[2])
    assert any(p < 0 for p in p0), "no case wraps the row-max p to a negative int8"
    assert {0, -1} <= tails and min(tails) <= -3, "far-negative tails not covered"
    assert len(flags) >= 6
    assert {32, 64, 128, 256} <= Ds
    assert any(n % 32 for n in Ns) and any(n % 32 == 0 for n in Ns) and 1 in Ns
    assert sum(c.masked for c in CASES.values()) >= 10


# --- planted mistakes: each must change the codes of at least one golden case -------

def _mutant_numpy(monkeypatch, which):
    if which == "shift_mod32":  # AMD's 5-bit shift instead of the clamp
        monkeypatch.setattr(O, "ashr32", lambda a, b: np.asarray(a, dtype=np.int64).astype(np.int32).astype(
            np.int64) >> (np.asarray(b, dtype=np.int64) & 31))
    elif which == "requant_saturate":
        monkeypatch.setattr(O, "i8", lambda x: np.clip(np.asarray(x, dtype=np.int64), -128, 127))
    elif which == "cvt_saturate":
        def cvt(f):
            f = np.asarray(f, dtype=np.float32).astype(np.float64)
            f = np.where(np.isnan(f), 0, f)  # GPU-style: NaN -> 0, +-inf -> INT_MAX / INT_MIN
            return np.clip(np.trunc(f), -2 ** 31, 2 ** 31 - 1).astype(np.int64)
        monkeypatch.setattr(O, "cvt_i32_x86", cvt)
    elif which == "block_64":
        monkeypatch.setattr(O, "BLOCK_N", 64)
    elif which == "floor_div":
        monkeypatch.setattr(O, "trunc_div", lambda a, b: np.asarray(a, dtype=np.int64) // np.asarray(b, np.int64))
    elif which == "exp_no_half":  # drop the (r >> 1): E = (r + rs) >> q
        def e(x, c, flags=O.Flags()):
            x = O.wrap32(x)
            q = O.ashr32(O.wrap32(x * c.exp_M), O.SHIFT) if flags.exp_use_shift else O.wrap32(
                O.trunc_div(O.wrap32(-x), c.sm_rscale))
            r = O.wrap32(x + O.wrap32(q * c.sm_rscale))
            return O.wrap32(O.ashr32(O.wrap32(r + c.sm_rscale), q))
        monkeypatch.setattr(O, "exp2_i32", e)
    elif which == "release_no_round":
        orig = O.scale_release

        def rel(x, alpha, M, shift, use_shift, rs):
            if use_shift:
                return O.wrap32((np.asarray(x, np.int64) * np.asarray(alpha, np.int64) * np.int64(M)) >> shift)
            return orig(x, alpha, M, shift, use_shift, rs)
        monkeypatch.setattr(O, "scale_release", rel)


MUTANTS = ["shift_mod32", "requant_saturate", "cvt_saturate", "block_64", "floor_div", "exp_no_half",
           "release_no_round", "l_starts_at_0", "no_pad_columns"]


@pytest.mark.parametrize("which", MUTANTS)
def test_planted_mistake_is_detected(which, monkeypatch):
    if which in ("l_starts_at_0", "no_pad_columns"):
        # restated inline: the kernel loop with one step changed
        def run(c):
            return _loop_variant(c, which)
    else:
        _mutant_numpy(monkeypatch, which)

        def run(c):
            return O.attention_codes(c["q_i8"], c["k_i8"], c["v_i8"], c.consts, c.flags, _bias(c))
    differing = 0
    for name in NAMES:
        c = CASES[name]
        with np.errstate(all="ignore"):
            got = run(c)
        differing += int(not np.array_equal(got, c["o_i8"]))
    assert differing > 0, f"mutant {which} is not caught by any golden case"


def _loop_variant(c, which):
    """attention_codes with l initialised to 0 or with padded columns left at 0."""
    q = c["q_i8"].astype(np.float64)
    k = c["k_i8"].astype(np.float64)
    v = c["v_i8"].astype(np.float64)
    Z, H, N, D = q.shape
    bias = None if not c.masked else np.broadcast_to(c["bias_i32"].astype(np.int64), (Z, H, N, N))
    k_, f = c.consts, c.flags
    m = np.full((Z, H, N), O.NEG_INF, dtype=np.int64)
    l = np.zeros((Z, H, N), dtype=np.int64) if which == "l_starts_at_0" else np.ones((Z, H, N), dtype=np.int64)
    acc = np.zeros((Z, H, N, D), dtype=np.int64)
    for start in range(0, N, 32):
        nv = min(32, N - start)
        kt = np.zeros((Z, H, 32, D))
        vt = np.zeros((Z, H, 32, D))
        kt[:, :, :nv] = k[:, :, start:start + nv]
        vt[:, :, :nv] = v[:, :, start:start + nv]
        s = np.rint(q @ kt.transpose(0, 1, 3, 2)).astype(np.int64)
        if bias is not None:
            bt = np.zeros((Z, H, N, 32), dtype=np.int64)
            bt[..., :nv] = bias[..., start:start + nv]
            s = O.wrap32(s + bt)
        if nv < 32 and which != "no_pad_columns":
            s[..., nv:] = O.NEG_INF
        mn = np.maximum(m, s.max(-1))
        p = O.requantize(O.exp2_i32(O.wrap32(s - mn[..., None]), k_, f), k_)
        alpha = O.exp2_i32(O.wrap32(m - mn), k_, f)
        l = O.wrap32(O.scale_release(l, alpha, k_.l_M, f.l_shift, f.l_use_shift, k_.sm_rscale) + p.sum(-1))
        acc = O.scale_release(acc, alpha[..., None], k_.acc_M, f.acc_shift, f.acc_use_shift, k_.sm_rscale)
        acc = O.wrap32(acc + np.rint(p.astype(np.float64) @ vt).astype(np.int64))
        m = mn
    quot = acc.astype(np.float32) / l[..., None].astype(np.float32)
    return O.i8(O.cvt_i32_x86(quot)).astype(np.int8)


def test_unmutated_loop_variant_is_the_oracle():
    """_loop_variant with no change reproduces the golden codes (the mutants above
    differ from it in exactly one step)."""
    for name in ("outlier_N33_D64", "swin_N49_D32", "boolmask_N33_D64"):
        c = CASES[name]
        with np.errstate(all="ignore"):
            got = _loop_variant(c, "none")
        np.testing.assert_array_equal(got, c["o_i8"])


def test_flags_dataclass_is_frozen():
    with pytest.raises(dataclasses.FrozenInstanceError):
        O.Flags().l_shift = 3


@pytest.mark.parametrize("scale", [-0.125, -1.0 / 57.3, -0.9])
def test_negative_scale_numpy_and_c_oracles_agree(scale):
    """A negative `scale` gives negative constants (kernel.py:300-307), which the
    reference's kernels take as they come; the numpy and C restatements agree on
    them (masked and not), and the scalar loops agree on a small case."""
    from qflash_amd.kernel import LOG2E, fixed_point_constants
    g = np.random.default_rng(int(-scale * 1000))
    Z, H, N, D = 1, 2, 45, 32
    q, k, v = (g.integers(-128, 128, (Z, H, N, D)).astype(np.int8) for _ in range(3))
    c = O.Consts(*fixed_point_constants(scale * LOG2E * 1e-3, 30, 30))
    assert c.sm_rscale < 0
    bias = g.integers(-3000, 3000, (Z, H, N, N)).astype(np.int32)
    bias[g.random((Z, H, N, N)) < 0.2] = O.NEG_INF
    for b in (None, bias):
        want = O.attention_codes(q, k, v, c, O.Flags(), b)
        np.testing.assert_array_equal(oracle_c.attention_codes(q, k, v, c, O.Flags(), b, threads=2), want)
    small = O.attention_codes_scalar(q[:, :1, :12], k[:, :1, :12], v[:, :1, :12], c, O.Flags())
    np.testing.assert_array_equal(small, O.attention_codes(q[:, :1, :12], k[:, :1, :12], v[:, :1, :12], c))
