"""Pins of the oracle's host-side and SQNR functions (CPU only).

``oracle/qflash_oracle.py`` restates, beside the kernel loop, the host steps of
``qflash_forward`` (qflash/kernel.py:287-311, :327-336) and the benchmark's
SQNR (benchmark.py:27-28).  Each is checked here against what fixes it
independently of this repository:

* host_constants, quantize_ref_torch, mask_to_bias_torch: the values the
  reference's own ``qflash_forward`` handed to its kernel in the golden
  launch records, plus hand-derived half-to-even ties;
* sqnr_db: hand-computed norms;
* softmax_attention_fp32: closed forms (equal logits give the mean of V, a
  dominant logit gives its V row, a -inf bias removes columns);
* bench.sqnr_db (the figure bench.py reports): equal to the oracle's
  definition on cfg1 codes from the C oracle.

``test_planted_mistakes_fail`` plants a plausible mistake in each function
and checks that the corresponding pin rejects it.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle.qflash_oracle as O
from golden_io import load_cases

CASES = load_cases()
FP = sorted(n for n, c in CASES.items() if c.has_fp)
MASKED = sorted(n for n in FP if CASES[n].masked)
INT8_MAX = 127


def _fp(c):
    return tuple(torch.from_numpy(np.ascontiguousarray(c[n])) for n in ("q_fp", "k_fp", "v_fp"))


def _scales(q, k, v):
    # kernel.py:294-296: per-tensor absmax / 127 in the input dtype
    return tuple(x.abs().amax() / INT8_MAX for x in (q, k, v))


def _scale_arg(c):
    s = float(c["scale_arg"])
    return None if math.isnan(s) else s


def _tuple(cs):
    return (cs.sm_rscale, cs.exp_M, cs.req_M, cs.l_M, cs.acc_M)


def _constants_of(c, fn=O.host_constants):
    q, k, v = _fp(c)
    qs, ks, _ = _scales(q, k, v)
    return _tuple(fn(float(qs * ks), q.shape[-1], _scale_arg(c), c.flags))


def _sm_scale(c):
    q, k, v = _fp(c)
    qs, ks, _ = _scales(q, k, v)
    s = _scale_arg(c)
    s = 1.0 / math.sqrt(q.shape[-1]) if s is None else s
    return s * O.LOG2E * float(qs * ks)


# ------------------------------------------------------------ host_constants ---

@pytest.mark.parametrize("name", FP)
def test_host_constants_match_reference_launch(name):
    c = CASES[name]
    assert _constants_of(c) == tuple(int(x) for x in c["consts"])


# scale = 1/LOG2E makes sm_scale equal qk_scale exactly (1/LOG2E * LOG2E == 1.0 in double)
_UNIT = 1.0 / O.LOG2E
assert _UNIT * O.LOG2E == 1.0


def test_host_constants_round_half_to_even():
    """Python's round on exact ties (kernel.py:302-305): -2.5 -> -2, -3.5 -> -4,
    317.5 -> 318, 444.5 -> 444, 1/0.4 = 2.5 -> 2."""
    c = O.host_constants(2.5 / 65536, 64, _UNIT)
    assert (c.exp_M, c.req_M) == (-2, 318)
    c = O.host_constants(3.5 / 65536, 64, _UNIT)
    assert (c.exp_M, c.req_M) == (-4, 444)
    c = O.host_constants(0.4, 64, _UNIT)
    assert c.sm_rscale == 2 and c.l_M == 1 << 29 and c.acc_M == 1 << 29


def test_host_constants_raise_where_the_reference_does():
    """sm_scale = 2 rounds 1/sm_scale = 0.5 to rs = 0, and l_M divides by it;
    a zero scale divides by zero; NaN cannot become an int."""
    with pytest.raises(ZeroDivisionError):
        O.host_constants(2.0, 64, _UNIT)
    with pytest.raises(ZeroDivisionError):
        O.host_constants(0.0, 64)
    with pytest.raises(ValueError):
        O.host_constants(float("nan"), 64)
    # just below 2: 1/s rounds to 1, no error
    assert O.host_constants(1.9, 64, _UNIT).sm_rscale == 1


def test_host_constants_default_scale_is_inverse_sqrt_head_dim():
    """scale=None is 1/sqrt(D) (kernel.py:289-290)."""
    for D in (32, 64, 128):
        assert O.host_constants(1e-4, D) == O.host_constants(1e-4, D, 1.0 / math.sqrt(D))


# ------------------------------------------------------- quantize_ref_torch ---

@pytest.mark.parametrize("name", FP)
def test_quantize_ref_torch_matches_reference_codes(name):
    c = CASES[name]
    q, k, v = _fp(c)
    for x, s, key in zip((q, k, v), _scales(q, k, v), ("q_i8", "k_i8", "v_i8")):
        np.testing.assert_array_equal(O.quantize_ref_torch(x, s).numpy(), c[key])


def test_quantize_ref_torch_rounds_half_to_even_and_clamps():
    s = torch.tensor(1.0)
    x = torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5, 126.5, 300.0, -300.0])
    assert O.quantize_ref_torch(x, s).tolist() == [0, 2, 2, 0, -2, 126, 127, -128]


# ------------------------------------------------------- mask_to_bias_torch ---

@pytest.mark.parametrize("name", MASKED)
def test_mask_to_bias_torch_matches_reference_bias(name):
    c = CASES[name]
    Z, H, N = c["q_i8"].shape[:3]
    mask = torch.from_numpy(np.ascontiguousarray(c["mask"]))
    got = O.mask_to_bias_torch(mask, _sm_scale(c), Z, H, N)
    assert got.shape == (Z, H, N, N) and got.dtype == torch.int32
    np.testing.assert_array_equal(got.numpy(), c["bias_i32"])


def test_mask_to_bias_torch_threshold_is_strict():
    """-100.0 itself is not masked (kernel.py:330: mask < -1e2)."""
    m = torch.tensor([-100.0, -100.001, 0.0]).view(1, 1, 1, 3).expand(1, 1, 3, 3)
    b = O.mask_to_bias_torch(m, 1.0, 1, 1, 3)[0, 0, 0].tolist()
    assert b == [round(-100.0 * O.LOG2E), O.NEG_INF, 0]


# ------------------------------------------------------------------ sqnr_db ---

def test_sqnr_db_hand_values():
    # ||ref|| = 5, ||err|| = 0.05 -> 20*log10(100) = 40 dB
    assert O.sqnr_db([3.0, 4.0], [3.0, 4.05]) == pytest.approx(40.0, abs=1e-9)
    # err = ref -> 0 dB; err = ref / 10 -> 20 dB (amplitude ratio, not power)
    assert O.sqnr_db([1.0, -2.0, 2.0], [0.0, 0.0, 0.0]) == pytest.approx(0.0, abs=1e-12)
    assert O.sqnr_db([1.0, -2.0, 2.0], [1.1, -2.2, 2.2]) == pytest.approx(20.0, abs=1e-9)
    # norms over all elements, whatever the shape
    r = np.arange(1, 25, dtype=np.float64).reshape(2, 3, 4)
    assert O.sqnr_db(r, r * 1.001) == pytest.approx(60.0, abs=1e-6)


# -------------------------------------------------- softmax_attention_fp32 ---

def test_softmax_attention_equal_logits_average_v():
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 2, 5, 8, generator=g)
    k = torch.randn(1, 2, 1, 8, generator=g).expand(1, 2, 7, 8)  # every key the same
    v = torch.randn(1, 2, 7, 8, generator=g)
    out = O.softmax_attention_fp32(q, k, v)
    want = v.mean(dim=2, keepdim=True).expand_as(out)
    torch.testing.assert_close(out, want, rtol=1e-5, atol=1e-6)


def test_softmax_attention_dominant_logit_selects_its_row():
    D = 16
    q = torch.zeros(1, 1, 3, D)
    q[..., 0] = 1.0
    k = torch.zeros(1, 1, 6, D)
    k[0, 0, 4, 0] = 400.0  # logit 400/sqrt(16) = 100 against 0 for the others
    v = torch.arange(6 * D, dtype=torch.float32).view(1, 1, 6, D)
    out = O.softmax_attention_fp32(q, k, v)
    torch.testing.assert_close(out, v[:, :, 4:5].expand(1, 1, 3, D), rtol=0, atol=1e-3)


def test_softmax_attention_scale_and_bias():
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 1, 4, 8, generator=g) for _ in range(3))
    # scale 0: equal logits whatever q, k
    torch.testing.assert_close(O.softmax_attention_fp32(q, k, v, scale=0.0),
                               v.mean(dim=2, keepdim=True).expand(1, 1, 4, 8), rtol=1e-5, atol=1e-6)
    # -inf bias on all columns but column 2 of every row: exactly V row 2
    b = torch.full((1, 1, 4, 4), -float("inf"))
    b[..., 2] = 0.0
    torch.testing.assert_close(O.softmax_attention_fp32(q, k, v, bias=b), v[:, :, 2:3].expand(1, 1, 4, 8),
                               rtol=0, atol=0)
    # the default scale is 1/sqrt(D): equal to an explicit 1/sqrt(8)
    torch.testing.assert_close(O.softmax_attention_fp32(q, k, v),
                               O.softmax_attention_fp32(q, k, v, scale=1.0 / math.sqrt(8)), rtol=0, atol=0)


# ------------------------------------------ SQNR of the benchmark (cfg1, CPU) ---

def _cfg1_codes(seed: int = 0):
    import bench
    from oracle import oracle_c

    w = bench.prepare("cfg1", seed, torch.device("cpu"))
    codes = oracle_c.attention_codes(w["q8"].numpy(), w["k8"].numpy(), w["v8"].numpy(), O.Consts(*w["consts"]),
                                     O.Flags(), threads=4)
    w["o"] = torch.from_numpy(np.ascontiguousarray(codes))
    return w


def test_bench_sqnr_equals_oracle_definition_on_cfg1():
    """bench.sqnr_db (per-chunk sums) equals sqnr_db(softmax_attention_fp32, codes * o_scale)."""
    import bench

    w = _cfg1_codes(0)
    got = bench.sqnr_db(w, torch.device("cpu"))
    ref = O.softmax_attention_fp32(w["q"], w["k"], w["v"])
    out = w["o"].float() * w["o_scale"].float()
    want = O.sqnr_db(ref.numpy(), out.numpy())
    assert got == pytest.approx(want, abs=1e-4)
    # the reference algorithm's own SQNR on this workload (outlier channels: low)
    assert 5.0 < got < 15.0


def test_oracle_sqnr_floor_on_uniform_inputs():
    """On U[-4, 4) inputs (the reference README's workload) the integer
    algorithm is within ~1 dB of its published 31-32.5 dB."""
    g = torch.Generator().manual_seed(199)
    q, k, v = ((torch.rand(2, 2, 197, 64, generator=g) * 8 - 4) for _ in range(3))
    qs, ks, vs = _scales(q, k, v)
    c = O.host_constants(float(qs * ks), 64)
    q8, k8, v8 = (O.quantize_ref_torch(x, s).numpy() for x, s in zip((q, k, v), (qs, ks, vs)))
    codes = O.attention_codes(q8, k8, v8, c)
    out = codes.astype(np.float32) * float(vs)
    sq = O.sqnr_db(O.softmax_attention_fp32(q, k, v).numpy(), out)
    assert 29.0 < sq < 35.0, sq


# ------------------------------------------------------------ planted mistakes ---

def _constants_pin(fn):
    try:
        if any(_constants_of(CASES[n], fn) != tuple(int(x) for x in CASES[n]["consts"]) for n in FP):
            return False
        c = fn(3.5 / 65536, 64, _UNIT, O.Flags())
        return (c.exp_M, c.req_M) == (-4, 444)
    except (ZeroDivisionError, ValueError, OverflowError):
        return False


def _floor_round_constants(qk_scale, head_dim, scale=None, flags=O.Flags()):
    scale = (1.0 / head_dim ** 0.5 if scale is None else scale) * O.LOG2E
    s = scale * qk_scale
    r = lambda x: int(math.floor(x + 0.5))  # noqa: E731  half up instead of half to even
    rs = r(1.0 / s)
    return O.Consts(rs, r(-s * 65536), r(s * 127 * 65536), r((1 << flags.l_shift) / rs),
                    r((1 << flags.acc_shift) / rs))


def _log_e_constants(qk_scale, head_dim, scale=None, flags=O.Flags()):
    scale = (1.0 / head_dim ** 0.5 if scale is None else scale) * math.log2(math.e)  # not the literal
    return O.host_constants(qk_scale, head_dim, scale / O.LOG2E, flags)


def _quant_pin(fn):
    for n in FP:
        q, k, v = _fp(CASES[n])
        for x, s, key in zip((q, k, v), _scales(q, k, v), ("q_i8", "k_i8", "v_i8")):
            if not np.array_equal(fn(x, s).numpy(), CASES[n][key]):
                return False
    return True


def _bias_pin(fn):
    for n in MASKED:
        c = CASES[n]
        Z, H, N = c["q_i8"].shape[:3]
        got = fn(torch.from_numpy(np.ascontiguousarray(c["mask"])), _sm_scale(c), Z, H, N)
        if not np.array_equal(got.numpy(), c["bias_i32"]):
            return False
    return True


def _bias_le(attn_mask, sm_scale, Z, H, N):
    if attn_mask.dtype == torch.bool:
        return O.mask_to_bias_torch(attn_mask, sm_scale, Z, H, N)
    is_masked = attn_mask <= -1e2  # not strict
    q = (attn_mask.masked_fill(is_masked, 0.0) * O.LOG2E / sm_scale).round().to(torch.int32)
    return q.masked_fill(is_masked, O.NEG_INF).expand(Z, H, N, N).contiguous()


def _bias_trunc(attn_mask, sm_scale, Z, H, N):
    if attn_mask.dtype == torch.bool:
        return O.mask_to_bias_torch(attn_mask, sm_scale, Z, H, N)
    is_masked = attn_mask < -1e2
    q = (attn_mask.masked_fill(is_masked, 0.0) * O.LOG2E / sm_scale).to(torch.int32)  # no round
    return q.masked_fill(is_masked, O.NEG_INF).expand(Z, H, N, N).contiguous()


def _softmax_pin(fn):
    g = torch.Generator().manual_seed(3)
    q = torch.randn(1, 2, 5, 8, generator=g)
    k = torch.randn(1, 2, 1, 8, generator=g).expand(1, 2, 7, 8).contiguous()
    v = torch.randn(1, 2, 7, 8, generator=g)
    ok = torch.allclose(fn(q, k, v), v.mean(dim=2, keepdim=True).expand(1, 2, 5, 8), rtol=1e-5, atol=1e-6)
    k2 = torch.zeros(1, 1, 6, 16)
    k2[0, 0, 4, 0] = 400.0
    q2 = torch.zeros(1, 1, 3, 16)
    q2[..., 0] = 1.0
    v2 = torch.arange(6 * 16, dtype=torch.float32).view(1, 1, 6, 16)
    ok = ok and torch.allclose(fn(q2, k2, v2), v2[:, :, 4:5].expand(1, 1, 3, 16), rtol=0, atol=1e-3)
    q3, k3, v3 = (torch.randn(1, 1, 4, 8, generator=g) for _ in range(3))
    ok = ok and torch.allclose(fn(q3, k3, v3), O.softmax_attention_fp32(q3, k3, v3, scale=1 / math.sqrt(8)),
                               rtol=0, atol=0)
    return bool(ok)


def _softmax_no_scale(q, k, v, bias=None, scale=None):
    return O.softmax_attention_fp32(q, k, v, bias, scale=1.0)


def _softmax_softmax_over_queries(q, k, v, bias=None, scale=None):
    q, k, v = (torch.as_tensor(x, dtype=torch.float32) for x in (q, k, v))
    s = torch.matmul(q, k.transpose(-1, -2)) / math.sqrt(q.shape[-1])
    return torch.matmul(torch.softmax(s, dim=-2), v)


def _sqnr_pin(fn):
    return (abs(fn([3.0, 4.0], [3.0, 4.05]) - 40.0) < 1e-9
            and abs(fn([1.0, -2.0, 2.0], [1.1, -2.2, 2.2]) - 20.0) < 1e-9)


def test_planted_mistakes_fail():
    # the oracle's functions pass their pins ...
    assert _constants_pin(O.host_constants)
    assert _quant_pin(O.quantize_ref_torch)
    assert _bias_pin(O.mask_to_bias_torch)
    assert _softmax_pin(O.softmax_attention_fp32)
    assert _sqnr_pin(O.sqnr_db)
    # ... and each planted mistake fails its pin
    assert not _constants_pin(_floor_round_constants)
    assert not _constants_pin(_log_e_constants)
    assert not _quant_pin(lambda x, s: torch.clamp(torch.trunc(x / s), -128, 127).to(torch.int8))
    assert not _quant_pin(lambda x, s: torch.clamp(torch.round(x.float() * (1.0 / s.float())), -128, 127)
                          .to(torch.int8))
    assert not _bias_pin(_bias_le)
    assert not _bias_pin(_bias_trunc)
    assert not _softmax_pin(_softmax_no_scale)
    assert not _softmax_pin(_softmax_softmax_over_queries)
    assert not _sqnr_pin(lambda r, o: 10.0 * math.log10(np.linalg.norm(r) / np.linalg.norm(np.subtract(o, r))))
    assert not _sqnr_pin(lambda r, o: 20.0 * math.log10(np.linalg.norm(o) / np.linalg.norm(np.subtract(o, r))))
