"""GPU parity: the gfx950 HIP kernels against the reference's own outputs and the oracle.

* golden vectors written by the reference (Triton interpreter) - every case,
  through the launcher with the reference's launch signature;
* the five benchmark configurations x seeds against the C oracle, bit-exact;
* the end-to-end host path (qflash.forward) against the reference's
  dequantised outputs;
* the MFMA register layouts the kernels rely on.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from golden_io import load_cases
from oracle import oracle_c
from oracle.qflash_oracle import Consts, Flags

pytestmark = pytest.mark.gpu

CASES = load_cases()
DEV = "cuda"


def _lib():
    from qflash_amd import _lib as L
    return L


def _launch(q8, k8, v8, o, consts: Consts, flags: Flags, bias=None):
    from qflash_amd.kernel import qflash_kernel, qflash_masked_kernel
    Z, H, N, D = q8.shape
    kw = dict(N_CTX=N, HEAD_DIM=D, EXP_USE_SHIFT=flags.exp_use_shift, L_USE_SHIFT=flags.l_use_shift,
              ACC_USE_SHIFT=flags.acc_use_shift, L_SHIFT=flags.l_shift, ACC_SHIFT=flags.acc_shift)
    c = (consts.sm_rscale, consts.exp_M, consts.req_M, consts.l_M, consts.acc_M)
    st = (*q8.stride(), *k8.stride(), *v8.stride(), *o.stride())
    if bias is None:
        qflash_kernel[None](q8, k8, v8, o, *c, *st, Z, H, **kw)
    else:
        qflash_masked_kernel[None](q8, k8, v8, o, bias, *c, *st, *bias.stride(), Z, H, **kw)


def test_library_loads_and_reports_version():
    L = _lib().load()
    assert b"gfx950" in L.qflash_hip_version()


def test_mfma_layout():
    rng = np.random.default_rng(7)
    A = rng.integers(-128, 128, (32, 32), dtype=np.int8)
    B = rng.integers(-128, 128, (32, 32), dtype=np.int8)
    a, b = torch.from_numpy(A).to(DEV), torch.from_numpy(B).to(DEV)
    c = torch.zeros(32, 32, dtype=torch.int32, device=DEV)
    L = _lib().load()
    import ctypes
    rc = L.qflash_hip_mfma_layout_check(ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()),
                                        ctypes.c_void_p(c.data_ptr()), None)
    assert rc == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(c.cpu().numpy(), A.astype(np.int32) @ B.astype(np.int32))


@pytest.mark.parametrize("name", sorted(CASES))
def test_golden_codes(name):
    c = CASES[name]
    q8 = torch.from_numpy(c["q_i8"]).to(DEV)
    k8 = torch.from_numpy(c["k_i8"]).to(DEV)
    v8 = torch.from_numpy(c["v_i8"]).to(DEV)
    bias = torch.from_numpy(c["bias_i32"]).to(DEV) if c.masked else None
    o = torch.empty_like(v8)
    _launch(q8, k8, v8, o, c.consts, c.flags, bias)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(o.cpu().numpy(), c["o_i8"])


HOOKS = ["FORCE_GENERAL", "FORCE_DYNAMIC_BOUND", "FORCE_ROBUST", "NO_LUT", "FORCE_LUT"]


@pytest.mark.parametrize("hook", HOOKS)
@pytest.mark.parametrize("name", sorted(CASES))
def test_golden_codes_forced_paths(name, hook, hip_hooks):
    """Every exact fallback on every case: the general kernel (used when the fast
    path's constant guards fail), the fast kernel's per-row dynamic bound for the
    identity rescale, its robust continuation (general arithmetic, used when a
    per-wave or per-step guard fails), and its arithmetic and table exp2 paths
    (the table off / on whatever the launch size)."""
    hip_hooks(hook)
    test_golden_codes(name)


@pytest.mark.parametrize("name", [n for n in sorted(CASES) if not CASES[n].masked][:12])
def test_golden_codes_token_major(name):
    """Same codes when Q/K/V/O are token-major (B, N, H, D) strided views."""
    c = CASES[name]

    def tm(a):
        return torch.from_numpy(a).to(DEV).permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)

    q8, k8, v8 = tm(c["q_i8"]), tm(c["k_i8"]), tm(c["v_i8"])
    o = torch.empty_like(v8)
    assert o.stride() == v8.stride()
    _launch(q8, k8, v8, o, c.consts, c.flags)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(o.cpu().numpy(), c["o_i8"])


@pytest.mark.parametrize("name", [n for n in sorted(CASES) if CASES[n].has_fp and not n.startswith("flags_")])
def test_golden_forward_end_to_end(name):
    """qflash.forward on the GPU reproduces the reference's dequantised output."""
    from qflash_amd import qflash
    c = CASES[name]
    dt = torch.float16 if "float16" in str(c["in_dtype"]) else torch.float32
    q = torch.from_numpy(c["q_fp"]).to(DEV, dt)
    k = torch.from_numpy(c["k_fp"]).to(DEV, dt)
    v = torch.from_numpy(c["v_fp"]).to(DEV, dt)
    mask = None
    if "mask" in c:
        mask = torch.from_numpy(c["mask"]).to(DEV)
    scale = None if np.isnan(c["scale_arg"]) else float(c["scale_arg"])
    out = qflash.forward(q, k, v, attn_mask=mask, scale=scale)
    torch.cuda.synchronize()
    ref = c["out_fp"]
    got = out.cpu().numpy()
    assert got.dtype == ref.dtype
    # bit-exact expected; the bar is 1 ulp of the output dtype
    ulp = np.spacing(np.abs(ref).astype(ref.dtype)).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - ref.astype(np.float64)) <= ulp), name


def _config_case(cfg_name: str, seed: int):
    from qflash_amd.kernel import LOG2E, fixed_point_constants, mask_to_bias, quantize
    from qflash_amd.workloads import CONFIGS, make_inputs
    cfg = CONFIGS[cfg_name]
    q, k, v, mask = make_inputs(cfg, seed)
    qs, ks, vs = (x.abs().amax() / 127 for x in (q, k, v))
    sm_scale = (1.0 / cfg.D ** 0.5) * LOG2E * (qs * ks).item()
    consts = Consts(*fixed_point_constants(sm_scale, 30, 30))
    q8, k8, v8 = quantize(q, qs), quantize(k, ks), quantize(v, vs)
    bias = None if mask is None else mask_to_bias(mask, sm_scale, cfg.Z, cfg.H, cfg.N)
    return cfg, consts, q8, k8, v8, bias


CONFIG_SEEDS = [(c, s) for c in ("cfg1", "cfg2", "cfg3", "cfg4") for s in (0, 1, 2)] + [("cfg5", 0)]


@pytest.mark.parametrize("hook", HOOKS[1:])
@pytest.mark.parametrize("cfg_name", ["cfg1", "cfg3", "cfg4"])
def test_config_codes_forced_paths(cfg_name, hook, hip_hooks):
    hip_hooks(hook)
    test_config_codes_vs_oracle(cfg_name, 1)


@pytest.mark.parametrize("cfg_name,seed", CONFIG_SEEDS)
def test_config_codes_vs_oracle(cfg_name, seed):
    cfg, consts, q8, k8, v8, bias = _config_case(cfg_name, seed)
    print(f"[case] {cfg_name} seed={seed} consts={consts}", flush=True)
    want = oracle_c.attention_codes(q8, k8, v8, consts, Flags(), bias=bias, threads=min(16, os.cpu_count() or 1))
    qd, kd, vd = q8.to(DEV), k8.to(DEV), v8.to(DEV)
    assert qd.stride() == q8.stride()
    o = torch.empty_like(vd)
    bd = None if bias is None else bias.to(DEV)
    _launch(qd, kd, vd, o, consts, Flags(), bd)
    torch.cuda.synchronize()
    got = o.cpu().numpy()
    n_bad = int((got != want).sum())
    assert n_bad == 0, f"{n_bad} of {got.size} codes differ"


def _adversarial(pattern: str, D: int, N: int, seed: int):
    g = np.random.default_rng(seed)
    if pattern == "uniform":
        q, k, v = (g.integers(-128, 128, (1, 2, N, D), dtype=np.int64) for _ in range(3))
    else:  # rows of constant +-128 / 127: the largest |q.k| the int8 range allows
        q = np.where(g.random((1, 2, N, 1)) < 0.5, -128, 127) * np.ones((1, 2, N, D), dtype=np.int64)
        k = np.where(g.random((1, 2, N, 1)) < 0.5, -128, 127) * np.ones((1, 2, N, D), dtype=np.int64)
        q[:, :, ::3] = g.integers(-128, 128, q[:, :, ::3].shape)
        v = g.integers(-128, 128, (1, 2, N, D), dtype=np.int64)
    return [torch.from_numpy(x.astype(np.int8)) for x in (q, k, v)]


@pytest.mark.parametrize("pattern", ["extreme", "uniform"])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("sm_scale", [600 / 65536, 0.0123, 0.09, 1.0 / 3000])
def test_adversarial_int8_inputs(pattern, D, sm_scale):
    """Full-range int8 operands (constant +-128 rows reach |s| = 128*128*D) under
    several scales: whichever path the guards pick must stay bit-exact."""
    from qflash_amd.kernel import fixed_point_constants
    consts = Consts(*fixed_point_constants(sm_scale, 30, 30))
    N = 97 if D != 64 else 160
    q8, k8, v8 = _adversarial(pattern, D, N, seed=D + int(sm_scale * 1e6))
    print(f"[case] {pattern} D={D} sm_scale={sm_scale} consts={consts}", flush=True)
    want = oracle_c.attention_codes(q8, k8, v8, consts, Flags(), threads=8)
    qd, kd, vd = q8.to(DEV), k8.to(DEV), v8.to(DEV)
    o = torch.empty_like(vd)
    _launch(qd, kd, vd, o, consts, Flags())
    torch.cuda.synchronize()
    got = o.cpu().numpy()
    assert int((got != want).sum()) == 0


@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("sm_scale", [1 / 3.4, 1 / 2.6, 1 / 57.3, 1 / 94.2, 0.0123])
def test_table_path_vs_oracle(sm_scale, D, masked, hip_hooks):
    """The exp2 table of the fast kernel under scales with both signs of
    kappa: with small zero ranges (1/3.4: lut_lim = 25) most steps fail the
    per-step check and mix with the arithmetic path; rows of growing spread
    reach every case."""
    import ctypes
    hip_hooks("FORCE_LUT")
    from qflash_amd.kernel import fixed_point_constants, mask_to_bias
    consts = Consts(*fixed_point_constants(sm_scale, 30, 30))
    n, lim = ctypes.c_int32(), ctypes.c_int32()
    _lib().load().qflash_hip_lut_bounds(consts.sm_rscale, consts.exp_M, consts.req_M, ctypes.byref(n),
                                        ctypes.byref(lim))
    print(f"[case] sm_scale={sm_scale} D={D} masked={masked} consts={consts} lut=({n.value}, {lim.value})",
          flush=True)
    assert n.value > 0
    g = np.random.default_rng(D + int(1e4 * sm_scale) + masked)
    N = 200
    spread = np.linspace(1, 40, N)[None, None, :, None]
    q8, k8, v8 = (torch.from_numpy(np.clip(np.rint(g.standard_normal((2, 2, N, D)) * s), -128, 127).astype(np.int8))
                  for s in (spread, np.full_like(spread, 6.0), np.full_like(spread, 50.0)))
    bias = None
    if masked:
        bias = mask_to_bias(torch.from_numpy(g.random((N, N)) > 0.1), sm_scale, 2, 2, N)
    want = oracle_c.attention_codes(q8, k8, v8, consts, Flags(), bias=bias, threads=8)
    qd, kd, vd = q8.to(DEV), k8.to(DEV), v8.to(DEV)
    o = torch.empty_like(vd)
    _launch(qd, kd, vd, o, consts, Flags(), None if bias is None else bias.to(DEV))
    torch.cuda.synchronize()
    assert int((o.cpu().numpy() != want).sum()) == 0


@pytest.mark.parametrize("sm_scale", [0.05, 1 / 57.3])
def test_table_path_at_score_bias_edge(sm_scale, hip_hooks):
    """The unmasked table path takes one saturating subtraction per score,
    which needs every biased score positive: a wave may use it only while
    128 * ||q_row||_1 + 4096 <= 2^19 (||q||_1 <= 4064).  Rows of wave 0 sit on
    that edge (||q||_1 = 4064, keys near -128, so the biased scores come down
    to 4096), rows of wave 1 one past it (4065: arithmetic path); the spread
    of the scores in a step stays small, so the steps do take the table."""
    import ctypes
    hip_hooks("FORCE_LUT")
    from qflash_amd.kernel import fixed_point_constants
    consts = Consts(*fixed_point_constants(sm_scale, 30, 30))
    n, lim = ctypes.c_int32(), ctypes.c_int32()
    _lib().load().qflash_hip_lut_bounds(consts.sm_rscale, consts.exp_M, consts.req_M, ctypes.byref(n),
                                        ctypes.byref(lim))
    print(f"[case] sm_scale={sm_scale} consts={consts} lut=({n.value}, {lim.value})", flush=True)
    assert n.value > 0
    g = np.random.default_rng(7)
    Z, H, N, D = 1, 2, 96, 64
    q = np.tile(np.array([64, 63] * (D // 2), dtype=np.int64), (Z, H, N, 1))  # ||q||_1 = 4064
    q[:, :, 32:64, 0] += 1                                                       # 4065
    assert q.sum(-1).max() == 4065 and 128 * 4064 + 4096 == 1 << 19
    k = -128 + g.integers(0, 3, (Z, H, N, D))
    v = g.integers(-128, 128, (Z, H, N, D))
    q8, k8, v8 = (torch.from_numpy(x.astype(np.int8)) for x in (q, k, v))
    want = oracle_c.attention_codes(q8, k8, v8, consts, Flags(), threads=8)
    qd, kd, vd = q8.to(DEV), k8.to(DEV), v8.to(DEV)
    o = torch.empty_like(vd)
    _launch(qd, kd, vd, o, consts, Flags())
    torch.cuda.synchronize()
    assert int((o.cpu().numpy() != want).sum()) == 0


@pytest.mark.parametrize("seed", [0, 1])
def test_speculative_table_check_fails_mid_row(seed):
    """cfg3's constants (kappa < 0: the table's zero range ends at u = 17455)
    on rows whose host bound (2 * 128 * ||q||_1 ~ 74k) does not cover it, so
    every wave runs the loop that issues each step's table loads before the
    range check.  One key far below the scores (step 3) and one far above
    them (step 12) put columns beyond the range: the check fails in those
    steps and every later one, and the step falls back to the arithmetic;
    the steps in between pass.  Codes equal the oracle's."""
    import ctypes
    from qflash_amd.kernel import fixed_point_constants
    consts = Consts(*fixed_point_constants(0.017487, 30, 30))
    assert (consts.sm_rscale, consts.exp_M) == (57, -1146)
    n, lim = ctypes.c_int32(), ctypes.c_int32()
    _lib().load().qflash_hip_lut_bounds(consts.sm_rscale, consts.exp_M, consts.req_M, ctypes.byref(n),
                                        ctypes.byref(lim))
    g = np.random.default_rng(seed)
    Z, H, N, D = 1, 4, 577, 64
    q = g.integers(-8, 9, (Z, H, N, D))
    k = g.integers(-8, 9, (Z, H, N, D))
    v = g.integers(-128, 128, (Z, H, N, D))
    # the key at 100 opposes every query (its scores ~ -128 ||q||_1), the one at
    # 400 follows it (+127 ||q||_1); both lie far outside lut_lim of the others
    sgn = np.sign(q.sum(axis=2, keepdims=True))
    sgn[sgn == 0] = 1
    k[:, :, 100, :] = np.where(sgn[:, :, 0, :] > 0, -128, 127)
    k[:, :, 400, :] = np.where(sgn[:, :, 0, :] > 0, 127, -128)
    X = 2 * 128 * np.abs(q).sum(-1)
    print(f"[case] seed={seed} consts={consts} lut=({n.value}, {lim.value}) X in [{X.min()}, {X.max()}]", flush=True)
    assert X.min() > lim.value and X.max() // 2 + 4096 <= 1 << 19  # lut_mode 2 for every wave
    q8, k8, v8 = (torch.from_numpy(x.astype(np.int8)) for x in (q, k, v))
    want = oracle_c.attention_codes(q8, k8, v8, consts, Flags(), threads=8)
    qd, kd, vd = q8.to(DEV), k8.to(DEV), v8.to(DEV)
    o = torch.empty_like(vd)
    _launch(qd, kd, vd, o, consts, Flags())
    torch.cuda.synchronize()
    assert int((o.cpu().numpy() != want).sum()) == 0


TAIL_MODES = {  # hooks, score spread
    "table": (("FORCE_LUT",), 4.0),     # every step on the table
    "mixed": (("FORCE_LUT",), 40.0),    # wide spreads: some steps fail the per-step table check
    "arith": (("NO_LUT",), 4.0),        # the 24-bit arithmetic exp2
    "robust": (("FORCE_ROBUST",), 4.0),  # general arithmetic inside the fast kernel
}


@pytest.mark.parametrize("mode", sorted(TAIL_MODES))
@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("N", [33, 36, 37, 40, 41, 48, 49, 56, 57, 60, 63, 68, 95])
def test_table_path_short_tails(N, D, masked, mode, hip_hooks):
    """Partial last steps of 1-5 keys (the upper lane half of the step has no
    real column up to 4), 8/9, 16/17, 24/25 and 28-31 keys (the edges of the
    kernel's 4-, 8-, 12- and 16-register last steps), masked or not, for
    every head dim of the fast kernel, on the table path (padded columns read
    entry 0 and l gets their exact p), with spreads wide enough that some
    steps leave the table, on the arithmetic path and on the robust path."""
    hooks, spread = TAIL_MODES[mode]
    hip_hooks(*hooks)
    from qflash_amd.kernel import fixed_point_constants
    consts = Consts(*fixed_point_constants(1 / 57.3, 30, 30))
    print(f"[case] N={N} D={D} masked={masked} mode={mode}", flush=True)
    g = np.random.default_rng(N * 7 + D + masked)
    Z, H = 2, 3
    q = np.clip(np.rint(g.standard_normal((Z, H, N, D)) * spread), -128, 127)
    k = np.clip(np.rint(g.standard_normal((Z, H, N, D)) * spread), -128, 127)
    v = g.integers(-128, 128, (Z, H, N, D))
    q8, k8, v8 = (torch.from_numpy(x.astype(np.int8)) for x in (q, k, v))
    bias = None
    if masked:
        bias = torch.from_numpy(g.integers(-40, 41, (Z, H, N, N)).astype(np.int32))
    want = oracle_c.attention_codes(q8, k8, v8, consts, Flags(), bias=bias, threads=8)
    qd, kd, vd = q8.to(DEV), k8.to(DEV), v8.to(DEV)
    o = torch.empty_like(vd)
    _launch(qd, kd, vd, o, consts, Flags(), None if bias is None else bias.to(DEV))
    torch.cuda.synchronize()
    assert int((o.cpu().numpy() != want).sum()) == 0


@pytest.mark.parametrize("case", range(24))
def test_random_shapes_vs_oracle(case, hip_hooks):
    """Seeded random shapes, scales, code spreads and biases through every
    fast-kernel path (table or not, masked or not, partial steps), bit-exact
    against the C oracle."""
    from qflash_amd.kernel import fixed_point_constants
    g = np.random.default_rng(1000 + case)
    N = int(g.integers(1, 300))
    D = int(g.choice([32, 64, 128]))
    Z, H = int(g.integers(1, 3)), int(g.integers(1, 4))
    sm = float(g.choice([1 / 3.4, 1 / 8, 0.05, 1 / 57.3, 0.0123, 1 / 94.2]))
    spread = float(g.choice([2.0, 8.0, 30.0, 90.0]))
    masked = bool(case % 3 == 0)
    if case % 2:
        hip_hooks("FORCE_LUT")
    consts = Consts(*fixed_point_constants(sm, 30, 30))
    print(f"[case] {case}: Z={Z} H={H} N={N} D={D} sm={sm:.4f} spread={spread} masked={masked} "
          f"force_lut={case % 2}", flush=True)
    q = np.clip(np.rint(g.standard_normal((Z, H, N, D)) * spread), -128, 127)
    k = np.clip(np.rint(g.standard_normal((Z, H, N, D)) * spread), -128, 127)
    v = g.integers(-128, 128, (Z, H, N, D))
    q8, k8, v8 = (torch.from_numpy(x.astype(np.int8)) for x in (q, k, v))
    bias = None
    if masked:
        lim = int(g.choice([4, 300, 1 << 20]))
        b = g.integers(-lim, lim + 1, (Z, H, N, N))
        b[g.random((Z, H, N, N)) < 0.2] = -(1 << 20)
        bias = torch.from_numpy(b.astype(np.int32))
    want = oracle_c.attention_codes(q8, k8, v8, consts, Flags(), bias=bias, threads=8)
    qd, kd, vd = q8.to(DEV), k8.to(DEV), v8.to(DEV)
    o = torch.empty_like(vd)
    _launch(qd, kd, vd, o, consts, Flags(), None if bias is None else bias.to(DEV))
    torch.cuda.synchronize()
    assert int((o.cpu().numpy() != want).sum()) == 0


@pytest.mark.parametrize("masked", [False, True])
@pytest.mark.parametrize("scale", [-0.125, -1.0 / 57.3, -0.9])
def test_negative_scale_vs_oracle(scale, masked):
    """A negative `scale` argument (accepted by the reference: its constants come
    out negative, kernel.py:300-307, and its kernels run on them) goes through
    the general kernel, exact for any constants: codes equal the oracle's, and
    qflash.forward returns them times o_scale."""
    from qflash_amd import qflash
    from qflash_amd.kernel import LOG2E, fixed_point_constants, mask_to_bias, quantize
    g = torch.Generator().manual_seed(int(-scale * 1000) + masked)
    Z, H, N, D = 2, 2, 77, 64
    q, k, v = (torch.randn(Z, H, N, D, generator=g) for _ in range(3))
    mask = None
    if masked:
        mask = torch.where(torch.rand(N, N, generator=g) < 0.2, -200.0, torch.randn(N, N, generator=g))
    qs, ks, vs = (x.abs().amax() / 127 for x in (q, k, v))
    sm = scale * LOG2E * (qs * ks).item()
    consts = Consts(*fixed_point_constants(sm, 30, 30))
    assert consts.sm_rscale < 0
    q8, k8, v8 = quantize(q, qs), quantize(k, ks), quantize(v, vs)
    bias = None if mask is None else mask_to_bias(mask, sm, Z, H, N, materialize=True)
    print(f"[case] scale={scale} masked={masked} consts={consts}", flush=True)
    want = oracle_c.attention_codes(q8, k8, v8, consts, Flags(), bias=bias, threads=8)
    qd, kd, vd = q8.to(DEV), k8.to(DEV), v8.to(DEV)
    o = torch.empty_like(vd)
    _launch(qd, kd, vd, o, consts, Flags(), None if bias is None else bias.to(DEV))
    torch.cuda.synchronize()
    assert int((o.cpu().numpy() != want).sum()) == 0
    out = qflash.forward(q.to(DEV), k.to(DEV), v.to(DEV), attn_mask=None if mask is None else mask.to(DEV),
                         scale=scale)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), torch.from_numpy(want).float() * vs)
