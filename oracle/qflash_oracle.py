"""CPU oracle for the integer-only attention forward.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (``qflash_amd``) may
import this module: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker.

This is a restatement, in numpy, of the reference's integer algorithm
(EfficientCompLab/qflash, ``qflash/kernel.py``) as Triton evaluates it
(int32 wrap, clamping arithmetic shifts, truncating integer ``//``, int/int
true division in fp32, x86 float->int conversion).  Every function cites the
reference lines it follows.

Three independent restatements exist and are checked against each other and
against golden vectors produced by the reference itself (``tests/golden``):

* ``attention_codes``      - vectorised numpy (this file)
* ``attention_codes_scalar`` - pure-Python loops with Python ints (this file;
  tiny shapes only)
* ``oracle/qflash_oracle.c`` - plain C with OpenMP, used for full-size checks
  and as the CPU baseline (loaded through ``oracle/oracle_c.py``)

Pinning status per function (what fails if the restatement is wrong):

* exp2_i32 (shift/idiv), requantize, scale_release (shift/idiv): golden
  vectors from the reference kernel run under the Triton interpreter, plus
  closed-form properties (E(0)=rs, E(-rs*k) ~= rs>>k, monotone segments).
* the kernel loop (K0-K6): golden vectors (masked/unmasked, N%32 != 0,
  fp16/fp32 hosts), scalar/numpy/C agreement, planted mistakes, and an SQNR
  floor against fp32 softmax attention on uniform inputs
  (tests/test_oracle_golden.py, tests/test_oracle_host.py).
* host_constants, quantize_ref_torch, mask_to_bias_torch: the constants,
  int8 codes and int32 biases of the reference host path's launch records
  for fp32 and fp16 inputs, half-to-even ties, the raising cases, planted
  mistakes (tests/test_oracle_host.py).
* sqnr_db: hand-computed norms; softmax_attention_fp32: closed forms (equal
  logits -> mean of V, a dominant logit -> its V row, -inf bias); both with
  planted mistakes (tests/test_oracle_host.py).
* qkv_int8_ref (the int8 QKV projection, which has no counterpart in the
  reference): its int32 products against pure-Python loops, its fp32 values
  against float64 within their rounding, its codes against quantize_ref_torch
  and its scales against amax / 127, with planted mistakes
  (tests/test_oracle_proj.py).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

# kernel.py:137,288 - NEG_INF used for padded / bool-masked logits.
NEG_INF = -(1 << 20)
# kernel.py:26-27 (BLOCK_N=32 in every config, kernel.py:12-23 never picks
# BN=64 because BM<=BN is skipped): the rescale chain rounds every 32 columns.
BLOCK_N = 32
# kernel.py:287 - the literal, not math.log2(math.e).
LOG2E = 1.44269504
# kernel.py:301 - fixed-point bits of exp_M / req_M.
SHIFT = 16
INT_MIN = -(1 << 31)


@dataclass(frozen=True)
class Flags:
    """Arithmetic-variant switches, kernel.py:30-36 (QFLASH_* env vars)."""

    exp_use_shift: bool = True
    l_use_shift: bool = True
    acc_use_shift: bool = True
    l_shift: int = 30
    acc_shift: int = 30


@dataclass(frozen=True)
class Consts:
    """Per-call fixed-point constants, kernel.py:302-307."""

    sm_rscale: int
    exp_M: int
    req_M: int
    l_M: int
    acc_M: int


# ---------------------------------------------------------------- helpers ---

def wrap32(x):
    """Two's-complement truncation to int32 (Triton int32 tensors wrap)."""
    return np.asarray(x, dtype=np.int64).astype(np.int32).astype(np.int64)


def ashr32(a, b):
    """Arithmetic right shift of int32 ``a`` by ``b`` with clamping.

    numpy's right_shift (what the Triton interpreter runs, interpreter.py
    create_ashr) reads the shift as unsigned and returns the sign fill when
    it is >= 32 - including negative shift counts.
    """
    a = np.asarray(a, dtype=np.int64)
    bu = np.asarray(b, dtype=np.int64) & 0xFFFFFFFF
    fill = np.where(a < 0, -1, 0)
    return np.where(bu >= 32, fill, a >> np.minimum(bu, 31))


def trunc_div(a, b):
    """C-style truncating integer division (Triton ``//`` on ints)."""
    a = np.asarray(a, dtype=np.int64)
    b = np.asarray(b, dtype=np.int64)
    q = np.abs(a) // np.abs(b)
    return np.where((a < 0) != (b < 0), -q, q)


def i8(x):
    """Low byte, sign-extended (``.to(tl.int8)`` wraps)."""
    return np.asarray(x, dtype=np.int64).astype(np.int8).astype(np.int64)


# ------------------------------------------------------ integer primitives ---

def exp2_i32(x, c: Consts, flags: Flags = Flags()):
    """E(x) ~= rs * 2**(x*sm_scale) for x <= 0.

    kernel.py:40-44 (shift variant, SHIFT=16) and kernel.py:47-51 (idiv
    variant, QFLASH_EXP_USE_SHIFT=0), dispatched at kernel.py:54-59.
    """
    x = wrap32(x)
    rs = c.sm_rscale
    if flags.exp_use_shift:
        q = ashr32(wrap32(x * c.exp_M), SHIFT)
    else:
        q = wrap32(trunc_div(wrap32(-x), rs))
    r = wrap32(x + wrap32(q * rs))
    return wrap32(ashr32(wrap32(ashr32(r, 1) + rs), q))


def requantize(e, c: Consts):
    """p = int8((E*req_M + 2**15) >> 16), kernel.py:62-64 (wraps 128->-128)."""
    return i8(ashr32(wrap32(wrap32(np.asarray(e, dtype=np.int64) * c.req_M) + (1 << (SHIFT - 1))), SHIFT))


def scale_release(x, alpha, M: int, shift: int, use_shift: bool, rs: int):
    """Fixed-point rescale of l / acc by alpha/rs.

    kernel.py:67-69 (int64 multiply, round-half-up, >> shift) and
    kernel.py:72-74 (int32 wrap multiply, truncating // rs), dispatched at
    kernel.py:77-82.
    """
    x = np.asarray(x, dtype=np.int64)
    alpha = np.asarray(alpha, dtype=np.int64)
    if use_shift:
        with np.errstate(over="ignore"):
            prod = (x * alpha).astype(np.int64) * np.int64(M)  # wraps mod 2**64
            prod = prod + np.int64(1 << (shift - 1))
        return wrap32(prod >> shift)
    return wrap32(trunc_div(wrap32(x * alpha), rs))


def cvt_i32_x86(f):
    """fp32 -> int32 as numpy/x86 does it: truncate, INT_MIN when invalid."""
    f = np.asarray(f, dtype=np.float32)
    bad = ~np.isfinite(f) | (f >= np.float32(2.0 ** 31)) | (f < np.float32(-(2.0 ** 31)))
    safe = np.where(bad, np.float32(0), f)
    return np.where(bad, INT_MIN, np.trunc(safe).astype(np.int64))


# ------------------------------------------------------------ host side ---

def host_constants(qk_scale: float, head_dim: int, scale: float | None = None,
                   flags: Flags = Flags()) -> Consts:
    """Fixed-point constants from the per-tensor scales, kernel.py:287-307.

    ``qk_scale`` is the Python float of ``(q_scale*k_scale)`` evaluated in the
    input dtype (kernel.py:297).  Python ``round`` is half-to-even; the
    divisions are Python true division on doubles/ints.
    """
    if scale is None:
        scale = 1.0 / (head_dim ** 0.5)
    scale = scale * LOG2E
    sm_scale = scale * qk_scale
    rs = int(round(1.0 / sm_scale))
    exp_M = int(round(-sm_scale * (1 << SHIFT)))
    req_M = int(round(sm_scale * 127 * (1 << SHIFT)))
    l_M = int(round((1 << flags.l_shift) / rs))
    acc_M = int(round((1 << flags.acc_shift) / rs))
    return Consts(rs, exp_M, req_M, l_M, acc_M)


def quantize_ref_torch(x, xs):
    """clamp(round(x / xs), -128, 127).to(int8), kernel.py:309-311 (torch)."""
    import torch

    return torch.clamp(torch.round(x / xs), -128, 127).to(torch.int8)


def mask_to_bias_torch(attn_mask, sm_scale: float, Z: int, H: int, N: int):
    """Float/bool mask -> int32 additive bias, kernel.py:327-336 (torch)."""
    import torch

    if attn_mask.dtype == torch.bool:
        b = torch.zeros(Z, H, N, N, dtype=torch.int32, device=attn_mask.device)
        b.masked_fill_(attn_mask.logical_not(), NEG_INF)
        return b
    is_masked = attn_mask < -1e2
    clipped = attn_mask.masked_fill(is_masked, 0.0)
    quant = (clipped * LOG2E / sm_scale).round().to(torch.int32)
    return quant.masked_fill(is_masked, NEG_INF).expand(Z, H, N, N).contiguous()


def sqnr_db(ref, out) -> float:
    """20*log10(||ref|| / ||out - ref||), benchmark.py:27-28."""
    ref = np.asarray(ref, dtype=np.float64)
    out = np.asarray(out, dtype=np.float64)
    return float(20.0 * np.log10(np.linalg.norm(ref) / np.linalg.norm(out - ref)))


# ------------------------------------------------------------ the kernel ---

def _as_zhnd(a):
    a = np.asarray(a)
    assert a.ndim == 4, a.shape
    return a


def attention_codes(q, k, v, c: Consts, flags: Flags = Flags(), bias=None):
    """int8 output codes of the integer attention forward (numpy, vectorised).

    Follows qflash_kernel (kernel.py:85-180) and qflash_masked_kernel
    (kernel.py:183-272) row by row; rows are independent, so all rows of all
    (z, h) are processed together, 32 key columns per step, in order.

    q, k, v: int8 (Z, H, N, D).  bias: int32 broadcastable to (Z, H, N, N)
    or None.  Returns int8 (Z, H, N, D).
    """
    q = _as_zhnd(q).astype(np.float64)
    k = _as_zhnd(k).astype(np.float64)
    v = _as_zhnd(v).astype(np.float64)
    Z, H, N, D = q.shape
    masked = bias is not None
    if masked:
        bias = np.broadcast_to(np.asarray(bias, dtype=np.int64), (Z, H, N, N))
    # kernel.py:106 - EVEN_CTX skips padding only when nothing is padded.
    pad_cols = masked or (N % BLOCK_N != 0)

    m = np.full((Z, H, N), NEG_INF, dtype=np.int64)          # kernel.py:138
    l = np.ones((Z, H, N), dtype=np.int64)                   # kernel.py:139
    acc = np.zeros((Z, H, N, D), dtype=np.int64)             # kernel.py:140
    rs = c.sm_rscale
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        for start in range(0, N, BLOCK_N):                   # kernel.py:147
            stop = min(start + BLOCK_N, N)
            nv = stop - start
            kt = np.zeros((Z, H, BLOCK_N, D))
            vt = np.zeros((Z, H, BLOCK_N, D))
            kt[:, :, :nv] = k[:, :, start:stop]
            vt[:, :, :nv] = v[:, :, start:stop]
            # kernel.py:153 - exact int8 dot products (|s| < 2**23, fp64 exact)
            s = np.rint(q @ kt.transpose(0, 1, 3, 2)).astype(np.int64)
            if masked:                                       # kernel.py:250-253
                bt = np.zeros((Z, H, N, BLOCK_N), dtype=np.int64)
                bt[..., :nv] = bias[..., start:stop]
                s = wrap32(s + bt)
            if pad_cols and nv < BLOCK_N:                    # kernel.py:154-156
                s[..., nv:] = NEG_INF
            m_new = np.maximum(m, s.max(axis=-1))            # kernel.py:158
            x = wrap32(s - m_new[..., None])                 # kernel.py:159
            p = requantize(exp2_i32(x, c, flags), c)         # kernel.py:160-161
            l_ij = p.sum(axis=-1)                            # kernel.py:162
            alpha = exp2_i32(wrap32(m - m_new), c, flags)    # kernel.py:163
            l = wrap32(scale_release(l, alpha, c.l_M, flags.l_shift,
                                     flags.l_use_shift, rs) + l_ij)  # :164
            acc = scale_release(acc, alpha[..., None], c.acc_M, flags.acc_shift,
                                flags.acc_use_shift, rs)     # kernel.py:165
            pv = np.rint(p.astype(np.float64) @ vt).astype(np.int64)  # :171
            acc = wrap32(acc + pv)
            m = m_new                                        # kernel.py:172
        # kernel.py:176 - int/int true division in fp32, then fp32 -> int32.
        quot = acc.astype(np.float32) / l[..., None].astype(np.float32)
        out = cvt_i32_x86(quot)
    return i8(out).astype(np.int8)                           # kernel.py:178


def attention_codes_scalar(q, k, v, c: Consts, flags: Flags = Flags(), bias=None):
    """Same contract as ``attention_codes`` with Python-int loops (tiny only).

    Written against kernel.py:85-180/183-272 independently of the numpy
    version so the two pin each other.
    """
    q = np.asarray(q).astype(np.int64).tolist()
    k = np.asarray(k).astype(np.int64).tolist()
    v = np.asarray(v).astype(np.int64).tolist()
    Z, H, N, D = len(q), len(q[0]), len(q[0][0]), len(q[0][0][0])
    if bias is not None:
        bias = np.broadcast_to(np.asarray(bias, dtype=np.int64), (Z, H, N, N)).tolist()
    pad_cols = bias is not None or N % BLOCK_N != 0

    def w32(a):
        a &= 0xFFFFFFFF
        return a - (1 << 32) if a >= (1 << 31) else a

    def w64(a):
        a &= 0xFFFFFFFFFFFFFFFF
        return a - (1 << 64) if a >= (1 << 63) else a

    def sra(a, b):
        b &= 0xFFFFFFFF
        if b >= 32:
            return -1 if a < 0 else 0
        return a >> b

    def tdiv(a, b):
        qq = abs(a) // abs(b)
        return -qq if (a < 0) != (b < 0) else qq

    def E(x):
        rs = c.sm_rscale
        if flags.exp_use_shift:
            qq = sra(w32(x * c.exp_M), SHIFT)
        else:
            qq = w32(tdiv(w32(-x), rs))
        r = w32(x + w32(qq * rs))
        return w32(sra(w32(sra(r, 1) + rs), qq))

    def req(e):
        t = sra(w32(w32(e * c.req_M) + (1 << 15)), 16)
        t &= 0xFF
        return t - 256 if t >= 128 else t

    def rel(x, a, M, sh, use_shift):
        if use_shift:
            return w32((w64(w64(x * a) * M) + (1 << (sh - 1))) >> sh)
        return w32(tdiv(w32(x * a), c.sm_rscale))

    f32 = np.float32
    out = np.zeros((Z, H, N, D), dtype=np.int8)
    for z in range(Z):
        for h in range(H):
            for i in range(N):
                m, lsum, acc = NEG_INF, 1, [0] * D
                for start in range(0, N, BLOCK_N):
                    s = []
                    for jj in range(BLOCK_N):
                        j = start + jj
                        if j < N:
                            val = sum(q[z][h][i][d] * k[z][h][j][d] for d in range(D))
                            if bias is not None:
                                val = w32(val + bias[z][h][i][j])
                        else:
                            val = 0 if not pad_cols else NEG_INF
                        s.append(val)
                    mn = max(m, max(s))
                    p = [req(E(w32(sj - mn))) for sj in s]
                    alpha = E(w32(m - mn))
                    lsum = w32(rel(lsum, alpha, c.l_M, flags.l_shift, flags.l_use_shift) + sum(p))
                    acc = [rel(a, alpha, c.acc_M, flags.acc_shift, flags.acc_use_shift) for a in acc]
                    for d in range(D):
                        tot = 0
                        for jj in range(BLOCK_N):
                            j = start + jj
                            if j < N:
                                tot += p[jj] * v[z][h][j][d]
                        acc[d] = w32(acc[d] + tot)
                    m = mn
                for d in range(D):
                    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
                        fq = f32(acc[d]) / f32(lsum)
                    if not math.isfinite(float(fq)) or fq >= 2.0 ** 31 or fq < -(2.0 ** 31):
                        iv = INT_MIN
                    else:
                        iv = int(math.trunc(float(fq)))
                    iv &= 0xFF
                    out[z, h, i, d] = iv - 256 if iv >= 128 else iv
    return out


# ----------------------------------------------------- fp32 SQNR reference ---

def softmax_attention_fp32(q, k, v, bias=None, scale: float | None = None):
    """softmax(q k^T * scale + bias) v in float32 (SQNR reference, benchmark.py:27)."""
    import torch

    q = torch.as_tensor(q, dtype=torch.float32)
    k = torch.as_tensor(k, dtype=torch.float32)
    v = torch.as_tensor(v, dtype=torch.float32)
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    if bias is not None:
        s = s + torch.as_tensor(bias, dtype=torch.float32)
    return torch.matmul(torch.softmax(s, dim=-1), v)


def qkv_int8_ref(x8, w8, x_scale, w_scale, bias=None):
    """The int8 QKV projection fused with the quantiser (qflash_hip_qkv_int8;
    no counterpart in the reference, which projects in floating point,
    qflash/attention.py:23-24, and quantises the result, kernel.py:294-311).

    x8: (M, K) int8, w8: (Nc, K) int8, x_scale: fp32 scalar, w_scale and bias:
    (Nc,) fp32.  acc = x8 . w8^T exactly; y = RN(RN(fp32(acc) * RN(x_scale *
    w_scale)) + bias) in fp32; for the column thirds q, k, v (C = Nc / 3):
    scale_t = RN(amax|y_t| * RN(1/127)) and codes clamp(rint(RN(y_t /
    scale_t)), -128, 127) (0 where the quotient is NaN).  Returns the (M, Nc)
    int8 codes and the 4 fp32 scales (q, k, v, q * k)."""
    x8 = np.asarray(x8, dtype=np.int64)
    w8 = np.asarray(w8, dtype=np.int64)
    acc = x8 @ w8.T
    assert np.abs(acc).max(initial=0) < (1 << 24), "fp32(acc) must be exact"
    g = np.float32(x_scale) * np.asarray(w_scale, dtype=np.float32)
    y = acc.astype(np.float32) * g[None, :]
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32)[None, :]
    C = y.shape[1] // 3
    inv127 = np.float32(1.0 / 127.0)
    scales = np.zeros(4, dtype=np.float32)
    codes = np.zeros(y.shape, dtype=np.int8)
    with np.errstate(divide="ignore", invalid="ignore"):
        for t in range(3):
            yt = y[:, t * C:(t + 1) * C]
            st = np.float32(np.abs(yt).max()) * inv127
            scales[t] = st
            qt = np.rint(yt / st)
            qt = np.where(np.isnan(qt), 0, np.clip(qt, -128, 127))
            codes[:, t * C:(t + 1) * C] = qt.astype(np.int8)
    scales[3] = scales[0] * scales[1]
    return codes, scales
