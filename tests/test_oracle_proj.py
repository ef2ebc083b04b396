"""CPU pins of oracle.qkv_int8_ref, the checker of the int8 QKV projection
(qflash_hip_qkv_int8), which has no counterpart in the reference.

* int32 products, fp32 values and codes against a pure-Python restatement
  (loops, one element at a time) on small shapes;
* codes against the reference's own quantiser formula (quantize_ref_torch,
  qflash/kernel.py:309-311) applied to the oracle's fp32 values;
* fp32 values against float64 within their two roundings, scales against
  amax / 127;
* planted mistakes (one rounding instead of two, the scale as a division,
  the weight not transposed, a dropped bias, the thirds swapped) each change
  the result.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle.qflash_oracle import qkv_int8_ref, quantize_ref_torch

F32 = np.float32


def _case(seed: int, M: int, K: int, C: int, bias: bool = True):
    g = np.random.default_rng(seed)
    x8 = g.integers(-128, 128, (M, K)).astype(np.int8)
    w8 = g.integers(-128, 128, (3 * C, K)).astype(np.int8)
    x_scale = F32(g.uniform(0.005, 0.05))
    w_scale = g.uniform(1e-4, 3e-3, 3 * C).astype(np.float32)
    b = g.normal(0, 2.0, 3 * C).astype(np.float32) if bias else None
    return x8, w8, x_scale, w_scale, b


def _scalar(x8, w8, x_scale, w_scale, b):
    """Element by element with Python ints and numpy fp32 scalars."""
    M, Nc = x8.shape[0], w8.shape[0]
    C = Nc // 3
    y = np.zeros((M, Nc), dtype=np.float32)
    for m in range(M):
        for c in range(Nc):
            acc = 0
            for k in range(x8.shape[1]):
                acc += int(x8[m, k]) * int(w8[c, k])
            v = F32(F32(acc) * F32(F32(x_scale) * F32(w_scale[c])))
            if b is not None:
                v = F32(v + F32(b[c]))
            y[m, c] = v
    scales = np.zeros(4, dtype=np.float32)
    codes = np.zeros((M, Nc), dtype=np.int8)
    for t in range(3):
        amax = F32(0)
        for m in range(M):
            for c in range(t * C, (t + 1) * C):
                amax = max(amax, F32(abs(y[m, c])))
        s = F32(amax * F32(1.0 / 127.0))
        scales[t] = s
        for m in range(M):
            for c in range(t * C, (t + 1) * C):
                q = float(F32(y[m, c] / s))
                r = round(q)  # Python round: half to even, as rint
                codes[m, c] = max(-128, min(127, r))
    scales[3] = F32(scales[0] * scales[1])
    return codes, scales, y


def test_against_scalar_restatement():
    for seed, (M, K, C) in enumerate([(3, 32, 32), (5, 64, 32), (2, 96, 64)]):
        for bias in (True, False):
            x8, w8, xs, ws, b = _case(seed, M, K, C, bias)
            codes, scales = qkv_int8_ref(x8, w8, xs, ws, b)
            want_codes, want_scales, _ = _scalar(x8, w8, xs, ws, b)
            np.testing.assert_array_equal(codes, want_codes)
            np.testing.assert_array_equal(scales, want_scales)


def test_codes_are_the_reference_quantiser_of_the_projection():
    x8, w8, xs, ws, b = _case(7, 40, 64, 96)
    codes, scales = qkv_int8_ref(x8, w8, xs, ws, b)
    _, _, y = _scalar(x8[:2], w8, xs, ws, b)  # the scalar fp32 values of two rows
    acc = x8.astype(np.int64) @ w8.astype(np.int64).T
    y_all = (acc.astype(np.float32) * (F32(xs) * ws)[None, :]) + b[None, :]
    np.testing.assert_array_equal(y_all[:2], y)
    for t in range(3):
        yt = torch.from_numpy(np.ascontiguousarray(y_all[:, t * 96:(t + 1) * 96]))
        ref = quantize_ref_torch(yt, torch.tensor(scales[t]))
        np.testing.assert_array_equal(codes[:, t * 96:(t + 1) * 96], ref.numpy())


def test_values_and_scales_against_float64():
    x8, w8, xs, ws, b = _case(3, 64, 128, 64)
    codes, scales = qkv_int8_ref(x8, w8, xs, ws, b)
    acc = x8.astype(np.int64) @ w8.astype(np.int64).T
    y64 = acc * (float(xs) * ws.astype(np.float64))[None, :] + b.astype(np.float64)[None, :]
    y = (acc.astype(np.float32) * (F32(xs) * ws)[None, :]) + b[None, :]
    # three fp32 roundings (x_scale * w_scale, the product, the sum), each within half an ulp
    assert np.all(np.abs(y - y64) <= 2.0 ** -22 * np.maximum(np.abs(y64), np.abs(acc * float(xs) * ws)) + 1e-30)
    for t in range(3):
        amax = np.abs(y[:, t * 64:(t + 1) * 64]).max()
        assert abs(float(scales[t]) - float(amax) / 127) <= 2.0 ** -23 * float(amax) / 127
    assert scales[3] == F32(scales[0] * scales[1])


def test_planted_mistakes_change_the_result():
    x8, w8, xs, ws, b = _case(5, 64, 64, 64)
    codes, scales = qkv_int8_ref(x8, w8, xs, ws, b)
    acc = x8.astype(np.int64) @ w8.astype(np.int64).T
    g = F32(xs) * ws

    def quant(y):
        out = np.zeros(y.shape, np.int8)
        sc = []
        for t in range(3):
            yt = y[:, t * 64:(t + 1) * 64]
            s = F32(np.abs(yt).max()) * F32(1.0 / 127.0)
            sc.append(s)
            out[:, t * 64:(t + 1) * 64] = np.clip(np.rint(yt / s), -128, 127).astype(np.int8)
        return out, np.array(sc, np.float32)

    one_rounding = (acc * g.astype(np.float64)[None, :] + b.astype(np.float64)[None, :]).astype(np.float32)
    assert (one_rounding != (acc.astype(np.float32) * g[None, :]) + b[None, :]).any()
    wrong = {
        "no bias": quant(acc.astype(np.float32) * g[None, :]),
        "thirds swapped": quant(np.concatenate([(acc.astype(np.float32) * g + b)[:, 64:128],
                                                (acc.astype(np.float32) * g + b)[:, :64],
                                                (acc.astype(np.float32) * g + b)[:, 128:]], axis=1)),
        "weight not transposed": quant((x8.astype(np.int64) @ w8.astype(np.int64)[:64].T)
                                       .repeat(3, axis=1).astype(np.float32) * g + b),
    }
    for name, (c2, s2) in wrong.items():
        assert (c2 != codes).any() or (s2 != scales[:3]).any(), name
    # the scale as a division instead of the product by RN(1/127): some amax tells them apart
    vals = np.random.default_rng(0).uniform(1, 100, 10000).astype(np.float32)
    assert (vals * F32(1.0 / 127.0) != vals / F32(127)).any()
