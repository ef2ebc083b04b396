"""Write golden vectors for the integer attention forward from the reference.

Runs ONLY in the build container, where the reference checkout exists at
/root/reference.  It loads ``qflash/kernel.py`` by file path (the package
``__init__`` needs timm, which is absent) under ``TRITON_INTERPRET=1`` so the
Triton kernels execute on the CPU with Triton's own typing rules, and records,
for each case:

* the fp inputs, mask and ``scale`` argument given to ``qflash_forward``;
* what ``qflash_forward`` handed to the kernel: int8 Q/K/V (in their strided
  layout, stored contiguous), the int32 bias, the five fixed-point constants
  and the arithmetic flags;
* the kernel's int8 output codes and ``qflash_forward``'s dequantised output.

The outputs are data (``golden_*.npz``); no reference source is copied.  The
GPU box never runs this script.  Usage:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import importlib.util
import os
import sys

import numpy as np

REF_KERNEL = "/root/reference/qflash/kernel.py"
HERE = os.path.dirname(os.path.abspath(__file__))


class _Recorder:
    """Stands in for a Triton kernel object: logs the launch, then runs it."""

    def __init__(self, kern, log, masked):
        self.kern, self.log, self.masked = kern, log, masked

    def __getitem__(self, grid):
        launcher = self.kern[grid]

        def run(*args, **kw):
            launcher(*args, **kw)
            n_t = 5 if self.masked else 4
            tensors = [a.clone() for a in args[:n_t]]
            consts = [int(a) for a in args[n_t:n_t + 5]]
            self.log.append(dict(tensors=tensors, consts=consts, kw=dict(kw)))

        return run


def load_reference(env: dict, tag: str):
    """Import kernel.py with the given QFLASH_* environment (read at import)."""
    saved = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        spec = importlib.util.spec_from_file_location(f"_qflash_ref_{tag}", REF_KERNEL)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
    finally:
        for k, old in saved.items():
            if old is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = old
    log = []
    mod.qflash_kernel = _Recorder(mod.qflash_kernel, log, masked=False)
    mod.qflash_masked_kernel = _Recorder(mod.qflash_masked_kernel, log, masked=True)
    return mod, log


def outlier_qkv(g, torch, Z, H, N, D, dtype, frac=0.02, factor=8.0, token_major=False):
    """BASELINE-style inputs: N(0,1) with round(frac*H*D) channels scaled x8."""
    out = []
    for _ in range(3):
        x = torch.randn(Z, N, H * D, generator=g)
        n_out = max(1, int(round(frac * H * D)))
        ch = torch.randperm(H * D, generator=g)[:n_out]
        x[:, :, ch] *= factor
        x = x.view(Z, N, H, D).permute(0, 2, 1, 3)
        if not token_major:
            x = x.contiguous()
        out.append(x.to(dtype))
    return out


def swin_mask(torch, g, nW, H, ws, shifted_windows, bias_std=0.02):
    """rel-pos bias (1,H,N,N) + 4-region shift mask (nW,N,N), like attention.py:58-72."""
    N = ws * ws
    table = torch.randn((2 * ws - 1) ** 2, H, generator=g) * bias_std
    coords = torch.stack(torch.meshgrid(torch.arange(ws), torch.arange(ws), indexing="ij")).flatten(1)
    rel = (coords[:, :, None] - coords[:, None, :]).permute(1, 2, 0)
    idx = (rel[:, :, 0] + ws - 1) * (2 * ws - 1) + (rel[:, :, 1] + ws - 1)
    bias = table[idx.view(-1)].view(N, N, H).permute(2, 0, 1).contiguous().unsqueeze(0)
    region = ((coords[0] >= ws // 2 + 1).long() * 2 + (coords[1] >= ws // 2 + 1).long())
    m = (region[:, None] != region[None, :]).float() * -100.0
    mask = torch.zeros(nW, N, N)
    for w in shifted_windows:
        mask[w] = m
    return bias, mask


def run_case(torch, mod, log, name, q, k, v, attn_mask=None, scale=None, keep_fp=True):
    log.clear()
    out = mod.qflash_forward(q, k, v, attn_mask=attn_mask, scale=scale)
    assert len(log) == 1, name
    rec = log[0]
    t = rec["tensors"]
    d = {
        "q_fp": q.float().numpy() if q.dtype != torch.float16 else q.numpy(),
        "k_fp": k.float().numpy() if k.dtype != torch.float16 else k.numpy(),
        "v_fp": v.float().numpy() if v.dtype != torch.float16 else v.numpy(),
        "in_dtype": np.array(str(q.dtype)),
        "scale_arg": np.array(np.nan if scale is None else scale, dtype=np.float64),
        "q_i8": t[0].contiguous().numpy(),
        "k_i8": t[1].contiguous().numpy(),
        "v_i8": t[2].contiguous().numpy(),
        "q_stride": np.array(t[0].stride(), dtype=np.int64),
        "o_i8": t[3].contiguous().numpy(),
        "o_stride": np.array(t[3].stride(), dtype=np.int64),
        "consts": np.array(rec["consts"], dtype=np.int64),
        "flags": np.array([int(rec["kw"]["EXP_USE_SHIFT"]), int(rec["kw"]["L_USE_SHIFT"]),
                           int(rec["kw"]["ACC_USE_SHIFT"]), rec["kw"]["L_SHIFT"],
                           rec["kw"]["ACC_SHIFT"]], dtype=np.int64),
        "out_fp": out.numpy(),
    }
    if not keep_fp:  # kernel-only case: int8 operands, constants and codes
        for key in ("q_fp", "k_fp", "v_fp", "out_fp"):
            del d[key]
    if attn_mask is not None:
        d["mask"] = attn_mask.numpy()
        d["bias_i32"] = t[4].contiguous().numpy()
    return name, d


def main():
    os.environ["TRITON_INTERPRET"] = "1"
    import torch

    torch.set_num_threads(8)
    ref, log = load_reference({}, "default")
    cases = []
    g = torch.Generator().manual_seed(1234)

    # 1. BASELINE-style outlier inputs across the N / D grid (fp32, contiguous).
    for N in (1, 31, 32, 33, 49, 63, 64, 65, 197):
        for D in (32, 64):
            q, k, v = outlier_qkv(g, torch, 1, 2, N, D, torch.float32)
            cases.append(run_case(torch, ref, log, f"outlier_N{N}_D{D}", q, k, v,
                                  keep_fp=N in (1, 33, 65)))
    for D in (128, 256):
        q, k, v = outlier_qkv(g, torch, 1, 1, 70, D, torch.float32)
        cases.append(run_case(torch, ref, log, f"outlier_N70_D{D}", q, k, v))
    # 2. token-major strided views (the QAttention layout) and fp16 inputs.
    q, k, v = outlier_qkv(g, torch, 2, 3, 97, 64, torch.float32, token_major=True)
    cases.append(run_case(torch, ref, log, "tokenmajor_N97_D64", q, k, v))
    q, k, v = outlier_qkv(g, torch, 1, 3, 197, 64, torch.float16)
    cases.append(run_case(torch, ref, log, "fp16_N197_D64", q, k, v))
    # 3. benchmark.py-style uniform inputs U[-4, 4) (benchmark.py:24).
    for (Z, H, N, D) in ((1, 2, 197, 64), (4, 2, 49, 32)):
        qkv = torch.rand(3, Z, H, N, D, generator=g) * 8 - 4
        cases.append(run_case(torch, ref, log, f"uniform_Z{Z}_N{N}_D{D}", qkv[0], qkv[1], qkv[2]))
    # 4. constants steered through `scale`: large/small sm_scale, the row-max
    #    int8 wrap (p(0) = 128 -> -128) and the far-negative -2/-3 tails.
    q, k, v = outlier_qkv(g, torch, 1, 2, 100, 64, torch.float32)
    for sc in (0.02, 0.05, 0.11, 0.3, 0.9, 2.5):
        cases.append(run_case(torch, ref, log, f"scale{sc}_N100_D64", q, k, v, scale=sc))
    # 5. masks: Swin rel-pos bias + shift mask (float), bool masks.
    bias, mask = swin_mask(torch, g, nW=2, H=3, ws=7, shifted_windows=(1,))
    swin_qkv = outlier_qkv(g, torch, 4, 3, 49, 32, torch.float32)
    amask = bias + mask.view(1, 2, 1, 49, 49).expand(2, -1, 3, -1, -1).reshape(-1, 3, 49, 49)
    cases.append(run_case(torch, ref, log, "swin_N49_D32", *swin_qkv, attn_mask=amask))
    # float mask with values exactly at and beyond the -1e2 boundary.
    q, k, v = outlier_qkv(g, torch, 1, 2, 40, 32, torch.float32)
    fm = torch.randn(1, 2, 40, 40, generator=g)
    sel = torch.rand(1, 2, 40, 40, generator=g)
    fm[sel < 0.15] = -100.0
    fm[(sel >= 0.15) & (sel < 0.3)] = -100.5
    fm[(sel >= 0.3) & (sel < 0.35)] = -1e4
    cases.append(run_case(torch, ref, log, "floatmask_boundary_N40_D32", q, k, v, attn_mask=fm))
    # broadcast float mask (1,1,N,N) and a bool mask.
    q, k, v = outlier_qkv(g, torch, 2, 2, 64, 64, torch.float32)
    fm = torch.randn(1, 1, 64, 64, generator=g) * 2
    cases.append(run_case(torch, ref, log, "floatmask_bcast_N64_D64", q, k, v, attn_mask=fm))
    bm = torch.rand(2, 2, 33, 33, generator=g) > 0.3
    bm[..., 0] = True
    q, k, v = outlier_qkv(g, torch, 2, 2, 33, 64, torch.float32)
    cases.append(run_case(torch, ref, log, "boolmask_N33_D64", q, k, v, attn_mask=bm))
    bm2 = torch.rand(1, 1, 70, 70, generator=g) > 0.9
    q, k, v = outlier_qkv(g, torch, 1, 2, 70, 32, torch.float32)
    cases.append(run_case(torch, ref, log, "boolmask_sparse_N70_D32", q, k, v, attn_mask=bm2))

    # 5b. l == 0 at the end of a row: equal logits (one-hot q = k) with the scale
    #     steered so that 4*p(0) + 28*p(pad) = 0; acc/l is then +-inf or NaN and the
    #     fp32 -> int32 conversion rule decides the codes.
    D = 32
    onehot = torch.zeros(1, 1, 4, D)
    onehot[..., 0] = 1.0
    qk32 = float((torch.tensor(1.0) / 127) * (torch.tensor(1.0) / 127))
    scale_l0 = 0.133345 / (1.44269504 * qk32)
    vz = torch.zeros(1, 1, 4, D)
    vz[..., 0, :] = torch.linspace(-1, 1, D)
    vz[..., 1, :] = torch.linspace(1, -1, D) * 0.5
    vz[..., 2, 3] = 2.0
    cases.append(run_case(torch, ref, log, "l_zero_cvt_N4_D32", onehot.clone(), onehot.clone(), vz,
                          scale=scale_l0))

    # 5c. the running sum starts at l = 1 (kernel.py:139, 242): rows that are fully masked
    #     and carry zero queries see every logit equal to the mask value, so the
    #     first step's release of l (alpha = E(NEG_INF - m')) is not rounded away
    #     and an initial l = 0 would shift every code of those rows.
    q, k, v = (torch.randn(1, 1, 8, 32, generator=g) for _ in range(3))
    q[:, :, :4] = 0.0
    v = (4.0 * (torch.arange(32) % 31 + 1)).float().expand(1, 1, 8, 32).clone()
    v[..., 0, 31] = 127.0
    bm3 = torch.ones(1, 1, 8, 8, dtype=torch.bool)
    bm3[:, :, :4] = False
    cases.append(run_case(torch, ref, log, "masked_rows_l_init_N8_D32", q, k, v, attn_mask=bm3))

    # 6. arithmetic-variant flags (kernel.py:30-36), each its own import.
    variants = {
        "expidiv": {"QFLASH_EXP_USE_SHIFT": "0"},
        "lidiv": {"QFLASH_L_USE_SHIFT": "0"},
        "accidiv": {"QFLASH_ACC_USE_SHIFT": "0"},
        "shift20_24": {"QFLASH_L_SHIFT": "20", "QFLASH_ACC_SHIFT": "24"},
        "allidiv": {"QFLASH_EXP_USE_SHIFT": "0", "QFLASH_L_USE_SHIFT": "0", "QFLASH_ACC_USE_SHIFT": "0"},
    }
    qv, kv, vv = outlier_qkv(g, torch, 1, 2, 97, 64, torch.float32)
    for tag, env in variants.items():
        mod, vlog = load_reference(env, tag)
        cases.append(run_case(torch, mod, vlog, f"flags_{tag}_N97_D64", qv, kv, vv))
        cases.append(run_case(torch, mod, vlog, f"flags_{tag}_swin_N49_D32", *swin_qkv, attn_mask=amask))

    # Identical arrays (shared inputs, masks, biases) are stored once; later
    # occurrences hold the string "@<first key>" (resolved by tests/golden_io.py).
    out, seen = {}, {}
    for name, d in cases:
        for key, val in d.items():
            val = np.asarray(val)
            sig = (val.dtype.str, val.shape, hashlib.sha1(val.tobytes()).hexdigest())
            if val.nbytes > 64 and sig in seen:
                out[f"{name}/{key}"] = np.array("@" + seen[sig])
            else:
                seen.setdefault(sig, f"{name}/{key}")
                out[f"{name}/{key}"] = val
    path = os.path.join(HERE, "golden_reference.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {len(cases)} cases to {path} ({os.path.getsize(path) / 1e6:.2f} MB)")


if __name__ == "__main__":
    sys.exit(main())
