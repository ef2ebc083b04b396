"""ctypes wrapper of the C oracle (oracle/qflash_oracle.c).

TEST INFRASTRUCTURE ONLY (tests/, smoke() checker, bench.py cpu_baseline).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

from .qflash_oracle import Consts, Flags

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libqflash_oracle.so")


class _Params(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "sm_rscale", "exp_M", "req_M", "l_M", "acc_M",
        "exp_use_shift", "l_use_shift", "acc_use_shift", "l_shift", "acc_shift")]


def build(force: bool = False) -> str:
    """Compile the oracle with oracle/Makefile (make decides what is stale)."""
    args = ["make", "-s", "-C", HERE]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.qfo_attention_codes.restype = ctypes.c_int
        L.qfo_attention_codes.argtypes = [ctypes.c_void_p] * 5 + [
            ctypes.POINTER(ctypes.c_int64), ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.POINTER(_Params), ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.qfo_exp2_requant.restype = None
        L.qfo_exp2_requant.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64, ctypes.POINTER(_Params)]
        L.qfo_release_n.restype = None
        L.qfo_release_n.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int64] + [ctypes.c_int32] * 2 + [
            ctypes.c_int, ctypes.c_int32]
        _lib = L
    return _lib


def params(c: Consts, f: Flags = Flags()) -> _Params:
    return _Params(c.sm_rscale, c.exp_M, c.req_M, c.l_M, c.acc_M,
                   int(f.exp_use_shift), int(f.l_use_shift), int(f.acc_use_shift), f.l_shift, f.acc_shift)


def _np_view(a):
    """numpy view (no copy) of a numpy array or CPU torch tensor, with element strides."""
    if hasattr(a, "numpy"):
        a = a.detach().numpy()
    a = np.asarray(a)
    return a, [s // a.itemsize for s in a.strides]


def attention_codes(q, k, v, c: Consts, f: Flags = Flags(), bias=None, threads: int | None = None,
                    zh_range: tuple[int, int] | None = None, out=None):
    """int8 codes (Z,H,N,D); inputs may be strided; bias broadcastable (Z,H,N,N)."""
    qa, qs = _np_view(q)
    ka, ks = _np_view(k)
    va, vs = _np_view(v)
    Z, H, N, D = qa.shape
    assert qa.dtype == np.int8 and ka.dtype == np.int8 and va.dtype == np.int8
    if out is None:
        out = np.zeros((Z, H, N, D), dtype=np.int8)
    oa, os_ = _np_view(out)
    bptr, bs = None, [0, 0, 0, 0]
    if bias is not None:
        ba, _ = _np_view(bias)
        ba = np.broadcast_to(ba.astype(np.int32, copy=False), (Z, H, N, N))
        bs = [s // ba.itemsize for s in ba.strides]
        bptr = ba.ctypes.data
    st = (ctypes.c_int64 * 20)(*(qs + ks + vs + os_ + bs))
    p = params(c, f)
    lo, hi = zh_range if zh_range else (0, 0)
    rc = lib().qfo_attention_codes(qa.ctypes.data, ka.ctypes.data, va.ctypes.data, oa.ctypes.data, bptr,
                                   st, Z, H, N, D, ctypes.byref(p), threads or os.cpu_count() or 1, lo, hi)
    if rc != 0:
        raise RuntimeError(f"qfo_attention_codes failed with code {rc}")
    return out


def exp2_requant(x, c: Consts, f: Flags = Flags()):
    x = np.ascontiguousarray(x, dtype=np.int32)
    e = np.empty_like(x)
    pq = np.empty_like(x)
    p = params(c, f)
    lib().qfo_exp2_requant(x.ctypes.data, e.ctypes.data, pq.ctypes.data, x.size, ctypes.byref(p))
    return e, pq


def release(x, alpha, M: int, shift: int, use_shift: bool, rs: int):
    x = np.ascontiguousarray(x, dtype=np.int32)
    alpha = np.ascontiguousarray(np.broadcast_to(alpha, x.shape), dtype=np.int32)
    out = np.empty_like(x)
    lib().qfo_release_n(x.ctypes.data, alpha.ctypes.data, out.ctypes.data, x.size, M, shift, int(use_shift), rs)
    return out
