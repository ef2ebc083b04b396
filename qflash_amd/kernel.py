"""Host side of the integer attention forward: the ``qflash`` op namespace.

Mirrors EfficientCompLab/qflash ``qflash/kernel.py`` for this hot path:

* ``qflash_forward`` follows kernel.py:275-351 step for step (asserts, scale,
  per-tensor absmax scales with the one ``.item()`` sync, fixed-point
  constants in Python double arithmetic, quantisation, mask -> int32 bias,
  launch on torch's current stream, ``o * o_scale``), and raises the same
  exceptions; the scales and the int8 quantisation run as two HIP passes
  (``quantize_qkv``) with torch's GPU arithmetic;
* ``qflash_kernel`` / ``qflash_masked_kernel`` are launchers with the
  reference's launch signature (kernel.py:319-326, :339-346) that call the
  gfx950 HIP kernels through the C ABI (include/qflash_hip.h);
* ``class qflash`` is the namespace of kernel.py:354-356.

There is no CPU fallback: inputs must live on a GPU and the HIP library
must be built, otherwise an exception is raised.
"""
from __future__ import annotations

import ctypes
import os
import statistics
import threading

import torch
from torch import Tensor

from . import _lib

# kernel.py:30-36 - read once at import, like the reference.
AUTOTUNE_SETTING = os.environ.get("QFLASH_AUTOTUNE", "default")
USE_CUDA_GRAPH = os.environ.get("QFLASH_CUDA_GRAPH", "0") == "1"
EXP_USE_SHIFT = os.environ.get("QFLASH_EXP_USE_SHIFT", "1") == "1"
L_USE_SHIFT = os.environ.get("QFLASH_L_USE_SHIFT", "1") == "1"
ACC_USE_SHIFT = os.environ.get("QFLASH_ACC_USE_SHIFT", "1") == "1"
L_SHIFT = int(os.environ.get("QFLASH_L_SHIFT", "30"))
ACC_SHIFT = int(os.environ.get("QFLASH_ACC_SHIFT", "30"))

LOG2E = 1.44269504      # kernel.py:287 (the literal)
NEG_INF = -(1 << 20)    # kernel.py:288
SHIFT = 16              # kernel.py:301
INT8_MAX = torch.iinfo(torch.int8).max
_I32 = (-(1 << 31), (1 << 31) - 1)


def fixed_point_constants(sm_scale: float, l_shift: int = None, acc_shift: int = None):
    """(sm_rscale, exp_M, req_M, l_M, acc_M) from sm_scale, kernel.py:300-307.

    Python double arithmetic and half-to-even ``round``; raises
    ZeroDivisionError / ValueError / OverflowError exactly where the reference
    does (sm_scale == 0, sm_scale > 2, NaN, inf).
    """
    l_shift = L_SHIFT if l_shift is None else l_shift
    acc_shift = ACC_SHIFT if acc_shift is None else acc_shift
    sm_rscale = int(round(1.0 / sm_scale))
    exp_M = int(round(-sm_scale * (1 << SHIFT)))
    req_M = int(round(sm_scale * 127 * (1 << SHIFT)))
    l_M = int(round((1 << l_shift) / sm_rscale))
    acc_M = int(round((1 << acc_shift) / sm_rscale))
    return sm_rscale, exp_M, req_M, l_M, acc_M


def quantize(x: Tensor, x_scale: Tensor) -> Tensor:
    """clamp(round(x / scale), -128, 127) as int8, kernel.py:309-311."""
    return torch.clamp(torch.round(x / x_scale), -128, 127).to(torch.int8)


def bias_values(attn_mask: Tensor, sm_scale: float) -> Tensor:
    """Elementwise mask -> int32 logit bias, same shape as the mask (kernel.py:327-336).

    bool: 0 where True, NEG_INF where False.  float: values < -1e2 are masked
    (NEG_INF), the others become round(x * LOG2E / sm_scale) in the mask's
    dtype, as the reference's torch ops compute them.
    """
    if attn_mask.dtype == torch.bool:
        bias = torch.zeros(attn_mask.shape, dtype=torch.int32, device=attn_mask.device)
        return bias.masked_fill_(attn_mask.logical_not(), NEG_INF)
    is_masked = attn_mask < -1e2
    clipped = attn_mask.masked_fill(is_masked, 0.0)
    quant = (clipped * LOG2E / sm_scale).round().to(torch.int32)
    return quant.masked_fill(is_masked, NEG_INF)


def window_bias(rel_bias: Tensor, mask: Tensor | None, sm_scale: float) -> Tensor:
    """bias_values(rel_bias + mask.view(nW, 1, N, N), sm_scale) (or of rel_bias
    alone when mask is None) as a contiguous (nW or 1, H, N, N) int32 tensor.

    fp32 inputs on the device take qflash_hip_window_bias (one pass instead
    of the eight torch kernels, same values); other dtypes keep the torch
    ops, whose arithmetic is in the mask's dtype.
    """
    H, N = rel_bias.shape[-3], rel_bias.shape[-1]
    fp32 = rel_bias.dtype == torch.float32 and (mask is None or mask.dtype == torch.float32)
    if not (fp32 and rel_bias.is_cuda and (mask is None or mask.is_cuda)):
        x = rel_bias.reshape(1, H, N, N) if mask is None else rel_bias + mask.view(mask.shape[0], 1, N, N)
        return bias_values(x, sm_scale).contiguous()
    rel = rel_bias.reshape(H, N, N).contiguous()
    m = None if mask is None else mask.contiguous()
    n_win = 1 if m is None else m.shape[0]
    out = torch.empty((n_win, H, N, N), dtype=torch.int32, device=rel.device)
    L = _lib.load()
    _lib.check(L.qflash_hip_window_bias(ctypes.c_void_p(rel.data_ptr()),
                                        ctypes.c_void_p(0 if m is None else m.data_ptr()), n_win, H, N,
                                        float(sm_scale), ctypes.c_void_p(out.data_ptr()), _stream_ptr(rel)),
               "qflash_hip_window_bias")
    return out


def mask_to_bias(attn_mask: Tensor, sm_scale: float, Z: int, H: int, N: int, materialize: bool = False) -> Tensor:
    """Boolean or float mask -> int32 logit bias of shape (Z, H, N, N), kernel.py:327-336.

    The values equal the reference's; by default the result is an expanded
    view (stride 0 on broadcast dims) instead of a materialised copy, which
    the kernels read through their strides.
    """
    if attn_mask.dtype == torch.float32 and attn_mask.is_cuda and 0 < attn_mask.numel() < (1 << 31):
        # one HIP pass (qflash_hip_mask_bias) with the values of bias_values' torch ops
        m = attn_mask.contiguous()
        b = torch.empty(m.shape, dtype=torch.int32, device=m.device)
        _lib.check(_lib.load().qflash_hip_mask_bias(ctypes.c_void_p(m.data_ptr()), m.numel(), float(sm_scale),
                                                    ctypes.c_void_p(b.data_ptr()), _stream_ptr(m)),
                   "qflash_hip_mask_bias")
    else:
        b = bias_values(attn_mask, sm_scale)
    bias = b.expand(Z, H, N, N)
    return bias.contiguous() if materialize else bias


def _check_i32(**consts):
    for name, val in consts.items():
        if not (_I32[0] <= val <= _I32[1]):
            raise _lib.QFlashLibraryError(
                f"{name}={val} does not fit int32; the gfx950 kernels take int32 constants")


def _stream_ptr(t: Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


class _Launcher:
    """Launch object with the reference's ``kernel[grid](...)`` call form.

    The grid argument is accepted and ignored: the HIP library chooses its
    own decomposition.  Positional arguments follow kernel.py:319-326
    (unmasked) or :339-346 (masked).
    """

    def __init__(self, masked: bool):
        self.masked = masked
        self.__name__ = "qflash_masked_kernel" if masked else "qflash_kernel"

    def __getitem__(self, grid):
        return self

    def __call__(self, *args, N_CTX: int, HEAD_DIM: int, EXP_USE_SHIFT: bool = True, L_USE_SHIFT: bool = True,
                 ACC_USE_SHIFT: bool = True, L_SHIFT: int = 16, ACC_SHIFT: int = 16, **_ignored):
        n_t = 5 if self.masked else 4
        n_s = 20 if self.masked else 16
        if len(args) != n_t + 7 + n_s:
            raise TypeError(f"{self.__name__}: expected {n_t + 7 + n_s} positional arguments, got {len(args)}")
        tensors = args[:n_t]
        consts = [int(c) for c in args[n_t:n_t + 5]]
        strides = [int(s) for s in args[n_t + 5:n_t + 5 + n_s]]
        Z, H = (int(x) for x in args[n_t + 5 + n_s:n_t + 7 + n_s])
        for t in tensors:
            if not t.is_cuda:
                raise ValueError(f"{self.__name__}: all tensors must be on a GPU device (got {t.device})")
        _check_i32(sm_rscale=consts[0], exp_M=consts[1], req_M=consts[2], l_M=consts[3], acc_M=consts[4])
        L = _lib.load()
        fl = _lib.Flags(int(EXP_USE_SHIFT), int(L_USE_SHIFT), int(ACC_USE_SHIFT), int(L_SHIFT), int(ACC_SHIFT))
        st = (ctypes.c_int64 * n_s)(*strides)
        stream = _stream_ptr(tensors[0])
        ptr = [ctypes.c_void_p(t.data_ptr()) for t in tensors]
        if self.masked:
            rc = L.qflash_hip_masked_kernel(*ptr, *consts, st, Z, H, int(N_CTX), int(HEAD_DIM), ctypes.byref(fl),
                                            stream)
        else:
            rc = L.qflash_hip_kernel(*ptr, *consts, st, Z, H, int(N_CTX), int(HEAD_DIM), ctypes.byref(fl), stream)
        _lib.check(rc, self.__name__)


qflash_kernel = _Launcher(masked=False)
qflash_masked_kernel = _Launcher(masked=True)


def qflash_window_kernel(q8: Tensor, k8: Tensor, v8: Tensor, o: Tensor, bias: Tensor, consts, bias_zmod: int,
                         flags: dict) -> None:
    """Masked launch with a window-periodic bias (include/qflash_hip.h: qflash_hip_window_kernel).

    bias has shape (bias_zmod, H, N, N); batch index z of Q/K/V/O uses
    bias[z % bias_zmod].  No counterpart in the reference: QWindowAttention's
    (B_, H, N, N) mask repeats every nW windows, and this launch reads the nW
    distinct slices instead of a materialised copy.
    """
    Z, H, N, D = q8.shape
    for t in (q8, k8, v8, o, bias):
        if not t.is_cuda:
            raise ValueError(f"qflash_window_kernel: all tensors must be on a GPU device (got {t.device})")
    if bias.dtype != torch.int32 or bias.shape != (bias_zmod, H, N, N):
        raise ValueError(f"qflash_window_kernel: bias must be int32 ({bias_zmod}, {H}, {N}, {N}), got "
                         f"{tuple(bias.shape)} {bias.dtype}")
    c = [int(x) for x in consts]
    _check_i32(sm_rscale=c[0], exp_M=c[1], req_M=c[2], l_M=c[3], acc_M=c[4])
    L = _lib.load()
    fl = _lib.Flags(int(flags["EXP_USE_SHIFT"]), int(flags["L_USE_SHIFT"]), int(flags["ACC_USE_SHIFT"]),
                    int(flags["L_SHIFT"]), int(flags["ACC_SHIFT"]))
    st = (ctypes.c_int64 * 20)(*q8.stride(), *k8.stride(), *v8.stride(), *o.stride(), *bias.stride())
    ptr = [ctypes.c_void_p(t.data_ptr()) for t in (q8, k8, v8, o, bias)]
    rc = L.qflash_hip_window_kernel(*ptr, *c, st, Z, H, N, D, int(bias_zmod), ctypes.byref(fl), _stream_ptr(q8))
    _lib.check(rc, "qflash_window_kernel")


def bench_latency_ms(fn, warmup: float = 10, rep: float = 100, flush_mb: int = 512, device=None) -> float:
    """Median kernel time in ms, like triton.testing.do_bench(return_mode='median').

    warmup / rep are time budgets in ms; before every timed run a buffer of
    flush_mb MB is zeroed so the last-level caches (256 MB MALL on MI355X)
    do not hold the inputs.  Events are recorded on torch's current stream,
    the stream the kernels are launched on.
    """
    dev = device or torch.device("cuda", torch.cuda.current_device())
    cache = torch.empty(flush_mb * (1 << 20) // 4, dtype=torch.int32, device=dev)
    fn()
    torch.cuda.synchronize(dev)
    s = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
    e = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
    for i in range(5):
        cache.zero_()
        s[i].record()
        fn()
        e[i].record()
    torch.cuda.synchronize(dev)
    est = max(sum(a.elapsed_time(b) for a, b in zip(s, e)) / 5, 1e-4)
    n_warmup = max(1, int(warmup / est))
    n_rep = max(1, int(rep / est))
    for _ in range(n_warmup):
        fn()
    s = [torch.cuda.Event(enable_timing=True) for _ in range(n_rep)]
    e = [torch.cuda.Event(enable_timing=True) for _ in range(n_rep)]
    for i in range(n_rep):
        cache.zero_()
        s[i].record()
        fn()
        e[i].record()
    torch.cuda.synchronize(dev)
    return statistics.median(a.elapsed_time(b) for a, b in zip(s, e))


_DT_CODE = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


_ws_cache = threading.local()
_host_cache = threading.local()


def _scalar_to_host(x: Tensor):
    """Start copying the 1-element device tensor ``x`` to pinned host memory on the
    current stream; the returned function waits for that copy only (not for work
    queued after it) and returns ``x.item()``."""
    bufs = getattr(_host_cache, "d", None)
    if bufs is None:
        bufs = _host_cache.d = {}
    buf = bufs.get(x.dtype)
    if buf is None:
        buf = bufs[x.dtype] = torch.empty(1, dtype=x.dtype, pin_memory=True)
    buf.copy_(x.reshape(1), non_blocking=True)
    done = torch.cuda.Event()
    done.record(torch.cuda.current_stream(x.device))

    def wait():
        done.synchronize()
        return buf.item()
    return wait


def _scales_workspace(device) -> Tensor:
    """The absmax pass's workspace for this thread and device's current stream:
    zeroed once, and left zeroed by every call when it completes (calls on one
    stream follow each other in stream order).  A stream seen for the first
    time during HIP graph capture takes the spare workspace that an earlier
    eager call zeroed, so that the zero fill is not captured into the graph and
    repeated by every replay."""
    cache = getattr(_ws_cache, "d", None)
    if cache is None:
        cache = _ws_cache.d = {}
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = cache.get(key)
    if ws is None:
        spare_key = (device.index, "spare")
        if torch.cuda.is_current_stream_capturing() and spare_key in cache:
            ws = cache[key] = cache.pop(spare_key)
        else:
            ws = cache[key] = torch.zeros(_lib.SCALES_WORKSPACE, dtype=torch.int32, device=device)
    if not torch.cuda.is_current_stream_capturing() and (device.index, "spare") not in cache:
        spare = torch.zeros(_lib.SCALES_WORKSPACE, dtype=torch.int32, device=device)
        torch.cuda.current_stream(device).synchronize()  # once per thread and device: zero before any capture
        cache[(device.index, "spare")] = spare
    return ws


def _drop_scales_workspace(device) -> None:
    """Forget this thread's workspace after a failed call: a launch that failed
    between the absmax pass and the pass that clears the slots would leave
    stale maxima in it, so the next call starts from a fresh zeroed one."""
    cache = getattr(_ws_cache, "d", None)
    if cache is not None:
        cache.pop((device.index, torch.cuda.current_stream(device).cuda_stream), None)


def quantize_qkv(query: Tensor, key: Tensor, value: Tensor):
    """Per-tensor scales and int8 codes of Q, K, V on the device (kernel.py:294-311).

    Returns ``(scales, finish)``: ``scales`` is a 4-element device tensor in the
    inputs' dtype holding q_scale, k_scale, o_scale and q_scale * k_scale
    (values identical to ``x.abs().amax() / 127`` and their product as torch
    computes them on the GPU); ``finish()`` launches the quantisation and
    returns (q8, k8, v8), each laid out like its input (``empty_like``).  The
    split lets the caller compute the fixed-point constants, which may raise,
    between the two, in the reference's order.  Two HIP passes replace torch's
    twelve; dtypes other than fp32 / fp16 / bf16 use the torch sequence.
    """
    T = query.dtype
    for x in (query, key, value):
        if not x.is_cuda:
            raise ValueError(f"qflash: all tensors must be on a GPU device (got {x.device})")
    if T not in _DT_CODE or key.dtype != T or value.dtype != T or query.dim() != 4 or key.dim() != 4 \
            or value.dim() != 4:
        q_scale = query.abs().amax() / INT8_MAX
        k_scale = key.abs().amax() / INT8_MAX
        o_scale = value.abs().amax() / INT8_MAX
        scales = torch.stack([q_scale, k_scale, o_scale, q_scale * k_scale])

        def finish_torch():
            return quantize(query, q_scale), quantize(key, k_scale), quantize(value, o_scale)
        return scales, finish_torch
    scales, _, finish = _hip_scales(query, key, value, None)
    return scales, finish


def _hip_scales(query: Tensor, key: Tensor, value: Tensor, plan):
    """quantize_qkv's HIP path for fp32 / fp16 / bf16 (Z, H, N, D) inputs of
    one dtype.  plan: None, or (scale, N, D, masked) of device_constants: then
    the constants are formed in the same one-wave kernel as the scales
    (qflash_hip_scales_constants).  Returns (scales, params or None, finish)."""
    L = _lib.load()
    code = _DT_CODE[query.dtype]
    geo = (ctypes.c_int64 * 24)(*query.shape, *query.stride(), *key.shape, *key.stride(), *value.shape,
                                 *value.stride())
    ws = _scales_workspace(query.device)
    scales = torch.empty(4, dtype=query.dtype, device=query.device)
    stream = _stream_ptr(query)
    ptrs = [ctypes.c_void_p(x.data_ptr()) for x in (query, key, value)]
    params = None
    if plan is None:
        rc = L.qflash_hip_scales(*ptrs, code, geo, ctypes.c_void_p(scales.data_ptr()),
                                 ctypes.c_void_p(ws.data_ptr()), ws.numel(), stream)
    else:
        scale, N, D, masked = plan
        params = torch.empty(_lib.PARAMS_WORDS, dtype=torch.int32, device=query.device)
        rc = L.qflash_hip_scales_constants(*ptrs, code, geo, ctypes.c_void_p(scales.data_ptr()),
                                           ctypes.c_void_p(ws.data_ptr()), ws.numel(), float(scale), int(N), int(D),
                                           int(masked), ctypes.byref(_flags()), ctypes.c_void_p(params.data_ptr()),
                                           stream)
    if rc != 0:
        _drop_scales_workspace(query.device)
    _lib.check(rc, "qflash_hip_scales" if plan is None else "qflash_hip_scales_constants")

    def finish():
        q8, k8, v8 = (torch.empty_like(x, dtype=torch.int8) for x in (query, key, value))
        ost = (ctypes.c_int64 * 12)(*q8.stride(), *k8.stride(), *v8.stride())
        _lib.check(L.qflash_hip_quantize(*ptrs, code, geo, ctypes.c_void_p(q8.data_ptr()),
                                         ctypes.c_void_p(k8.data_ptr()), ctypes.c_void_p(v8.data_ptr()), ost,
                                         ctypes.c_void_p(scales.data_ptr()), _stream_ptr(query)),
                   "qflash_hip_quantize")
        return q8, k8, v8
    return scales, params, finish


def launch_forward(q8: Tensor, k8: Tensor, v8: Tensor, out: Tensor, consts, flags: dict, bias: Tensor | None = None,
                   bias_zmod: int = 0, o_scale: Tensor | None = None) -> None:
    """One launch of the integer forward through qflash_hip_forward.

    ``out`` is int8 (the codes) or fp32 / fp16 / bf16: then it receives
    ``code * o_scale`` rounded to its dtype, the reference's final ``o * o_scale``
    (kernel.py:351) fused into the kernel; ``o_scale`` is a device scalar of
    that dtype.  ``bias``: None, (Z, H, N, N) strided, or (bias_zmod, H, N, N)
    window-periodic.
    """
    Z, H, N, D = q8.shape
    for t in (q8, k8, v8, out) + (() if bias is None else (bias,)):
        if not t.is_cuda:
            raise ValueError(f"qflash: all tensors must be on a GPU device (got {t.device})")
    if out.dtype == torch.int8:
        code, sp = _lib.I8, None
    else:
        code = _DT_CODE.get(out.dtype)
        if code is None or o_scale is None or o_scale.dtype != out.dtype or not o_scale.is_cuda:
            raise ValueError("qflash: a dequantised output needs a device o_scale of the output dtype "
                             f"(fp32 / fp16 / bf16), got {out.dtype} and {o_scale}")
        sp = ctypes.c_void_p(o_scale.data_ptr())
    c = [int(x) for x in consts]
    _check_i32(sm_rscale=c[0], exp_M=c[1], req_M=c[2], l_M=c[3], acc_M=c[4])
    L = _lib.load()
    fl = _lib.Flags(int(flags["EXP_USE_SHIFT"]), int(flags["L_USE_SHIFT"]), int(flags["ACC_USE_SHIFT"]),
                    int(flags["L_SHIFT"]), int(flags["ACC_SHIFT"]))
    bst = (0, 0, 0, 0) if bias is None else bias.stride()
    st = (ctypes.c_int64 * 20)(*q8.stride(), *k8.stride(), *v8.stride(), *out.stride(), *bst)
    bp = None if bias is None else ctypes.c_void_p(bias.data_ptr())
    rc = L.qflash_hip_forward(ctypes.c_void_p(q8.data_ptr()), ctypes.c_void_p(k8.data_ptr()),
                              ctypes.c_void_p(v8.data_ptr()), ctypes.c_void_p(out.data_ptr()), code, sp, bp,
                              int(bias_zmod), *c, st, Z, H, N, D, ctypes.byref(fl), _stream_ptr(q8))
    _lib.check(rc, "qflash_hip_forward")


def _flags():
    return _lib.Flags(int(EXP_USE_SHIFT), int(L_USE_SHIFT), int(ACC_USE_SHIFT), int(L_SHIFT), int(ACC_SHIFT))


def _flag_kw():
    return dict(EXP_USE_SHIFT=EXP_USE_SHIFT, L_USE_SHIFT=L_USE_SHIFT, ACC_USE_SHIFT=ACC_USE_SHIFT,
                L_SHIFT=L_SHIFT, ACC_SHIFT=ACC_SHIFT)


def device_constants(scales: Tensor, scale: float, N: int, D: int, masked: bool,
                     params: Tensor | None = None) -> Tensor:
    """The fixed-point constants on the device (qflash_hip_constants): a device
    int32 block of _lib.PARAMS_WORDS words holding a status (0, or the
    exception the reference's host would raise, see raise_status), sm_rscale,
    exp_M, req_M, l_M, acc_M (kernel.py:297-307, Python's double arithmetic),
    the fast kernel's plan and sm_scale.  `scales` from quantize_qkv; `scale`
    the host's (scale or 1/sqrt(D)) * LOG2E; `params`: the block to write (a
    new one when None).  Asynchronous, no host sync."""
    if params is None:
        params = torch.empty(_lib.PARAMS_WORDS, dtype=torch.int32, device=scales.device)
    fl = _flags()
    _lib.check(_lib.load().qflash_hip_constants(ctypes.c_void_p(scales.data_ptr()), _DT_CODE[scales.dtype],
                                                float(scale), int(N), int(D), int(masked), ctypes.byref(fl),
                                                ctypes.c_void_p(params.data_ptr()), _stream_ptr(scales)),
               "qflash_hip_constants")
    return params


def raise_status(status: int) -> None:
    """Raise what the reference's host raises for the value that produced this
    status of qflash_hip_constants (kernel.py:302-307, then the int32 check of
    the launch); nothing for 0."""
    if status == 0:
        return
    if status == _lib.STATUS_ZERODIV_SCALE:
        raise ZeroDivisionError("float division by zero")
    if status == _lib.STATUS_NAN:
        raise ValueError("cannot convert float NaN to integer")
    if status == _lib.STATUS_INF:
        raise OverflowError("cannot convert float infinity to integer")
    if status == _lib.STATUS_ZERODIV_RSCALE:
        raise ZeroDivisionError("division by zero")
    if status == _lib.STATUS_RANGE:
        raise _lib.QFlashLibraryError("a fixed-point constant does not fit int32; the gfx950 kernels take int32 "
                                      "constants")
    raise _lib.QFlashLibraryError(f"qflash_hip_constants: unknown status {status}")


def _status_check(params: Tensor):
    """Call right after the constants kernel is queued.  Eager mode: returns a
    function that copies the status word to pinned host memory on a side
    stream (after the constants kernel: the launch stream goes straight on),
    waits for that copy only and raises the reference's exception; call it
    once the rest of the forward is queued.  Under HIP graph capture: no copy,
    no check (nothing may synchronise; a failing status leaves the outputs
    unwritten)."""
    if torch.cuda.is_current_stream_capturing():
        return lambda: None
    done = torch.cuda.Event()
    done.record(torch.cuda.current_stream(params.device))

    def check():
        side = _side_stream(params.device)
        side.wait_event(done)
        with torch.cuda.stream(side):
            wait = _scalar_to_host(params[0])
        raise_status(int(wait()))
    return check


def _side_stream(device) -> torch.cuda.Stream:
    """This thread's side stream on `device` (default priority)."""
    cache = getattr(_host_cache, "side", None)
    if cache is None:
        cache = _host_cache.side = {}
    st = cache.get(device.index)
    if st is None:
        st = cache[device.index] = torch.cuda.Stream(device=device)
    return st


def mask_to_bias_planned(attn_mask: Tensor, params: Tensor, Z: int, H: int, N: int) -> Tensor:
    """mask_to_bias with sm_scale read on the device from `params` (fp32 masks:
    qflash_hip_mask_bias_planned; bool masks need no sm_scale)."""
    if attn_mask.dtype == torch.bool:
        return bias_values(attn_mask, 1.0).expand(Z, H, N, N)
    m = attn_mask.contiguous()
    b = torch.empty(m.shape, dtype=torch.int32, device=m.device)
    _lib.check(_lib.load().qflash_hip_mask_bias_planned(ctypes.c_void_p(m.data_ptr()), m.numel(),
                                                        ctypes.c_void_p(params.data_ptr()),
                                                        ctypes.c_void_p(b.data_ptr()), _stream_ptr(m)),
               "qflash_hip_mask_bias_planned")
    return b.expand(Z, H, N, N)


def window_bias_planned(rel_bias: Tensor, mask: Tensor | None, params: Tensor) -> Tensor:
    """window_bias with sm_scale read on the device from `params` (fp32 tables)."""
    H, N = rel_bias.shape[-3], rel_bias.shape[-1]
    rel = rel_bias.reshape(H, N, N).contiguous()
    m = None if mask is None else mask.contiguous()
    n_win = 1 if m is None else m.shape[0]
    out = torch.empty((n_win, H, N, N), dtype=torch.int32, device=rel.device)
    _lib.check(_lib.load().qflash_hip_window_bias_planned(
        ctypes.c_void_p(rel.data_ptr()), ctypes.c_void_p(0 if m is None else m.data_ptr()), n_win, H, N,
        ctypes.c_void_p(params.data_ptr()), ctypes.c_void_p(out.data_ptr()), _stream_ptr(rel)),
        "qflash_hip_window_bias_planned")
    return out


def launch_forward_planned(q8: Tensor, k8: Tensor, v8: Tensor, out: Tensor, params: Tensor,
                           bias: Tensor | None = None, bias_zmod: int = 0, o_scale: Tensor | None = None) -> None:
    """launch_forward with the constants in the device block `params`
    (qflash_hip_forward_planned)."""
    Z, H, N, D = q8.shape
    if out.dtype == torch.int8:
        code, sp = _lib.I8, None
    else:
        code = _DT_CODE[out.dtype]
        sp = ctypes.c_void_p(o_scale.data_ptr())
    fl = _flags()
    bst = (0, 0, 0, 0) if bias is None else bias.stride()
    st = (ctypes.c_int64 * 20)(*q8.stride(), *k8.stride(), *v8.stride(), *out.stride(), *bst)
    bp = None if bias is None else ctypes.c_void_p(bias.data_ptr())
    rc = _lib.load().qflash_hip_forward_planned(
        ctypes.c_void_p(q8.data_ptr()), ctypes.c_void_p(k8.data_ptr()), ctypes.c_void_p(v8.data_ptr()),
        ctypes.c_void_p(out.data_ptr()), code, sp, bp, int(bias_zmod), ctypes.c_void_p(params.data_ptr()), st, Z, H,
        N, D, ctypes.byref(fl), _stream_ptr(q8))
    _lib.check(rc, "qflash_hip_forward_planned")


def _device_path(query: Tensor, key: Tensor, value: Tensor, attn_mask: Tensor | None) -> bool:
    """Inputs whose whole forward runs on the device (constants included):
    fp32 / fp16 / bf16 (Z, H, N, D) tensors of one dtype, and no mask, a bool
    mask or an fp32 mask on the device."""
    T = query.dtype
    if T not in _DT_CODE or key.dtype != T or value.dtype != T:
        return False
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        return False
    if attn_mask is None or attn_mask.dtype == torch.bool:
        return True
    return attn_mask.dtype == torch.float32 and attn_mask.is_cuda and 0 < attn_mask.numel() < (1 << 31)


def qflash_forward(
    query: Tensor,
    key: Tensor,
    value: Tensor,
    attn_mask: Tensor | None = None,
    scale: float | None = None,
    return_mode: str = 'output',
):
    """Integer-only attention, drop-in for qflash.forward (kernel.py:275-351).

    query/key/value: (Z, H, N, D) floating tensors on the GPU, any strides.
    attn_mask: None, bool (True = keep) or float additive mask broadcastable
    to (Z, H, N, N).  Returns ``o_int8 * o_scale`` in the input dtype, or the
    median kernel time in ms for return_mode='latency'.

    fp32 / fp16 / bf16 inputs run entirely on the device, constants included
    (no host synchronisation, so the call can be captured in a HIP graph);
    in eager mode the exceptions the reference raises while forming its
    constants are raised before the call returns.  Other dtypes follow the
    reference's host sequence.
    """
    d_q, d_k, d_v = query.shape[-1], key.shape[-1], value.shape[-1]
    assert d_q == d_k and d_k == d_v
    assert d_k in {16, 32, 64, 128, 256}

    if scale is None:
        scale = 1.0 / (d_q ** 0.5)
    scale = scale * LOG2E
    for x in (query, key, value):
        if not x.is_cuda:
            raise ValueError(f"qflash: all tensors must be on a GPU device (got {x.device})")
    if _device_path(query, key, value, attn_mask):
        return _forward_device(query, key, value, attn_mask, scale, return_mode)

    scales, finish = quantize_qkv(query, key, value)  # kernel.py:294-296 on the device
    o_scale = scales[2]
    qk_scale = _scalar_to_host(scales[3])
    # kernel.py:309-311: the quantisation needs only the device scales, so it is
    # queued before the host waits for q_scale * k_scale (the reference's one
    # sync, kernel.py:297); the host then forms the constants while it runs
    q8, k8, v8 = finish()
    sm_scale = scale * qk_scale()
    sm_rscale, exp_M, req_M, l_M, acc_M = fixed_point_constants(sm_scale)
    Z, H, N = q8.shape[0], q8.shape[1], q8.shape[2]
    consts = (sm_rscale, exp_M, req_M, l_M, acc_M)
    flag_kw = dict(EXP_USE_SHIFT=EXP_USE_SHIFT, L_USE_SHIFT=L_USE_SHIFT, ACC_USE_SHIFT=ACC_USE_SHIFT,
                   L_SHIFT=L_SHIFT, ACC_SHIFT=ACC_SHIFT)
    bias = None if attn_mask is None else mask_to_bias(attn_mask, sm_scale, Z, H, N)

    if return_mode == 'latency':  # the kernel alone, int8 codes out (kernel.py:348-349)
        o = torch.empty_like(v8)
        return bench_latency_ms(lambda: launch_forward(q8, k8, v8, o, consts, flag_kw, bias), device=query.device)
    if o_scale.dtype in _DT_CODE:  # o * o_scale fused into the kernel's stores
        out = torch.empty_like(v8, dtype=o_scale.dtype)
        launch_forward(q8, k8, v8, out, consts, flag_kw, bias, o_scale=o_scale)
        return out
    o = torch.empty_like(v8)
    launch_forward(q8, k8, v8, o, consts, flag_kw, bias)
    return o * o_scale


def _forward_device(query: Tensor, key: Tensor, value: Tensor, attn_mask: Tensor | None, scale: float,
                    return_mode: str):
    """qflash_forward on the device: scales, constants, quantisation, bias,
    attention with the dequantisation fused, in stream order."""
    # kernel.py:294-307: scales, then the constants from them (one kernel)
    scales, params, finish = _hip_scales(query, key, value,
                                         (scale, query.shape[2], query.shape[-1], attn_mask is not None))
    q8, k8, v8 = finish()                                       # kernel.py:309-311
    return forward_codes(q8, k8, v8, scales, attn_mask, scale, return_mode, params=params)


def forward_codes(q8: Tensor, k8: Tensor, v8: Tensor, scales: Tensor, attn_mask: Tensor | None, scale: float,
                  return_mode: str = 'output', params: Tensor | None = None):
    """The device forward from int8 codes and their device scales (q_scale,
    k_scale, o_scale, q_scale * k_scale, as quantize_qkv returns them):
    constants, bias, attention with the dequantisation fused (kernel.py:297-351).
    `scale` is the host's (scale or 1/sqrt(D)) * LOG2E; `params`: the constants
    already queued for these scales (device_constants), or None."""
    Z, H, N = q8.shape[0], q8.shape[1], q8.shape[2]
    if params is None:
        params = device_constants(scales, scale, N, q8.shape[-1], attn_mask is not None)  # kernel.py:297-307
    check = _status_check(params)
    bias = None if attn_mask is None else mask_to_bias_planned(attn_mask, params, Z, H, N)  # kernel.py:327-336
    if return_mode == 'latency':  # the kernel alone, int8 codes out (kernel.py:348-349)
        check()
        o = torch.empty_like(v8)
        return bench_latency_ms(lambda: launch_forward_planned(q8, k8, v8, o, params, bias), device=q8.device)
    out = torch.empty_like(v8, dtype=scales.dtype)              # o * o_scale fused (kernel.py:351)
    launch_forward_planned(q8, k8, v8, out, params, bias, o_scale=scales[2])
    check()
    return out


def int8_weights(weight: Tensor) -> tuple[Tensor, Tensor]:
    """Per-output-channel int8 codes of a projection weight (Nc x K) for
    qkv_int8: w_scale = amax|W[c, :]| / 127 in fp32 (1 for all-zero rows) and
    w8 = clamp(rint(W / w_scale), -128, 127)."""
    w = weight.detach().to(torch.float32)
    w_scale = w.abs().amax(dim=1) / INT8_MAX
    w_scale = torch.where(w_scale > 0, w_scale, torch.ones_like(w_scale))
    w8 = torch.clamp(torch.round(w / w_scale[:, None]), -128, 127).to(torch.int8)
    return w8.contiguous(), w_scale.contiguous()


def qkv_int8(x: Tensor, w8: Tensor, w_scale: Tensor, bias: Tensor | None, num_heads: int):
    """The int8 QKV projection fused with the quantiser (qflash_hip_qkv_int8).

    x: (B, N, C) fp32 activations on the device; w8 / w_scale from int8_weights
    of the (3C, C) qkv weight; bias: (3C,) fp32 or None.  The activations are
    quantised per tensor (quantize_qkv's arithmetic), the projection runs on
    int8 MFMA, and its q, k, v thirds come back as int8 codes with their
    per-tensor scales, exactly as quantize_qkv would quantise a materialised
    fp32 projection y = RN(RN(fp32(x8 . w8^T) * RN(x_scale * w_scale)) + bias).
    Returns (q8, k8, v8, scales): (B, H, N, D) token-major views of one
    (B, N, 3, H, D) code buffer, and the 4 fp32 scales."""
    B, N, C = x.shape
    if x.dtype != torch.float32 or not x.is_cuda:
        raise ValueError("qkv_int8: fp32 activations on a GPU device")
    M = B * N
    x4 = x.reshape(1, 1, M, C)
    one = x4.reshape(-1)[:1].view(1, 1, 1, 1)  # stand-ins for the key / value slots of the quantiser
    x_scales, finish = quantize_qkv(x4, one, one)
    x8 = finish()[0]
    ws = _scales_workspace(x.device)
    scales = torch.empty(4, dtype=torch.float32, device=x.device)
    codes = torch.empty((B, N, 3, num_heads, C // num_heads), dtype=torch.int8, device=x.device)
    L = _lib.load()
    vp = ctypes.c_void_p
    rc = L.qflash_hip_qkv_int8(vp(x8.data_ptr()), vp(w8.data_ptr()), vp(w_scale.data_ptr()),
                               vp(0 if bias is None else bias.data_ptr()), vp(x_scales.data_ptr()), M, C, 3 * C,
                               vp(scales.data_ptr()), vp(codes.data_ptr()), vp(ws.data_ptr()), ws.numel(),
                               _stream_ptr(x))
    if rc != 0:
        _drop_scales_workspace(x.device)
    _lib.check(rc, "qflash_hip_qkv_int8")
    q8, k8, v8 = codes.permute(2, 0, 3, 1, 4).unbind(0)
    return q8, k8, v8, scales


def qflash_forward_window(query: Tensor, key: Tensor, value: Tensor, rel_bias: Tensor, mask: Tensor | None = None,
                          scale: float | None = None) -> Tensor:
    """QWindowAttention's attention call without the materialised mask.

    Equal, code for code, to ``qflash_forward(query, key, value, attn_mask=M)``
    with ``M = rel_bias + mask.view(1, nW, 1, N, N).expand(Z // nW, -1, H, -1, -1)
    .reshape(-1, H, N, N)`` (qflash/attention.py:68-74): every element of M is
    the fp32 sum rel_bias[0, h, i, j] + mask[z % nW, i, j], so the int32 bias
    is computed on the (nW, H, N, N) distinct sums only and the kernel reads
    slice z % nW.  rel_bias: (1, H, N, N); mask: (nW, N, N) or None.
    """
    d_q, d_k, d_v = query.shape[-1], key.shape[-1], value.shape[-1]
    assert d_q == d_k and d_k == d_v
    assert d_k in {16, 32, 64, 128, 256}
    if scale is None:
        scale = 1.0 / (d_q ** 0.5)
    scale = scale * LOG2E
    Z, H, N = query.shape[0], query.shape[1], query.shape[2]
    tables_fp32 = rel_bias.dtype == torch.float32 and rel_bias.is_cuda and (
        mask is None or (mask.dtype == torch.float32 and mask.is_cuda))
    if tables_fp32 and _device_path(query, key, value, None):
        if mask is not None and Z % mask.shape[0]:
            raise ValueError(f"batch {Z} is not a multiple of the {mask.shape[0]} windows of the mask")
        scales, params, finish = _hip_scales(query, key, value, (scale, N, d_q, True))
        wb = window_bias_planned(rel_bias, mask, params)
        q8, k8, v8 = finish()
        check = _status_check(params)
        bias, zmod = (wb.expand(Z, H, N, N), 0) if mask is None else (wb, mask.shape[0])
        out = torch.empty_like(v8, dtype=scales.dtype)
        launch_forward_planned(q8, k8, v8, out, params, bias, zmod, o_scale=scales[2])
        check()
        return out
    scales, finish = quantize_qkv(query, key, value)
    o_scale = scales[2]
    qk_scale = _scalar_to_host(scales[3])
    q8, k8, v8 = finish()
    sm_scale = scale * qk_scale()
    consts = fixed_point_constants(sm_scale)
    o = torch.empty_like(v8)
    Z, H, N = q8.shape[0], q8.shape[1], q8.shape[2]
    flag_kw = dict(EXP_USE_SHIFT=EXP_USE_SHIFT, L_USE_SHIFT=L_USE_SHIFT, ACC_USE_SHIFT=ACC_USE_SHIFT,
                   L_SHIFT=L_SHIFT, ACC_SHIFT=ACC_SHIFT)
    if mask is None:
        bias, zmod = window_bias(rel_bias, None, sm_scale).expand(Z, H, N, N), 0
    else:
        n_win = mask.shape[0]
        if Z % n_win:
            raise ValueError(f"batch {Z} is not a multiple of the {n_win} windows of the mask")
        bias, zmod = window_bias(rel_bias, mask, sm_scale), n_win
    if o_scale.dtype in _DT_CODE:  # o * o_scale fused into the kernel's stores
        out = torch.empty_like(v8, dtype=o_scale.dtype)
        launch_forward(q8, k8, v8, out, consts, flag_kw, bias, zmod, o_scale=o_scale)
        return out
    launch_forward(q8, k8, v8, o, consts, flag_kw, bias, zmod)
    return o * o_scale


class qflash:
    """Op namespace of the reference (kernel.py:354-356)."""

    kernel = [qflash_kernel, qflash_masked_kernel]
    forward = qflash_forward
