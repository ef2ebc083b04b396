"""ctypes binding of libqflash_hip.so (declared in include/qflash_hip.h).

The product path has no fallback: if the library is missing or a call
fails, an exception is raised.
"""
from __future__ import annotations

import ctypes
import os
import threading

from ._build import LIB_PATH


class QFlashLibraryError(RuntimeError):
    """The HIP library is missing, failed to load, or rejected a call."""


class QFlashCompilationError(QFlashLibraryError):
    """HEAD_DIM the kernels cannot be built for.

    The reference fails at Triton compile time for HEAD_DIM=16
    (tl.static_assert(BLOCK_N <= HEAD_DIM), qflash/kernel.py:105,204).
    """


class Flags(ctypes.Structure):
    _fields_ = [("exp_use_shift", ctypes.c_int32), ("l_use_shift", ctypes.c_int32),
                ("acc_use_shift", ctypes.c_int32), ("l_shift", ctypes.c_int32),
                ("acc_shift", ctypes.c_int32)]


EXPORTS = ("qflash_hip_kernel", "qflash_hip_masked_kernel", "qflash_hip_window_kernel", "qflash_hip_forward",
           "qflash_hip_scales", "qflash_hip_scales_noalloc", "qflash_hip_qkv_int8",
           "qflash_hip_quantize", "qflash_hip_window_bias", "qflash_hip_mask_bias", "qflash_hip_constants",
           "qflash_hip_scales_constants",
           "qflash_hip_forward_planned", "qflash_hip_window_bias_planned", "qflash_hip_mask_bias_planned",
           "qflash_hip_last_error",
           "qflash_hip_mfma_layout_check", "qflash_hip_lut_bounds", "qflash_hip_far_bounds",
           "qflash_hip_set_test_hooks", "qflash_hip_version")

# test-hook bits of qflash_hip_set_test_hooks (include/qflash_hip.h)
HOOKS = {"FORCE_GENERAL": 1, "FORCE_DYNAMIC_BOUND": 2, "FORCE_ROBUST": 4, "NO_LUT": 8, "FORCE_LUT": 16}

# element type codes of qflash_hip_scales / qflash_hip_quantize, and its workspace
F32, F16, BF16, I8 = 0, 1, 2, 3
SCALES_WORKSPACE = 256
# device parameter block of qflash_hip_constants and its status codes
PARAMS_WORDS = 20
STATUS_ZERODIV_SCALE, STATUS_NAN, STATUS_INF, STATUS_ZERODIV_RSCALE, STATUS_RANGE = 1, 2, 3, 4, 5

E_HEADDIM = -2

_lock = threading.Lock()
_lib = None


def _declare(L):
    vp, i32, i64p = ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(ctypes.c_int64)
    fp = ctypes.POINTER(Flags)
    L.qflash_hip_kernel.restype = ctypes.c_int
    L.qflash_hip_kernel.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i64p, i32, i32, i32, i32, fp, vp]
    L.qflash_hip_masked_kernel.restype = ctypes.c_int
    L.qflash_hip_masked_kernel.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i64p, i32, i32, i32, i32,
                                           fp, vp]
    L.qflash_hip_window_kernel.restype = ctypes.c_int
    L.qflash_hip_window_kernel.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i64p, i32, i32, i32, i32, i32,
                                           fp, vp]
    L.qflash_hip_scales.restype = ctypes.c_int
    L.qflash_hip_scales.argtypes = [vp, vp, vp, i32, i64p, vp, vp, ctypes.c_int64, vp]
    L.qflash_hip_qkv_int8.restype = ctypes.c_int
    L.qflash_hip_qkv_int8.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, vp, vp, vp, ctypes.c_int64, vp]
    L.qflash_hip_scales_noalloc.restype = ctypes.c_int
    L.qflash_hip_scales_noalloc.argtypes = [vp, vp, vp, i32, i64p, vp, vp]
    L.qflash_hip_quantize.restype = ctypes.c_int
    L.qflash_hip_quantize.argtypes = [vp, vp, vp, i32, i64p, vp, vp, vp, i64p, vp, vp]
    L.qflash_hip_window_bias.restype = ctypes.c_int
    L.qflash_hip_window_bias.argtypes = [vp, vp, i32, i32, i32, ctypes.c_double, vp, vp]
    L.qflash_hip_mask_bias.restype = ctypes.c_int
    L.qflash_hip_mask_bias.argtypes = [vp, ctypes.c_int64, ctypes.c_double, vp, vp]
    L.qflash_hip_constants.restype = ctypes.c_int
    L.qflash_hip_constants.argtypes = [vp, i32, ctypes.c_double, i32, i32, i32, fp, vp, vp]
    L.qflash_hip_scales_constants.restype = ctypes.c_int
    L.qflash_hip_scales_constants.argtypes = [vp, vp, vp, i32, i64p, vp, vp, ctypes.c_int64, ctypes.c_double, i32, i32,
                                              i32, fp, vp, vp]
    L.qflash_hip_forward_planned.restype = ctypes.c_int
    L.qflash_hip_forward_planned.argtypes = [vp, vp, vp, vp, i32, vp, vp, i32, vp, i64p, i32, i32, i32, i32, fp, vp]
    L.qflash_hip_window_bias_planned.restype = ctypes.c_int
    L.qflash_hip_window_bias_planned.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp]
    L.qflash_hip_mask_bias_planned.restype = ctypes.c_int
    L.qflash_hip_mask_bias_planned.argtypes = [vp, ctypes.c_int64, vp, vp, vp]
    L.qflash_hip_forward.restype = ctypes.c_int
    L.qflash_hip_forward.argtypes = [vp, vp, vp, vp, i32, vp, vp, i32, i32, i32, i32, i32, i32, i64p, i32, i32, i32,
                                     i32, fp, vp]
    L.qflash_hip_last_error.restype = ctypes.c_char_p
    L.qflash_hip_last_error.argtypes = []
    L.qflash_hip_mfma_layout_check.restype = ctypes.c_int
    L.qflash_hip_mfma_layout_check.argtypes = [vp, vp, vp, vp]
    L.qflash_hip_lut_bounds.restype = ctypes.c_int
    L.qflash_hip_lut_bounds.argtypes = [i32, i32, i32, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]
    L.qflash_hip_far_bounds.restype = ctypes.c_int
    L.qflash_hip_far_bounds.argtypes = [i32, i32, i32] + [ctypes.POINTER(ctypes.c_int32)] * 3
    L.qflash_hip_set_test_hooks.restype = ctypes.c_uint32
    L.qflash_hip_set_test_hooks.argtypes = [ctypes.c_uint32]
    L.qflash_hip_version.restype = ctypes.c_char_p
    L.qflash_hip_version.argtypes = []


def load(path: str | None = None):
    """Load (once) and return the library; raise if it is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = path or os.environ.get("QFLASH_HIP_LIB", LIB_PATH)
        if not os.path.exists(path):
            raise QFlashLibraryError(
                f"{path} is not built: run `python -m qflash_amd._build` (or __graft_entry__.build()) first")
        try:
            L = ctypes.CDLL(path)
        except OSError as e:  # pragma: no cover - depends on the box
            raise QFlashLibraryError(f"cannot load {path}: {e}") from e
        missing = [s for s in EXPORTS if not hasattr(L, s)]
        if missing:
            raise QFlashLibraryError(f"{path} lacks exports {missing}")
        _declare(L)
        _lib = L
        return L


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().qflash_hip_last_error().decode(errors="replace")
        cls = QFlashCompilationError if rc == E_HEADDIM else QFlashLibraryError
        raise cls(f"{what} failed ({rc}): {msg}")


def set_test_hooks(*names: str) -> int:
    """Set the library's test hooks to exactly `names` (keys of HOOKS); returns
    the previous bits.  Tests only: each hook forces an exact fallback path."""
    bits = 0
    for n in names:
        bits |= HOOKS[n]
    return int(load().qflash_hip_set_test_hooks(bits))
