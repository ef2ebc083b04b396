"""The C ABI (include/qflash_hip.h) on the CPU: the built library loads, exports
every function the header declares, and rejects bad arguments with the
documented codes before it touches the GPU (no kernel is launched here)."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest
import torch

from qflash_amd import _build, _lib

# Fake device addresses are passed below to calls that must reject them before
# any launch; on a machine with a GPU a regression in that checking would
# launch kernels on them, so the module runs on GPU-less hosts only.
pytestmark = pytest.mark.skipif(torch.cuda.is_available(), reason="CPU-only checks of the C ABI")

HEADER = os.path.join(_build.ROOT, "include", "qflash_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qflash_hip_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_build.LIB_PATH):
        pytest.fail(f"{_build.LIB_PATH} is not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_declares_the_entry_points():
    assert _declared() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", _build.LIB_PATH], capture_output=True, text=True,
                        check=True).stdout
    exported = set(re.findall(r"\sT\s(\w+)$", nm, flags=re.M))
    assert set(_declared()) <= exported


def test_version_string(lib):
    assert b"gfx950" in lib.qflash_hip_version()


def _call(lib, masked=False, Q=1, D=64, Z=1, H=1, N=32, rs=100, strides=True, flags=None, bias=1):
    """Call an entry point with fake non-null pointers: only the host-side checks run."""
    st = (ctypes.c_int64 * 20)(*([0] * 20)) if strides else None
    p = ctypes.c_void_p(Q) if Q else None
    fake = ctypes.c_void_p(64)
    fl = ctypes.byref(flags) if flags is not None else None
    if masked:
        b = ctypes.c_void_p(bias) if bias else None
        return lib.qflash_hip_masked_kernel(p, fake, fake, fake, b, rs, -1, 1, 1, 1, st, Z, H, N, D, fl, None)
    return lib.qflash_hip_kernel(p, fake, fake, fake, rs, -1, 1, 1, 1, st, Z, H, N, D, fl, None)


@pytest.mark.parametrize("masked", [False, True])
def test_invalid_arguments_return_codes_and_messages(lib, masked):
    assert _call(lib, masked, Q=0) == -1
    assert b"null pointer" in lib.qflash_hip_last_error()
    assert _call(lib, masked, strides=False) == -1
    assert _call(lib, masked, Z=0) == -1
    assert b"bad shape" in lib.qflash_hip_last_error()
    assert _call(lib, masked, N=-3) == -1
    assert _call(lib, masked, rs=0) == -1
    assert b"sm_rscale" in lib.qflash_hip_last_error()
    assert _call(lib, masked, D=16) == -2
    assert b"BLOCK_N" in lib.qflash_hip_last_error()
    assert _call(lib, masked, D=48) == -2
    bad = _lib.Flags(1, 1, 1, 0, 30)
    assert _call(lib, masked, flags=bad) == -1
    assert b"l_shift" in lib.qflash_hip_last_error()
    bad = _lib.Flags(1, 1, 1, 30, 63)
    assert _call(lib, masked, flags=bad) == -1
    assert b"acc_shift" in lib.qflash_hip_last_error()


def test_masked_entry_needs_a_bias(lib):
    assert _call(lib, masked=True, bias=0) == -1
    assert b"attn_bias" in lib.qflash_hip_last_error()


def test_window_entry_checks_its_period(lib):
    st = (ctypes.c_int64 * 20)(*([0] * 20))
    fake = ctypes.c_void_p(64)
    rc = lib.qflash_hip_window_kernel(fake, fake, fake, fake, fake, 100, -1, 1, 1, 1, st, 4, 1, 49, 32, 0, None,
                                      None)
    assert rc == -1 and b"bias_zmod" in lib.qflash_hip_last_error()
    rc = lib.qflash_hip_window_kernel(fake, fake, fake, fake, None, 100, -1, 1, 1, 1, st, 4, 1, 49, 32, 2, None, None)
    assert rc == -1 and b"attn_bias" in lib.qflash_hip_last_error()
    rc = lib.qflash_hip_window_kernel(fake, fake, fake, fake, fake, 100, -1, 1, 1, 1, st, 4, 1, 49, 16, 2, None, None)
    assert rc == -2


def test_layout_check_rejects_null(lib):
    assert lib.qflash_hip_mfma_layout_check(None, None, None, None) == -1


def test_error_codes_map_to_python_exceptions(lib):
    _call(lib, D=16)
    with pytest.raises(_lib.QFlashCompilationError, match="BLOCK_N"):
        _lib.check(-2, "qflash_kernel")
    _call(lib, Z=0)
    with pytest.raises(_lib.QFlashLibraryError, match="bad shape"):
        _lib.check(-1, "qflash_kernel")
    _lib.check(0, "ok")


def test_header_compiles_as_c_and_cxx(tmp_path):
    src = tmp_path / "use.c"
    src.write_text('#include "qflash_hip.h"\nint main(void){qflash_hip_flags f={1,1,1,30,30};'
                   'return f.l_shift==30 && sizeof(qflash_hip_flags)==20 ? 0 : 1;}\n')
    inc = os.path.dirname(HEADER)
    for cc in (["gcc", "-std=c99"], ["g++", "-x", "c++", "-std=c++17"]):
        exe = tmp_path / ("a_" + cc[0])
        subprocess.run([*cc, "-Wall", "-Werror", "-I", inc, str(src), "-o", str(exe)], check=True)
        subprocess.run([str(exe)], check=True)


def test_forward_entry_checks_output_and_bias(lib):
    st = (ctypes.c_int64 * 20)(*([0] * 20))
    fake = ctypes.c_void_p(64)
    args = [100, -1, 1, 1, 1, st, 1, 1, 32, 64, None, None]
    # unknown output dtype; dequantised output without o_scale; bias period without a bias
    assert lib.qflash_hip_forward(fake, fake, fake, fake, 7, fake, None, 0, *args) == -1
    assert b"output dtype" in lib.qflash_hip_last_error()
    assert lib.qflash_hip_forward(fake, fake, fake, fake, _lib.F16, None, None, 0, *args) == -1
    assert b"o_scale" in lib.qflash_hip_last_error()
    assert lib.qflash_hip_forward(fake, fake, fake, fake, _lib.I8, None, None, 4, *args) == -1
    assert b"bias_zmod" in lib.qflash_hip_last_error()
    args[9] = 16
    assert lib.qflash_hip_forward(fake, fake, fake, fake, _lib.I8, None, None, 0, *args) == -2


def test_quantiser_entries_check_arguments(lib):
    geo = (ctypes.c_int64 * 24)(*([1, 1, 4, 32, 128, 128, 32, 1] * 3))
    fake = ctypes.c_void_p(64)
    ws = ctypes.c_void_p(64)
    assert lib.qflash_hip_scales(fake, fake, fake, 9, geo, fake, ws, _lib.SCALES_WORKSPACE, None) == -1
    assert b"dtype" in lib.qflash_hip_last_error()
    assert lib.qflash_hip_scales(fake, fake, fake, _lib.F32, geo, fake, ws, 3, None) == -1
    assert b"workspace" in lib.qflash_hip_last_error()
    bad = (ctypes.c_int64 * 24)(*([1, 1, 0, 32, 128, 128, 32, 1] * 3))
    assert lib.qflash_hip_scales(fake, fake, fake, _lib.F32, bad, fake, ws, _lib.SCALES_WORKSPACE, None) == -1
    assert b"empty" in lib.qflash_hip_last_error()
    ost = (ctypes.c_int64 * 12)(*([128, 128, 32, 1] * 3))
    assert lib.qflash_hip_quantize(fake, fake, fake, _lib.F32, geo, None, fake, fake, ost, fake, None) == -1
    assert b"null" in lib.qflash_hip_last_error()
    # the scales and constants entry checks both halves' arguments before any launch
    fl = _lib.Flags(1, 1, 1, 30, 30)
    params = ctypes.c_void_p(64)
    assert lib.qflash_hip_scales_constants(fake, fake, fake, _lib.F32, geo, None, ws, _lib.SCALES_WORKSPACE, 0.18,
                                           32, 32, 0, ctypes.byref(fl), params, None) == -1
    assert b"null" in lib.qflash_hip_last_error()
    assert lib.qflash_hip_scales_constants(fake, fake, fake, _lib.F32, geo, fake, ws, _lib.SCALES_WORKSPACE, 0.18,
                                           0, 32, 0, ctypes.byref(fl), params, None) == -1
    assert b"N_CTX" in lib.qflash_hip_last_error()
    assert lib.qflash_hip_scales_constants(fake, fake, fake, _lib.F32, geo, fake, ws, 3, 0.18, 32, 32, 0,
                                           ctypes.byref(fl), params, None) == -1
    assert b"workspace" in lib.qflash_hip_last_error()
    bad_fl = _lib.Flags(1, 1, 1, 0, 30)
    assert lib.qflash_hip_scales_constants(fake, fake, fake, _lib.F32, geo, fake, ws, _lib.SCALES_WORKSPACE, 0.18,
                                           32, 32, 0, ctypes.byref(bad_fl), params, None) == -1
    assert b"l_shift" in lib.qflash_hip_last_error()


def test_bias_entries_check_arguments(lib):
    fake = ctypes.c_void_p(64)
    assert lib.qflash_hip_window_bias(None, fake, 4, 3, 49, 0.25, fake, None) == -1
    assert b"null" in lib.qflash_hip_last_error()
    assert lib.qflash_hip_window_bias(fake, None, 4, 3, 49, 0.25, fake, None) == -1
    assert b"nW must be 1" in lib.qflash_hip_last_error()
    assert lib.qflash_hip_window_bias(fake, fake, 4, 0, 49, 0.25, fake, None) == -1
    assert b"shape" in lib.qflash_hip_last_error()
    assert lib.qflash_hip_window_bias(fake, fake, 4, 3, 49, 0.0, fake, None) == -1
    assert b"sm_scale" in lib.qflash_hip_last_error()
    assert lib.qflash_hip_window_bias(fake, fake, 1 << 20, 64, 64, 0.25, fake, None) == -1
    assert b"too large" in lib.qflash_hip_last_error()
    assert lib.qflash_hip_mask_bias(fake, 0, 0.25, fake, None) == -1
    assert b"size" in lib.qflash_hip_last_error()
    assert lib.qflash_hip_mask_bias(fake, 100, float("nan"), fake, None) == -1
    assert b"sm_scale" in lib.qflash_hip_last_error()
    assert lib.qflash_hip_mask_bias(None, 100, 0.25, fake, None) == -1
    assert b"null" in lib.qflash_hip_last_error()
