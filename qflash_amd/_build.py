"""Build the gfx950 HIP library in-tree (qflash_amd/libqflash_hip.so).

The built .so is git-ignored but travels with the working tree, so the GPU
box loads exactly what was compiled here.
"""
from __future__ import annotations

import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = [os.path.join(HERE, "csrc", "qflash_fwd.hip"), os.path.join(HERE, "csrc", "qflash_quant.hip")]
HEADERS = [os.path.join(ROOT, "include", "qflash_hip.h"), os.path.join(HERE, "csrc", "qf_common.h")]
LIB_PATH = os.path.join(HERE, "libqflash_hip.so")
ARCH = "gfx950"

# -packed-fp32-ops is disabled for all device code (some packed fp32 forms
# are unreliable on the target pool); the host pass warns that it does not
# know the feature, which is harmless.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    # MFMA results in VGPRs: the kernels post-process every result with VALU ops
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
]


def hipcc() -> str:
    cand = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(cand):
        raise RuntimeError("hipcc not found; set HIPCC or install ROCm")
    return cand


def stale() -> bool:
    if not os.path.exists(LIB_PATH):
        return True
    t = os.path.getmtime(LIB_PATH)
    return any(os.path.getmtime(s) > t for s in SOURCES + HEADERS)


def build(force: bool = True, verbose: bool = False) -> str:
    """Compile libqflash_hip.so for gfx950 (always when force=True)."""
    if not force and not stale():
        return LIB_PATH
    tmp = LIB_PATH + f".tmp{os.getpid()}"
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", tmp, *SOURCES]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(force=True, verbose=True))
