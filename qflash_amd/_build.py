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
CSRC = os.path.join(HERE, "csrc")
SOURCES = [os.path.join(CSRC, "qflash_fwd.hip"), os.path.join(CSRC, "qflash_quant.hip"),
           os.path.join(CSRC, "qflash_fwd_inst.hip")]
HEADERS = [os.path.join(ROOT, "include", "qflash_hip.h"), os.path.join(CSRC, "qf_common.h"),
           os.path.join(CSRC, "qf_fwd.h")]
LIB_PATH = os.path.join(HERE, "libqflash_hip.so")
OBJ_DIR = os.path.join(HERE, "_build")
ARCH = "gfx950"
# qflash_fwd_inst.hip is compiled once per (head dim, masked) pair: the kernel
# instantiations of the pairs build in parallel
INST = [(d, m) for d in (32, 64, 128, 256) for m in (0, 1)]

# -packed-fp32-ops is disabled for all device code (some packed fp32 forms
# are unreliable on the target pool); the host pass warns that it does not
# know the feature, which is harmless.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC",
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


def _units():
    """(object path, compile command) of every translation unit."""
    cc = hipcc()
    units = []
    for src in SOURCES[:2]:
        obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
        units.append((obj, [cc, *HIPCC_FLAGS, "-c", "-o", obj, src]))
    for d, m in INST:
        obj = os.path.join(OBJ_DIR, f"qflash_fwd_inst_d{d}_m{m}.o")
        units.append((obj, [cc, *HIPCC_FLAGS, f"-DQF_INST_D={d}", f"-DQF_INST_MASKED={m}", "-c", "-o", obj,
                            SOURCES[2]]))
    return units


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build(force: bool = True, verbose: bool = False, jobs: int | None = None) -> str:
    """Compile libqflash_hip.so for gfx950 (always when force=True): every
    translation unit to an object in parallel, then one link."""
    if not force and not stale():
        return LIB_PATH
    from concurrent.futures import ThreadPoolExecutor

    os.makedirs(OBJ_DIR, exist_ok=True)
    units = _units()
    jobs = jobs or max(1, min(len(units), os.cpu_count() or 1, 16))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_run, cmd, verbose) for _, cmd in units]:
            f.result()
    tmp = LIB_PATH + f".tmp{os.getpid()}"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *[o for o, _ in units]], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(force=True, verbose=True))
