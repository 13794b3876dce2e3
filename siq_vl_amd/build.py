"""Builds ``libsiq_kernels.so`` (gfx950) in-tree with hipcc.

The library is the C-ABI declared in ``include/siq_kernels.h``; every source
under ``siq_vl_amd/csrc`` is compiled for gfx950 only and linked into one
shared object next to this file, so it travels with the repository.
"""

from __future__ import annotations

import concurrent.futures as _cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
REPO = PKG_DIR.parent
LIB_NAME = "libsiq_kernels.so"
LIB_PATH = PKG_DIR / LIB_NAME
OBJ_DIR = PKG_DIR / "_build"

ARCH = "gfx950"
# Packed-FP32 instructions are disabled for every device compile: only scalar
# and float2 fp32 code is emitted.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-Wall", "-Wno-unused-function",
                f"-I{REPO / 'include'}"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the SiQ-VL MI355X kernels need the ROCm toolchain to build")


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


# MFMA results in VGPRs instead of AGPRs for the attention kernels: their
# score / dP accumulators feed VALU softmax code every step, and the AGPR form
# made the register allocator shuttle values between the two files.
PER_FILE_FLAGS = {
    "attn_fwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "attn_bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.name + ".o")
    cmd = [_hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, *PER_FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compiles every source and links the shared library; returns its path."""
    OBJ_DIR.mkdir(exist_ok=True)
    srcs = sources()
    with _cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
