"""Build the gfx950 C-ABI library ``ringmaster_amd/_lib/libringmaster_amd.so``.

Each ``csrc/*.hip`` translation unit is compiled by ``hipcc --offload-arch=gfx950``
into ``_build/`` (in parallel), then linked into one shared library. The library
is built in-tree so that it travels with the source tree; nothing is installed.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB_NAME = "libringmaster_amd.so"
LIB_PATH = OUT_DIR / LIB_NAME
BUILD_DIR = ROOT / "_build"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# Packed-FP32 VALU ops are disabled for every device pass: some of their forms have
# given wrong results on MI355X without any error.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-std=c++20", "-fPIC", f"--offload-arch={ARCH}", "-Wall",
                "-Wno-unused-function", "-Wno-unused-variable"]


# Per-unit device flags. attn_bwd_vf (the head-dim-64 and -128 backward): MFMAs write
# VGPRs (the S / dP tiles the VALU reads then need no v_accvgpr_read); the compiler's
# AGPR-copy rewrite still places the operands pinned to AGPRs there. The head-dim-256
# backward (attn_bwd) keeps the compiler's choice: its dK and dV accumulators fill the
# AGPRs, and there its dQ kernel measured 15% faster than with VGPR-form MFMAs.
# attn_fwd: VGPR-form MFMAs change only the head-dim-256 forward (59-65 AGPRs in use
# against 147; the 64 and 128 code is identical), whose configs[1]-shaped step measured
# 0.8% faster.
_VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
UNIT_FLAGS = {"attn_bwd_vf": _VGPR_FORM, "attn_fwd": _VGPR_FORM}


def _sources():
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *DEVICE_FLAGS, *UNIT_FLAGS.get(src.stem, []), "-I", str(CSRC),
           "-I", str(ROOT / "include"), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def build_library(jobs: int | None = None) -> Path:
    """Compile every HIP source for gfx950 and link the C-ABI library. Always rebuilds."""
    if not Path(HIPCC).exists() and shutil.which(HIPCC) is None:
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    OUT_DIR.mkdir(parents=True, exist_ok=True)
    srcs = _sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *[str(o) for o in objs]]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library())
