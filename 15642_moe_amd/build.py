"""Compile the HIP sources into the in-tree C-ABI library (gfx950 only).

    python -m <package>.build          (or call build_library())

Each translation unit is compiled with hipcc in parallel, then linked into
``lib15642_moe_fp8.so`` next to this file.  The packed-FP32 VALU ops are
disabled for all device code.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_NAME = "lib15642_moe_fp8.so"
LIB_PATH = PKG_DIR / LIB_NAME
SOURCES = ["route.hip", "pack.hip", "gemm.hip", "prefill.hip", "upstream.hip", "capi.hip"]
ARCH = "gfx950"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


def compile_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Wno-unused-result",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # MFMA results in VGPRs: the per-K-block scale FMAs read them directly
        # instead of through v_accvgpr_read copies.
        "-mllvm", "-amdgpu-mfma-vgpr-form=1",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
    ]


def build_library(verbose: bool = False) -> Path:
    hipcc = _hipcc()
    obj_dir = PKG_DIR / "_build"
    obj_dir.mkdir(exist_ok=True)
    flags = compile_flags()

    def compile_one(src: str) -> Path:
        obj = obj_dir / (Path(src).stem + ".o")
        cmd = [hipcc, *flags, "-c", str(CSRC / src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        noise = "packed-fp32-ops"  # host pass warns about the device-only feature
        err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{err}")
        if verbose and err.strip():
            print(err, file=sys.stderr)
        return obj

    with cf.ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose=True))
