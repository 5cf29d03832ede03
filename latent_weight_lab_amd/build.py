"""Build ``lib/liblwl_bfht.so`` from ``csrc/`` with hipcc for gfx950.

Usage: ``python -m latent_weight_lab_amd.build`` (also called by
``__graft_entry__.build()``).  Objects compile in parallel; the library is
written to a temporary name and renamed, so a reader never sees half a file.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
OUT_DIR = PKG / "lib"
OBJ_DIR = OUT_DIR / "obj"
LIB = OUT_DIR / "liblwl_bfht.so"

ARCH = "gfx950"
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall", f"-I{INCLUDE}"]
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    # Packed fp32 VALU ops (v_pk_*_f32) stay off: the kernels use scalar fp32 VALU.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in VGPRs (the VALU reads them directly; AGPRs would
    # need a v_accvgpr_read per value)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build latent_weight_lab_amd)")
    return path


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.name + ".o")
    flags = COMMON_FLAGS + (DEVICE_FLAGS if src.suffix == ".hip" else [])
    cmd = [hipcc(), *flags, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
