"""Build ``lib/liblwl_bfht.so`` from ``csrc/`` with hipcc for gfx950.

Usage: ``python -m latent_weight_lab_amd.build`` (also called by
``__graft_entry__.build()``).  Objects compile in parallel; the library is
written to a temporary name and renamed, so a reader never sees half a file.

``python -m latent_weight_lab_amd.build --sanitize`` builds a second library,
``lib/sanitize/liblwl_bfht.so``, whose host code (validators, planners, the
C ABI) carries AddressSanitizer and UndefinedBehaviorSanitizer; device code is
compiled as usual.  It is for the CPU test suite only, never for kernels:

    LD_PRELOAD=<clang>/lib/linux/libclang_rt.asan-x86_64.so ASAN_OPTIONS=detect_leaks=0 \
    LWL_BFHT_LIBRARY=latent_weight_lab_amd/lib/sanitize/liblwl_bfht.so python -m pytest tests -m "not gpu"
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


# Host-only sanitizers (each flag behind -Xarch_host, so no device code is built with them).
SANITIZE_FLAGS = ["-O1", "-g", "-Xarch_host", "-fno-omit-frame-pointer",
                  "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                  "-Xarch_host", "-fno-sanitize-recover=undefined"]


def _compile(src: Path, obj_dir: Path = OBJ_DIR, sanitize: bool = False) -> Path:
    obj = obj_dir / (src.name + ".o")
    flags = COMMON_FLAGS + (DEVICE_FLAGS if src.suffix == ".hip" else [])
    if sanitize:
        flags = [f for f in flags if f != "-O3"] + SANITIZE_FLAGS
    cmd = [hipcc(), *flags, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = False, sanitize: bool = False) -> Path:
    out_dir = OUT_DIR / "sanitize" if sanitize else OUT_DIR
    obj_dir = out_dir / "obj"
    lib = out_dir / LIB.name
    obj_dir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objs = list(pool.map(lambda s: _compile(s, obj_dir, sanitize), srcs))
    tmp = lib.with_suffix(".so.tmp")
    link = ["-shared-libasan", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined"] if sanitize else []
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *link, "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


if __name__ == "__main__":
    build(verbose=True, sanitize="--sanitize" in sys.argv[1:])
    sys.exit(0)
