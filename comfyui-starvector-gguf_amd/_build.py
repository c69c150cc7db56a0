"""Compile libsvq.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

Each .hip source under csrc/ becomes an object in _obj/ (compiled in
parallel; the host-only .cpp sources with the host C++ compiler), then the
objects are linked into libsvq.so next to this file. The
library is always rebuilt when this runs; callers that only need it loaded use
`_native.load()`.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
OBJ_DIR = PKG_DIR / "_obj"
LIB_PATH = PKG_DIR / "libsvq.so"
INCLUDE_DIR = PKG_DIR.parent / "include"

ARCH = "gfx950"
# Packed FP32 instructions are disabled for all device code: hipcc would
# otherwise form v_pk_{add,mul,fma}_f32 from ordinary float code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
                "-Wall", "-Wno-unused-function", f"-I{INCLUDE_DIR}"]


def hipcc() -> str:
    path = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError(f"hipcc not found (looked for {path})")
    return path


HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-pthread", "-Wall", f"-I{INCLUDE_DIR}"]


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    if src.suffix == ".cpp":  # host-only code (the GGUF reader)
        cmd = [os.environ.get("CXX") or "g++", *HOST_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj


def build_library(jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libsvq.so; returns its path."""
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    OBJ_DIR.mkdir(exist_ok=True)
    workers = jobs or min(len(sources), os.cpu_count() or 1, 8)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", "-o", str(tmp),
           *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of libsvq.so failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


# The timeline build (libsvq_timeline.so): the units holding the streaming
# MFMA kernel and the C ABI recompiled with SVQ_TIMELINE, linked with the other
# objects of the product build. The kernel then writes per-wave phase stamps
# when svq_timeline_stamps has set a buffer; libsvq.so carries no stamp code.
TIMELINE_LIB = PKG_DIR / "libsvq_timeline.so"
TIMELINE_OBJ_DIR = PKG_DIR / "_obj_timeline"
TIMELINE_UNITS = ("svq_api", "svq_gemv_mfma4", "svq_gemv_mfma4_wide")


def _compile_timeline(src: Path) -> Path:
    obj = TIMELINE_OBJ_DIR / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *DEVICE_FLAGS, "-DSVQ_TIMELINE=1", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc (timeline) failed for {src.name}:\n{proc.stderr}")
    return obj


def build_timeline_library(jobs: int | None = None) -> Path:
    """Link libsvq_timeline.so (after build_library, whose objects it reuses)."""
    TIMELINE_OBJ_DIR.mkdir(exist_ok=True)
    units = [CSRC / f"{u}.hip" for u in TIMELINE_UNITS]
    with ThreadPoolExecutor(max_workers=jobs or len(units)) as pool:
        objects = list(pool.map(_compile_timeline, units))
    objects += [o for o in sorted(OBJ_DIR.glob("*.o")) if o.stem not in TIMELINE_UNITS]
    tmp = TIMELINE_LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", "-o", str(tmp),
           *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of libsvq_timeline.so failed:\n{proc.stderr}")
    os.replace(tmp, TIMELINE_LIB)
    return TIMELINE_LIB


if __name__ == "__main__":
    print(build_library())
    print(build_timeline_library())
