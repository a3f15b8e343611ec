"""Builds the MI355X plugin library in-tree.

    python safetyraise-lmengine_amd/build.py     # -> safetyraise-lmengine_amd/libsafetyraise_mi355x.so

Device code (.hip) is compiled by hipcc for gfx950 only; host code (.cpp) is
plain C++17 against the HIP runtime headers.  Packed FP32 instructions are
disabled for device code (they are not trusted on this hardware pool).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libsafetyraise_mi355x.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

COMMON = ["-std=c++17", "-O3", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wextra",
          "-Wno-unused-parameter", f"-I{ROOT / 'include'}", f"-I{CSRC}"]
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _hipcc() -> str:
    found = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    return found


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    if src.suffix == ".hip":
        cmd = [_hipcc(), "-x", "hip", *COMMON, *DEVICE, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [_hipcc(), "-x", "c++", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", *COMMON,
               "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs), f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    try:
        build(verbose=True)
    except RuntimeError as exc:
        print(exc, file=sys.stderr)
        sys.exit(1)
