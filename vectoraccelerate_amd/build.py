"""Builds libva_hip.so (HIP for gfx950) in-tree.

Every ``csrc/*.hip`` file is compiled with hipcc for gfx950 only and linked into
``vectoraccelerate_amd/libva_hip.so``.  Objects go to ``vectoraccelerate_amd/_build/``.
Packed-fp32 instruction selection is disabled (``-packed-fp32-ops``): ordinary float code
is compiled to scalar v_fma_f32 / v_add_f32.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libva_hip.so"
INCLUDE = PKG.parent / "include"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
CXXFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-parameter",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *CXXFLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    # hipcc's host pass does not know the device-only feature; drop only that warning
    noise = "is not a recognized feature for this target"
    rest = [ln for ln in proc.stderr.splitlines() if noise not in ln and ln.strip()]
    if rest:
        sys.stderr.write("\n".join(rest) + "\n")
    return obj


def build(jobs: int | None = None) -> Path:
    """Compile every HIP source and link libva_hip.so.  Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build())


def build_cpp_example() -> Path:
    """Compile tests/cpp/example.cpp (the C++ host mirror's check program) against libva_hip.so."""
    root = PKG.parent
    src = root / "tests" / "cpp" / "example.cpp"
    out = root / "tests" / "cpp" / "va_example"
    cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", f"-I{root / 'include'}", str(src), f"-L{PKG}", "-lva_hip",
           "-Wl,-rpath,$ORIGIN/../../vectoraccelerate_amd", "-Wl,-rpath-link,/opt/rocm/lib", "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed for {src.name}:\n{proc.stdout}\n{proc.stderr}")
    return out
