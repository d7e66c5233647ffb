"""Build the gfx950 library in-tree: deltafin_amd/lib/libk3hipmoe.so.

Kernels are compiled by hipcc for gfx950 only, with packed-FP32 instructions
disabled and the IEEE math flag set the reference uses for its HIP build
(native/deltafin-native-build/src/lib.rs:35-41).  Host translation units are
plain C++ compiled by g++ against the HIP runtime headers.

Usage:  python -m deltafin_amd.build        (always rebuilds)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libk3hipmoe.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-fast-math",
    "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-approx-transcendentals",
    "-ffp-contract=fast-honor-pragmas",
    "-mcode-object-version=5",
    "-Wall",
]
CXX_FLAGS = [
    "-O2",
    "-fPIC",
    "-std=c++17",
    "-D__HIP_PLATFORM_AMD__",
    f"-I{ROCM / 'include'}",
    f"-I{INCLUDE}",
    "-Wall",
    "-Wextra",
    "-Wno-unused-parameter",
]
KERNEL_SOURCES = ["k3_kernels.hip", "k3_verify_mfma.hip", "k3_spine.hip", "k3_spine_mfma.hip",
                  "k3_noalloc.hip"]
HOST_SOURCES = ["k3_abi.cpp", "k3_cache.cpp", "k3_timing.cpp", "k3_spine_abi.cpp"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines()
        if "is not a recognized feature for this target" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def build(verbose: bool = True, defines: list[str] | None = None, out: Path | None = None) -> Path:
    """Compile the library; `defines` (NAME=VALUE) override tuning constants in
    every translation unit and `out` redirects the library (both for tuning
    sweeps)."""
    hipcc = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    target = Path(out) if out is not None else LIB
    target.parent.mkdir(parents=True, exist_ok=True)
    dflags = [f"-D{d}" for d in (defines or [])]
    with tempfile.TemporaryDirectory(prefix="k3build_") as tmp:
        objs = []
        for src in KERNEL_SOURCES:
            obj = Path(tmp) / (src + ".o")
            _run([hipcc, *HIP_FLAGS, *dflags, f"-I{INCLUDE}", "-c", str(CSRC / src), "-o", str(obj)])
            objs.append(str(obj))
        for src in HOST_SOURCES:
            obj = Path(tmp) / (src + ".o")
            _run(["g++", *CXX_FLAGS, *dflags, "-c", str(CSRC / src), "-o", str(obj)])
            objs.append(str(obj))
        tmp_lib = Path(tmp) / LIB.name
        _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp_lib), *objs,
              f"-L{ROCM / 'lib'}", "-lamdhip64"])
        shutil.move(str(tmp_lib), str(target))
    if verbose:
        print(f"built {target}")
    return target


if __name__ == "__main__":
    build()
    sys.exit(0)
