"""Build libhx_exl3.so (HIP, gfx950) in-tree, and the CPU oracle used by the tests.

Usage: python -m helios_glm53flash_amd.build [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_build"
LIB = PKG / "libhx_exl3.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # packed fp32 VALU ops are kept out of every code object on this target
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


# Per-file flags.  The MFMA-tile kernels keep their accumulators in VGPRs: with the default
# selection the accumulators live in AGPRs while the MFMAs are selected in their VGPR form, and every
# k step copies them back and forth (3 extra VALU moves per MFMA on gfx950, measured in the
# generated code).
FILE_FLAGS = {
    "hx_moe_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "hx_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _compile(src: Path) -> Path:
    obj = OUT_DIR / (src.stem + ".o")
    deps = [src] + sorted(CSRC.glob("*.hpp")) + [ROOT / "include" / "hx" / "exl3.h", Path(__file__)]
    if obj.exists() and obj.stat().st_mtime > max(d.stat().st_mtime for d in deps):
        return obj
    cmd = [HIPCC, *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed for {src.name}")
    return obj


def build_hip(jobs: int = 8, force: bool = False) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if force:
        for o in OUT_DIR.glob("*.o"):
            o.unlink()
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(LIB), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link of libhx_exl3.so failed")
    return LIB


DRIVER_SRC = ROOT / "tests" / "cpp" / "compat_driver.cpp"
DRIVER = ROOT / "tests" / "cpp" / "compat_driver"


def build_cpp_driver() -> Path:
    """The C++ test driver of the reference-signature layer (include/helios/exl3_compat.hpp), linked
    against the in-tree library (found through its rpath, relative to the driver)."""
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-O2", "-std=c++17", f"-I{ROOT / 'include'}", str(DRIVER_SRC), "-o",
           str(DRIVER), f"-L{PKG}", "-lhx_exl3", "-Wl,-rpath,$ORIGIN/../../helios_glm53flash_amd"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("build of tests/cpp/compat_driver failed")
    return DRIVER


def build_oracle() -> Path:
    r = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("oracle build failed")
    return ROOT / "oracle" / "liboracle.so"


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    ap.add_argument("--force", action="store_true")
    a = ap.parse_args()
    print(build_hip(a.jobs, a.force))
    print(build_oracle())
    print(build_cpp_driver())


if __name__ == "__main__":
    main()
