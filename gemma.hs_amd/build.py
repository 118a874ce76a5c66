"""Build libgemma_hip.so (hipcc, gfx950) and the oracle's liboracle.so (gcc).

Usage: python gemma.hs_amd/build.py [--only lib|oracle] [--no-marks] [-j N]

Objects go to gemma.hs_amd/_build/, the library to
gemma.hs_amd/gemma_hip/libgemma_hip.so and the oracle to
oracle/build/liboracle.so (all git-ignored; the built .so files travel to
the GPU box with the source tree).  Beside the library, the same pool
builds libgemma_hip_marks.so: the library with the step kernels compiled
from csrc/marks/marks.hip (phase timestamps, for gemma_hip.kernel_profile
phases); nothing loads it unless GEMMA_HIP_LIB names it.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
REPO = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "gemma_hip" / "libgemma_hip.so"
MARKS_LIB = PKG / "gemma_hip" / "libgemma_hip_marks.so"
MARKS_SRC = CSRC / "marks" / "marks.hip"
MARKS_TUS = (1, 5, 6, 7)  # the decode step's kernels: attention, then the matvec phases
ORACLE_DIR = REPO / "oracle"
ORACLE_LIB = ORACLE_DIR / "build" / "liboracle.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
KERNEL_TUS = 7  # kernels.hip: step, persistent step, prefill, op level, 3 x step matvec phases
ARCH = "gfx950"
# Packed FP32 (v_pk_*_f32) is disabled for every HIP translation unit.
# MFMA results go to VGPRs (gfx950 allows it): the compiler's default AGPR
# destinations cost two v_accvgpr_read per MFMA in the prefill GEMM and the
# matrix-core matvec, whose results feed VALU scale-and-add.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wno-unused-result", "-Wno-unused-value",
]
HOST_CXX = shutil.which("g++") or "c++"
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-result", "-Wno-unused-value",
              "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise SystemExit(f"build failed: {cmd[-1] if cmd else ''}")
    # surface real warnings only (the host pass warns about the packed-fp32 feature flag)
    for line in (r.stdout + r.stderr).splitlines():
        if "packed-fp32-ops" in line or "target-feature" in line:
            continue
        if "warning" in line or "error" in line:
            sys.stderr.write(line + "\n")


def build_lib(jobs: int = 8, marks: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    units = []
    if marks:  # the longest units first
        for tu in MARKS_TUS:
            units.append((MARKS_SRC, [HIPCC, *DEVICE_FLAGS, f"-DGH_TU={tu}", "-x", "hip"], f"marks_tu{tu}"))
    for src in sorted(CSRC.iterdir()):
        if src.name == "kernels.hip":
            # compiled as KERNEL_TUS translation units in parallel (GH_TU in kernels.hip)
            for tu in range(1, KERNEL_TUS + 1):
                units.append((src, [HIPCC, *DEVICE_FLAGS, f"-DGH_TU={tu}", "-x", "hip"], f"{src.stem}_tu{tu}"))
        elif src.suffix == ".hip":
            units.append((src, [HIPCC, *DEVICE_FLAGS, "-x", "hip"], src.stem))
        elif src.suffix == ".cpp":
            units.append((src, [HOST_CXX, *HOST_FLAGS], src.stem))
    objs = []

    def compile_one(item):
        src, cmd, stem = item
        obj = OBJ / (stem + ".o")
        _run([*cmd, "-c", str(src), "-o", str(obj)])
        return obj

    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, units))
    lib_objs = [o for o in objs if not o.name.startswith("marks_")]
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, lib_objs),
          "-lpthread"])
    os.replace(tmp, LIB)
    if marks:
        marked = {f"kernels_tu{tu}.o" for tu in MARKS_TUS}
        mobjs = [o for o in objs if o.name.startswith("marks_")] + [o for o in lib_objs if o.name not in marked]
        tmp = MARKS_LIB.with_suffix(".so.tmp")
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, mobjs), "-lpthread"])
        os.replace(tmp, MARKS_LIB)
    return LIB


HOST_TEST_SRC = REPO / "tests" / "cpp" / "host_api_test.cpp"
HOST_TEST_LIB = REPO / "tests" / "cpp" / "libhost_api_test.so"


def build_host_tests() -> Path:
    """The C++ host-API checks (tests/cpp/host_api_test.cpp) as a shared
    library linked against libgemma_hip and the oracle; it finds both through
    an $ORIGIN-relative runpath."""
    tmp = HOST_TEST_LIB.with_suffix(".so.tmp")
    _run([HOST_CXX, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall",
          f"-I{REPO / 'include'}", f"-I{PKG / 'host'}", f"-I{ORACLE_DIR}", str(HOST_TEST_SRC), "-o", str(tmp),
          f"-L{LIB.parent}", "-lgemma_hip", f"-L{ORACLE_LIB.parent}", "-loracle",
          "-Wl,-rpath,$ORIGIN/../../gemma.hs_amd/gemma_hip", "-Wl,-rpath,$ORIGIN/../../oracle/build",
          "-Wl,--allow-shlib-undefined"])
    os.replace(tmp, HOST_TEST_LIB)
    return HOST_TEST_LIB


def build_oracle() -> Path:
    ORACLE_LIB.parent.mkdir(exist_ok=True)
    cc = shutil.which("gcc") or "cc"
    tmp = ORACLE_LIB.with_suffix(".so.tmp")
    _run([cc, "-O2", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-std=c11",
          "-Wall", str(ORACLE_DIR / "gemma_oracle.c"), "-o", str(tmp), "-lm"])
    os.replace(tmp, ORACLE_LIB)
    return ORACLE_LIB


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", choices=["lib", "oracle"])  # default: lib, oracle and the C++ host tests
    ap.add_argument("--no-marks", action="store_true", help="skip libgemma_hip_marks.so")
    ap.add_argument("-j", type=int, default=8)
    a = ap.parse_args(argv)
    if a.only in (None, "oracle"):
        print("built", build_oracle())
    if a.only in (None, "lib"):
        print("built", build_lib(a.j, marks=not a.no_marks))
    if a.only is None:
        print("built", build_host_tests())


if __name__ == "__main__":
    main()
