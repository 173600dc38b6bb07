"""Build recipe for ane_amd/libane_amd.so (gfx950), the benchmark's
bench_peaks.so (beside bench.py, not part of the package) and the CPU
oracle.

Run ``python -m ane_amd.build`` (or ``__graft_entry__.build()``).  The
library is built in-tree so it travels with the repository snapshot; object
files go to ``ane_amd/_build/``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libane_amd.so"
PEAKS_SRC = ROOT / "bench_peaks.hip"
PEAKS_LIB = ROOT / "bench_peaks.so"
GGML_SRC = PKG / "ggml" / "ggml-ane.cpp"
GGML_IFACE = ROOT / "tests" / "ggml_iface"
GGML_TEST_LIB = GGML_IFACE / "libggml_ane_test.so"

ARCH = "gfx950"

# -ffp-contract=off: the epilogues and quantizers must round after every
# fmul/fadd exactly like the reference's unfused SVE instructions.
# packed-fp32-ops is disabled for every HIP translation unit.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build ane_amd)")


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build_library(verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    cc = hipcc()
    jobs = []
    for src in sorted(CSRC.glob("*.hip")):
        obj = OBJ / (src.stem + ".o")
        jobs.append([cc, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
    for src in sorted(CSRC.glob("*.cpp")):
        obj = OBJ / (src.stem + ".host.o")
        jobs.append([cc, *HOST_FLAGS, "-I/opt/rocm/include", "-c", str(src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as ex:
        list(ex.map(_run, jobs))
    objs = [str(p) for p in sorted(OBJ.glob("*.o"))]
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def build_peaks(verbose: bool = False) -> Path:
    """bench_peaks.so: the MFMA-loop and HBM-stream ceilings bench.py reports."""
    tmp = PEAKS_LIB.with_suffix(".so.tmp")
    _run([hipcc(), *HIP_FLAGS, "-shared", str(PEAKS_SRC), "-o", str(tmp)])
    os.replace(tmp, PEAKS_LIB)
    if verbose:
        print(f"built {PEAKS_LIB}")
    return PEAKS_LIB


def ggml_adapter_cmd(out: Path) -> list[str]:
    """g++ line building the ggml registry adapter (ane_amd/ggml/ggml-ane.cpp)
    against the restated ggml interface of tests/ggml_iface, with that
    folder's test harness, into one shared library linking libane_amd.so.
    In a real build the adapter is compiled inside a ggml tree instead."""
    return ["g++", "-std=c++17", "-O1", "-fPIC", "-shared", "-Wall", "-D__HIP_PLATFORM_AMD__",
            "-I/opt/rocm/include", f"-I{ROOT / 'include'}", f"-I{PKG / 'ggml'}", f"-I{GGML_IFACE}",
            str(GGML_SRC), str(GGML_IFACE / "ggml_test_support.cpp"), "-o", str(out),
            f"-L{PKG}", "-lane_amd", f"-Wl,-rpath,{PKG}", "-Wl,-rpath,$ORIGIN/../../ane_amd",
            "-L/opt/rocm/lib", "-lamdhip64"]


def build_ggml_adapter(verbose: bool = False) -> Path:
    tmp = GGML_TEST_LIB.with_suffix(".so.tmp")
    _run(ggml_adapter_cmd(tmp))
    os.replace(tmp, GGML_TEST_LIB)
    if verbose:
        print(f"built {GGML_TEST_LIB}")
    return GGML_TEST_LIB


DISPATCH_SRC = ROOT / "tests" / "cpp" / "mnist_i8_dispatch.cpp"
DISPATCH_BIN = ROOT / "tests" / "cpp" / "mnist_i8_dispatch"


def build_dispatch_program(verbose: bool = False) -> Path:
    """tests/cpp/mnist_i8_dispatch: the reference's MNIST-i8 call sequence
    written against include/ane/ane.hpp, linked against libane_amd.so (a GPU
    test runs it as a child process)."""
    tmp = DISPATCH_BIN.with_suffix(".tmp")
    _run(["g++", "-std=c++20", "-O1", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
          f"-I{ROOT / 'include'}", str(DISPATCH_SRC), "-o", str(tmp), f"-L{PKG}", "-lane_amd",
          "-Wl,-rpath,$ORIGIN/../../ane_amd", "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"])
    os.replace(tmp, DISPATCH_BIN)
    if verbose:
        print(f"built {DISPATCH_BIN}")
    return DISPATCH_BIN


def build_oracle(verbose: bool = False) -> Path:
    _run(["make", "-s", "-C", str(ROOT / "oracle")])
    out = ROOT / "oracle" / "libane_oracle.so"
    if verbose:
        print(f"built {out}")
    return out


def build_all(verbose: bool = False) -> None:
    build_oracle(verbose)
    build_library(verbose)
    build_peaks(verbose)
    build_ggml_adapter(verbose)
    build_dispatch_program(verbose)


if __name__ == "__main__":
    build_all(verbose=True)
    sys.exit(0)
