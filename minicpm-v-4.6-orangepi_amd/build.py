"""Build the gfx950 quantized-matmul library and its C++ operator layer in-tree.

Outputs (all git-ignored, all shipped to the GPU box with the source tree):
  lib/libmcv_quant.so     C-ABI (include/mcv_quant.h): HIP kernels + host packers
  lib/libminicpmv_ops.so  C++ operator surface (namespace minicpmv) over the C-ABI
  tests/cpp/bin/*         C++ test programs mirroring the reference's tests

Every call recompiles everything (objects go to _build/); compiles run in
parallel.  Only hipcc/g++ are used -- no CMake, no JIT cache outside the tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
CPP = PKG / "cpp"
LIB = PKG / "lib"
BUILD = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Device flags.  Packed-fp32 instructions are disabled; fp32 division and
# sqrt stay correctly rounded.  Contraction is off: the epilogues must round
# to fp32 before the fp16 conversion exactly as the reference does (with
# contraction on, clang folds mul + fp32->fp16 into one v_fma_mixlo_f16, a
# single rounding); fused multiply-adds are written explicitly (fmaf, dot2,
# MFMA builtins).
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-command-line-argument",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", f"-I{ROOT / 'include'}", f"-I{CPP / 'include'}",
             "-I/opt/rocm/include", "-D__HIP_PLATFORM_AMD__"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = ("packed-fp32-ops", "is not a recognized feature for this target")
    err = "\n".join(l for l in (proc.stderr or "").splitlines() if not any(n in l for n in noise))
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}\n{proc.stdout}")
    if err.strip():
        sys.stderr.write(err + "\n")


def _compile_hip(src: Path) -> Path:
    obj = BUILD / (src.name + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
    return obj


def _compile_cxx(src: Path) -> Path:
    obj = BUILD / ("cpp_" + src.name + ".o")
    _run(["g++", *CXX_FLAGS, "-c", str(src), "-o", str(obj)])
    return obj


def build_capi(jobs: int | None = None) -> Path:
    """Compile csrc/ into lib/libmcv_quant.so."""
    BUILD.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile_hip, srcs))
    out = LIB / "libmcv_quant.so"
    tmp = LIB / "libmcv_quant.so.tmp"
    # --no-undefined: a kernel whose host stub was not emitted fails here,
    # not at dlopen on the GPU box
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, out)
    return out


def build_cpp_layer(jobs: int | None = None) -> Path:
    """Compile the C++ operator surface into lib/libminicpmv_ops.so (links the C-ABI)."""
    srcs = sorted((CPP / "lib").glob("*.cpp"))
    if not srcs:
        return LIB / "libminicpmv_ops.so"
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile_cxx, srcs))
    out = LIB / "libminicpmv_ops.so"
    tmp = LIB / "libminicpmv_ops.so.tmp"
    _run(["g++", "-shared", "-o", str(tmp), *map(str, objs), f"-L{LIB}", "-lmcv_quant",
          "-L/opt/rocm/lib", "-lamdhip64", "-lrocblas", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,/opt/rocm/lib"])
    os.replace(tmp, out)
    return out


def build_cpp_tests(jobs: int | None = None) -> list[Path]:
    """Compile tests/cpp/*.cpp into tests/cpp/bin/ against the C++ layer.  The
    test programs also link the CPU oracle (oracle/build/libmcv_oracle.so, test
    infrastructure) as their checker; the product libraries never do."""
    tdir = ROOT / "tests" / "cpp"
    srcs = sorted(tdir.glob("test_*.cpp"))
    bindir = tdir / "bin"
    bindir.mkdir(parents=True, exist_ok=True)
    oracle = ROOT / "oracle"
    if not (oracle / "build" / "libmcv_oracle.so").exists():
        _run(["make", "-C", str(oracle)])

    def one(src: Path) -> Path:
        exe = bindir / src.stem
        _run(["g++", *CXX_FLAGS, f"-I{oracle}", str(src), "-o", str(exe), f"-L{LIB}", "-lminicpmv_ops", "-lmcv_quant",
              f"-L{oracle / 'build'}", "-lmcv_oracle", "-L/opt/rocm/lib", "-lamdhip64",
              "-Wl,-rpath,$ORIGIN/../../../minicpm-v-4.6-orangepi_amd/lib", "-Wl,-rpath,$ORIGIN/../../../oracle/build",
              "-Wl,-rpath,/opt/rocm/lib"])
        return exe

    if not srcs:
        return []
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(srcs))) as ex:
        return list(ex.map(one, srcs))


def build_all() -> None:
    build_capi()
    build_cpp_layer()
    build_cpp_tests()


if __name__ == "__main__":
    build_all()
    print("built", LIB)
