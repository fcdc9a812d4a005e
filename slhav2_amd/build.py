"""Build libslha.so (HIP, gfx950) and the CPU oracle library.

No cmake/ninja: one hipcc link line for the product library and one gcc line
per oracle library. Everything is written in-tree so the built files travel
with the repository snapshot to the GPU box.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libslha.so"
# bench.py's floor kernel (not part of the product library)
BENCH_LIB = PKG / "libslha_bench.so"
ORACLE = ROOT / "oracle"
ORACLE_LIB = ORACLE / "liboracle_slha.so"
CPU_BASELINE_LIB = ORACLE / "libcpu_baseline.so"

ARCH = os.environ.get("SLHA_GPU_ARCH", "gfx950")

HIP_SOURCES = ["slha_kernels.hip", "slha_abi.cpp"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Rust never contracts a*b+c; exact kernels rely on this. Fast kernels
    # call fmaf() explicitly.
    "-ffp-contract=off",
    # Keep hipcc away from packed-FP32 instructions (v_pk_add/mul/fma_f32):
    # some of their forms have given sporadic wrong results on these GPUs.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs rather than AGPRs: the score kernels read every
    # accumulator back with VALU, and AGPRs would cost a copy per register
    # and one wave of occupancy.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: cannot build libslha.so")


def _run(cmd: list[str], cwd: Path) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, cwd=cwd, check=True)


def _layout_defines() -> list[str]:
    # SLHA_CACHE_LINE_128=1: 128-byte tile alignment (include/slha.h); callers
    # then compile against the header with the same definition.
    v = os.environ.get("SLHA_CACHE_LINE_128", "")
    return ["-DSLHA_CACHE_LINE_128=1"] if v not in ("", "0") else []


def build_library(verbose: bool = True) -> Path:
    srcs = [str(CSRC / s) for s in HIP_SOURCES]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), *HIPCC_FLAGS, *_layout_defines(), "-I", str(ROOT / "include"), *srcs, "-o", str(tmp)]
    _run(cmd, CSRC)
    os.replace(tmp, LIB)
    return LIB


# Host-side sanitizer build of the product library (CPU tests only; the GPU
# code is compiled as usual): AddressSanitizer and UndefinedBehaviorSanitizer
# on the host C++ - the .slhw loader, the EventLog file side, the CCOS host
# mirror and every argument check. tests/run_sanitized.sh runs the CPU tests
# against it.
ASAN_LIB = PKG / "libslha_asan.so"
SANITIZE_HOST = [
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=undefined",
    "-Xarch_host", "-fno-omit-frame-pointer",
    "-shared-libasan",
]


def build_sanitized_library() -> Path:
    srcs = [str(CSRC / s) for s in HIP_SOURCES]
    tmp = ASAN_LIB.with_suffix(".so.tmp")
    flags = [f for f in HIPCC_FLAGS if f != "-O3"] + ["-O1", "-g"]
    cmd = [_hipcc(), *flags, *SANITIZE_HOST, *_layout_defines(), "-I", str(ROOT / "include"), *srcs,
           "-o", str(tmp)]
    _run(cmd, CSRC)
    os.replace(tmp, ASAN_LIB)
    return ASAN_LIB


def build_bench_library() -> Path:
    tmp = BENCH_LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), *HIPCC_FLAGS, str(CSRC / "bench_floor.hip"), "-o", str(tmp)]
    _run(cmd, CSRC)
    os.replace(tmp, BENCH_LIB)
    return BENCH_LIB


def build_oracle() -> Path:
    cc = shutil.which("gcc") or "cc"
    common = ["-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
              "-Wall", "-Wextra"]
    _run([cc, *common, "slha_oracle.c", "-lm", "-o", ORACLE_LIB.name], ORACLE)
    # The CPU baseline (AVX-512/AVX2 restatement of simd.rs) is runtime
    # dispatched, so it builds without host-specific -march flags.
    _run([cc, "-O3", "-std=c11", "-fPIC", "-shared", "-Wall", "-pthread", "-ffp-contract=off",
          "cpu_baseline.c",
          "slha_oracle.c", "-lm", "-o", CPU_BASELINE_LIB.name], ORACLE)
    return ORACLE_LIB


def build_all() -> None:
    build_oracle()
    build_library()
    build_bench_library()


if __name__ == "__main__":
    what = sys.argv[1] if len(sys.argv) > 1 else "all"
    if what == "oracle":
        build_oracle()
    elif what == "lib":
        build_library()
    elif what == "bench":
        build_bench_library()
    elif what == "sanitize":
        build_sanitized_library()
    else:
        build_all()
