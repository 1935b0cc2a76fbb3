"""Build libtinyengine.so (gfx950 HIP kernels + C ABI) in-tree.

    python -m tinymetalagent_amd.build        # or __graft_entry__.build()

Outputs:
    tinymetalagent_amd/_build/*.o
    tinymetalagent_amd/libtinyengine.so      (next to the package, where the
                                              ctypes loader looks for it)

Every HIP source is compiled for gfx950 only, with packed-FP32 instruction
selection disabled (-Xclang -target-feature -Xclang -packed-fp32-ops).
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
BUILD = PKG / "_build"
INCLUDE = ROOT / "include"
LIBRARY = PKG / "libtinyengine.so"

HIP_SOURCES = ["te_rope_append.hip", "te_decode.hip", "te_prefill.hip", "te_mma_kat.hip", "te_calibrate.hip",
               "te_vecops.hip", "te_decode_layers.hip", "te_prefill_layers.hip", "te_gemm.hip", "te_sample.hip", "te_model.hip",
               "te_hip_runtime.hip"]
C_SOURCES = ["te_abi.c"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).is_file():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libtinyengine.so)")


HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "--offload-arch=gfx950",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]
# Per-source additions.  te_gemm.hip: MFMA results in VGPRs rather than
# accumulation registers (its blocks' integer sums are shifted and scaled by
# VALU code; the accumulation-register form moved every one through v_accvgpr
# reads and writes: gate GEMM at 512 rows 103 -> 92 us).
# te_vecops.hip and te_gemm.hip: the iterative-ilp scheduling strategy (the
# 3B decode token Q4_0 1,431 -> 1,404 us, Q8_0 1,646 -> 1,627 us; the prompt
# GEMM at 512 rows, gate 87.1 -> 84.7 us, down 91.0 -> 90.3 us; same box,
# alternating builds).  The prefill, decode and append sources measured no
# better with it or the other strategies.
HIP_SOURCE_FLAGS = {
    "te_gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
    "te_vecops.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
}


def build(verbose: bool = False) -> Path:
    """Compile every source and link the shared library; returns its path."""
    hipcc = _hipcc()
    BUILD.mkdir(exist_ok=True)
    jobs = []
    objs = []
    for src in HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        cmd = [hipcc, *HIP_FLAGS, *HIP_SOURCE_FLAGS.get(src, []), f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / src),
               "-o", str(obj)]
        jobs.append((src, cmd))
        objs.append(obj)
    for src in C_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        cmd = ["gcc", "-std=c11", "-O2", "-fPIC", "-Wall", "-Wextra", "-pedantic", f"-I{INCLUDE}",
               "-D_POSIX_C_SOURCE=200809L", "-c", str(CSRC / src), "-o", str(obj)]
        jobs.append((src, cmd))
        objs.append(obj)
    procs = []
    for src, cmd in jobs:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for src, p in procs:
        out, _ = p.communicate()
        # hipcc's host pass does not know the packed-fp32 target feature; drop that note.
        lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
        if lines and (verbose or p.returncode != 0):
            print(f"--- {src}\n" + "\n".join(lines), file=sys.stderr)
        if p.returncode != 0:
            failed.append(src)
    if failed:
        raise RuntimeError(f"compilation failed: {', '.join(failed)}")
    tmp = LIBRARY.with_suffix(".so.tmp")
    # -z defs: an unresolved symbol (e.g. a kernel stub the host pass did not
    # emit) fails the link here instead of the first dlopen.
    link = [hipcc, "-shared", "-fPIC", "--offload-arch=gfx950", "-Wl,-z,defs", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(link), flush=True)
    subprocess.run(link, check=True)
    os.replace(tmp, LIBRARY)
    return LIBRARY


# Host-sanitizer build (CPU testing only): the host code of the GGUF loader,
# tokenizer and C ABI (te_model.hip, te_abi.c) compiled with AddressSanitizer
# and UndefinedBehaviorSanitizer, linked with the other objects of the normal
# build into a separate library.  GPU code is compiled as usual (the
# sanitizer flags apply to the host pass only).  Load it with the clang ASan
# runtime preloaded (asan_runtime()) and TINYENGINE_LIBRARY pointing at it.
SAN_BUILD = PKG / "_build_san"
SAN_LIBRARY = SAN_BUILD / "libtinyengine_san.so"
SAN_SOURCES = ["te_model.hip"]
SAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer", "-g"]


def asan_runtime() -> Path:
    """The clang AddressSanitizer runtime that the sanitized library needs preloaded."""
    llvm = Path(_hipcc()).resolve().parent.parent / "lib" / "llvm"
    for cand in sorted(llvm.glob("lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")) + \
            sorted(Path("/opt/rocm/lib/llvm").glob("lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so")):
        return cand
    raise RuntimeError("clang AddressSanitizer runtime not found")


def build_sanitized(verbose: bool = False) -> Path:
    """Build libtinyengine_san.so (needs the objects of build() for the rest)."""
    hipcc = _hipcc()
    clang = Path(hipcc).resolve().parent.parent / "lib" / "llvm" / "bin" / "clang"
    if not clang.is_file():
        clang = Path("/opt/rocm/lib/llvm/bin/clang")
    SAN_BUILD.mkdir(exist_ok=True)
    objs = []
    for src in HIP_SOURCES:
        if src in SAN_SOURCES:
            obj = SAN_BUILD / (Path(src).stem + ".o")
            cmd = [hipcc, *HIP_FLAGS, *HIP_SOURCE_FLAGS.get(src, []), *SAN_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c",
                   str(CSRC / src), "-o", str(obj)]
            if verbose:
                print(" ".join(cmd), flush=True)
            subprocess.run(cmd, check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
        else:
            obj = BUILD / (Path(src).stem + ".o")
            if not obj.is_file():
                raise RuntimeError(f"{obj} missing: run build() first")
        objs.append(obj)
    obj = SAN_BUILD / "te_abi.o"
    cmd = [str(clang), "-std=c11", "-O1", "-g", "-fPIC", "-Wall", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", f"-I{INCLUDE}", "-D_POSIX_C_SOURCE=200809L",
           "-c", str(CSRC / "te_abi.c"), "-o", str(obj)]
    subprocess.run(cmd, check=True)
    objs.append(obj)
    link = [hipcc, "-shared", "-fPIC", "--offload-arch=gfx950", "-fsanitize=address,undefined", "-fno-gpu-sanitize",
            "-shared-libsan", *map(str, objs), "-o", str(SAN_LIBRARY)]
    if verbose:
        print(" ".join(link), flush=True)
    subprocess.run(link, check=True)
    return SAN_LIBRARY


# Phase-instrumented build (profiling only): te_prefill.hip with
# -DTE_PREFILL_PHASES (the causal prefill kernel sums shader-clock cycles per
# phase of its step loop into a log set by te_hip_prefill_phase_log_set),
# linked with the other objects of the normal build.  bench.py --phases runs
# it and prints the phase table.
PHASE_BUILD = PKG / "_build_phases"
PHASE_LIBRARY = PHASE_BUILD / "libtinyengine_phases.so"


def build_phases(verbose: bool = False) -> Path:
    """Build libtinyengine_phases.so (needs the objects of build() for the rest)."""
    hipcc = _hipcc()
    PHASE_BUILD.mkdir(exist_ok=True)
    objs = []
    for src in HIP_SOURCES:
        if src == "te_prefill.hip":
            obj = PHASE_BUILD / "te_prefill.o"
            cmd = [hipcc, *HIP_FLAGS, *HIP_SOURCE_FLAGS.get(src, []), "-DTE_PREFILL_PHASES", f"-I{INCLUDE}",
                   f"-I{CSRC}", "-c", str(CSRC / src), "-o", str(obj)]
            if verbose:
                print(" ".join(cmd), flush=True)
            subprocess.run(cmd, check=True, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
        else:
            obj = BUILD / (Path(src).stem + ".o")
            if not obj.is_file():
                raise RuntimeError(f"{obj} missing: run build() first")
        objs.append(obj)
    objs += [BUILD / (Path(src).stem + ".o") for src in C_SOURCES]
    link = [hipcc, "-shared", "-fPIC", "--offload-arch=gfx950", "-Wl,-z,defs", *map(str, objs), "-o",
            str(PHASE_LIBRARY)]
    subprocess.run(link, check=True)
    return PHASE_LIBRARY


if __name__ == "__main__":
    if "--phases" in sys.argv:
        print(build_phases(verbose="-v" in sys.argv))
    elif "--sanitize" in sys.argv:
        print(build_sanitized(verbose="-v" in sys.argv))
    else:
        print(build(verbose="-v" in sys.argv))
