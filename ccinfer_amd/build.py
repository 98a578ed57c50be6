"""Builds libccinfer_attn.so (HIP kernels + C ABI + C++ drop-in layer) for gfx950, in-tree.

Usage: python -m ccinfer_amd.build   (also called by __graft_entry__.build()).
Objects go to ccinfer_amd/_build/, the library to ccinfer_amd/lib/libccinfer_attn.so.
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
BUILD = PKG / "_build"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libccinfer_attn.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 VALU ops are disabled for device code (some forms have given wrong results on
# this pool); hipcc's host pass warns that it does not know the feature, which is harmless.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-command-line-argument",
    # Kernels mask with -inf and never rely on NaN semantics; this drops the NaN
    # canonicalisation fmaxf would otherwise emit in the softmax max reductions.
    "-fno-honor-nans",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
    f"-I{CSRC / 'dropin'}",
]

SOURCES = [
    CSRC / "write_kv_cache.hip",
    CSRC / "decode_attn.hip",
    CSRC / "prefill_attn.hip",
    CSRC / "layout.hip",
    CSRC / "qkv_prologue.hip",
    CSRC / "batch_meta.hip",
    CSRC / "kv_fp8.hip",
    CSRC / "noalloc.hip",
    CSRC / "capi.cpp",
    CSRC / "dropin" / "launchers.cpp",
    CSRC / "dropin" / "hip_backend.cpp",
]


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + src.suffix.replace(".", "_") + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [HIPCC, *HIP_FLAGS, *lang, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    noise = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
    if any("warning" in ln for ln in noise):
        sys.stderr.write("\n".join(noise) + "\n")
    return obj


def build(verbose: bool = True) -> Path:
    """Compiles every source and links the shared library. Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    jobs = min(len(SOURCES), max(1, (os.cpu_count() or 2)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    # --no-undefined: a kernel whose host launch stub went missing fails here, not at load.
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o",
           str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    _build_cpp_tests()
    if verbose:
        print(f"[ccinfer_amd] built {LIB}")
    return LIB


CPP_TEST = BUILD / "test_dropin"


def _build_cpp_tests() -> None:
    """The C++ drop-in test program (tests/cpp/test_dropin.cpp), linked against the library."""
    src = ROOT / "tests" / "cpp" / "test_dropin.cpp"
    cmd = [HIPCC, *HIP_FLAGS, "-x", "hip", str(src), "-o", str(CPP_TEST), f"-L{LIBDIR}",
           "-lccinfer_attn", f"-Wl,-rpath,{LIBDIR}", "-Wl,-rpath,$ORIGIN/../lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"test build failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build_oracle(verbose: bool = True) -> Path:
    """Compiles the CPU oracle (test infrastructure) with its Makefile."""
    oracle = ROOT / "oracle"
    res = subprocess.run(["make", "-s", "-B", "-C", str(oracle)], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed\n{res.stdout}\n{res.stderr}")
    if verbose:
        print(f"[ccinfer_amd] built {oracle / 'liboracle.so'}")
    return oracle / "liboracle.so"


if __name__ == "__main__":
    build()
    build_oracle()
