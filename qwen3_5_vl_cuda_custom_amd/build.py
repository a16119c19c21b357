"""Ahead-of-time build of libq3vl.so for gfx950 (MI355X).

Compiles every csrc/*.hip with hipcc into objects under _build/ and links them
into `qwen3_5_vl_cuda_custom_amd/lib/libq3vl.so`, next to the package so the
built library travels with the source tree. Usage: `python -m
qwen3_5_vl_cuda_custom_amd.build` (or `__graft_entry__.build()`).
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
INCLUDE = ROOT / "include"
BUILD = ROOT / "_build"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libq3vl.so"

ARCH = "gfx950"
# Packed-fp32 VALU ops are disabled for all device code (the compiler is free
# to emit them from scalar float code otherwise).
HIPFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Wno-unused-function",
    "-Wno-unused-variable", "-Wno-unused-but-set-variable",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


# Per-source extra flags. attention.hip: MFMA results in arch VGPRs rather than
# AGPRs (its kernels' whole state fits the 256 registers of 2 waves per SIMD;
# with AGPRs the softmax copied every score tile out of them).
EXTRA_FLAGS: dict[str, list[str]] = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _hipcc() -> str:
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(p).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build libq3vl.so")
    return p


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [_hipcc(), *HIPFLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature and says so; drop that line.
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile all HIP sources and link libq3vl.so. Always recompiles."""
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [BUILD / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, o, verbose) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
