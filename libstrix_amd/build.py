# SPDX-License-Identifier: MIT
"""Builds libstrix_amd/_strix_amd.so from csrc/*.hip for gfx950 only.

One hipcc compile per source (in parallel), one link. Replaces the
reference's CMake build (CMakeLists.txt:4-25, build.sh:8-14), whose arch was
gfx1151; this library is gfx950-only and carries no torch symbols, so a plain
`hipcc -shared` is all it needs.

    python libstrix_amd/build.py [-j N] [-v]

(run as a script, not through the package: importing the package loads the
built library, which may predate the sources)
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
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "_strix_amd.so"
INCLUDE = PKG.parent / "include"

ARCH = "gfx950"
# Packed-fp32 VALU forms are disabled on purpose (plain float code only).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=fast",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # MFMA results in arch VGPRs: the block-scale fold reads every result
    # with a VALU FMA, which cannot take AGPR operands.
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: libstrix_amd needs ROCm's hipcc to build")


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr[-6000:]}")
    if verbose and res.stderr.strip():
        print(res.stderr[-3000:], file=sys.stderr)
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    """Compiles every csrc/*.hip and links the shared library. Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-6000:]}")
    os.replace(tmp, LIB)
    return LIB


TORCH_EXT_SRC = PKG / "torch_ext" / "strix_ops.cpp"
TORCH_EXT = PKG / "_strix_torch.so"


def build_torch_ext(verbose: bool = False) -> Path:
    """The C++ torch.ops.strix registration (torch_ext/strix_ops.cpp): host
    code only, compiled with the system C++ compiler against the installed
    torch's headers and libraries, linked to _strix_amd.so (found next to it
    at run time through an $ORIGIN rpath)."""
    import torch

    tdir = Path(torch.__file__).resolve().parent
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("no C++ compiler for the torch extension")
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    tmp = TORCH_EXT.with_suffix(".so.tmp")
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=strix_torch",
           f"-I{tdir / 'include'}", f"-I{tdir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
           "-I/opt/rocm/include", f"-I{INCLUDE}", str(TORCH_EXT_SRC), "-o", str(tmp),
           f"-L{tdir / 'lib'}", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-lc10", "-lc10_hip", "-lamdhip64",
           f"-L{PKG}", "-l:_strix_amd.so", "-Wl,-rpath,$ORIGIN", "-Wl,--no-undefined"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch extension build failed:\n{res.stderr[-6000:]}")
    os.replace(tmp, TORCH_EXT)
    return TORCH_EXT


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.v))
    print(build_torch_ext(a.v))


if __name__ == "__main__":
    main()
