"""Builds libgrinnder_amd.so (HIP for gfx950 + host C++) in-tree with hipcc.

Usage: ``python -m grinnder_amd.build`` (or ``__graft_entry__.build()``).
The library links against the HIP runtime that ships with torch so that a
process which imports torch holds exactly one HIP runtime.
"""

from __future__ import annotations

import concurrent.futures as cf
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libgrinnder_amd.so"
ARCH = os.environ.get("GRINNDER_AMD_ARCH", "gfx950")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

SOURCES = [
    "status.cpp",
    "graph_prep.cpp",
    "io_engine.cpp",
    "transfer.hip",
    "aggregate.hip",
    "gat.hip",
    "gat_narrow.hip",
    "gemm.hip",
    "loss.hip",
]

# Packed-FP32 instructions are disabled for every device compile.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def source_hash() -> str:
    """Hex SHA-256 over the library's sources (csrc/*, the public header), the
    target architecture and the device flags.  Embedded in the library as
    gr_source_hash(); the loader compares the two."""
    h = hashlib.sha256()
    files = sorted(p for p in CSRC.iterdir() if p.suffix in (".hip", ".cpp", ".h"))
    files.append(PKG_DIR.parent / "include" / "grinnder_amd.h")
    for p in files:
        h.update(p.name.encode() + b"\0" + p.read_bytes() + b"\0")
    h.update(ARCH.encode() + b"\0" + " ".join(DEVICE_FLAGS).encode())
    return h.hexdigest()


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the HIP toolchain is required to build")
    return path


def _torch_lib_dir() -> Path:
    import torch  # noqa: F401  (only to locate its bundled HIP runtime)

    return Path(torch.__file__).resolve().parent / "lib"


def _compile(src: Path, obj: Path, digest: str) -> None:
    cmd = [_hipcc(), "-std=c++17", "-O3", "-fPIC", "-Wall", "-Wno-unused-result",
           f"-I{PKG_DIR.parent / 'include'}", f'-DGR_SOURCE_HASH="{digest}"', "-c", str(src),
           "-o", str(obj)]
    if src.suffix == ".hip":
        cmd[1:1] = ["-x", "hip", f"--offload-arch={ARCH}", *DEVICE_FLAGS]
    else:
        cmd[1:1] = ["-x", "c++", "-D__HIP_PLATFORM_AMD__=1", f"-I{ROCM}/include"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")


def build(verbose: bool = True) -> Path:
    """Compiles every source and links the shared library; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    digest = source_hash()
    objs = []
    jobs = []
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        for name in SOURCES:
            src = CSRC / name
            obj = BUILD_DIR / (name + ".o")
            objs.append(obj)
            jobs.append(ex.submit(_compile, src, obj, digest))
        for j in jobs:
            j.result()
    torch_lib = _torch_lib_dir()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp),
           *[str(o) for o in objs], f"-L{torch_lib}", f"-Wl,-rpath,{torch_lib}",
           "-lamdhip64", "-pthread"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
