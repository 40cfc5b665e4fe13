"""Build libpagedkv.so for gfx950 from the HIP sources in ../csrc, and libpkhost.so (the
host-side serving core, plain C++) from ../csrc/pkhost.cpp.

Each .hip file is compiled to an object with hipcc (in parallel), then the objects
are linked into one shared library placed next to this file, where
``pagedkv._lib`` loads it; libpkhost.so is compiled with g++ and loaded by
``pagedkv._host``. The build always recompiles; there is no JIT cache.

    python -m pagedkv.build          # from the nano-vllm-diy_amd directory
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
ROOT = PKG_DIR.parent
CSRC = ROOT / "csrc"
INCLUDE = ROOT.parent / "include"
BUILD_DIR = ROOT / "_build"
LIB_NAME = "libpagedkv.so"
LIB_PATH = PKG_DIR / LIB_NAME
HOST_LIB_PATH = PKG_DIR / "libpkhost.so"
HOST_SRC = CSRC / "pkhost.cpp"
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU ops.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm")


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature; drop that line.
    noise = "-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l).strip()
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err and verbose:
        print(err, file=sys.stderr)
    return obj


def build_host(verbose: bool = False) -> Path:
    """Compile csrc/pkhost.cpp into libpkhost.so with the host C++ compiler."""
    cxx = os.environ.get("CXX") or shutil.which("g++") or "g++"
    tmp = HOST_LIB_PATH.with_name(HOST_LIB_PATH.name + f".tmp{os.getpid()}")
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", f"-I{INCLUDE}",
           str(HOST_SRC), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{cxx} failed on {HOST_SRC.name}:\n{res.stderr}")
    os.replace(tmp, HOST_LIB_PATH)
    return HOST_LIB_PATH


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libpagedkv.so (and build
    libpkhost.so); return the path of libpagedkv.so."""
    build_host(verbose)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB_PATH.with_name(LIB_NAME + f".tmp{os.getpid()}")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
