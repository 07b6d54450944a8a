"""Build libgqa_hip.so (the C-ABI of include/gqa_attn.h) in-tree for gfx950.

Usage: python gqa-flash-attn-rtx3060_amd/build.py [-v]

Each csrc/*.hip file is compiled to an object in parallel, then linked into
gqa_kernels/libgqa_hip.so next to the Python package that loads it; then
csrc/host/gqa_host.cpp (the torch-tensor binding of the decode call) is
built into gqa_kernels/_gqa_host.so against it.  The
build always runs (no up-to-date check): callers that need the library to
match the sources call this after every source change.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
OBJ_DIR = PKG_ROOT / "_build"
LIB_PATH = PKG_ROOT / "gqa_kernels" / "libgqa_hip.so"
HOST_PATH = PKG_ROOT / "gqa_kernels" / "_gqa_host.so"

ARCH = "gfx950"
# -packed-fp32-ops: keep hipcc from emitting v_pk_{add,mul,fma}_f32.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{REPO_ROOT / 'include'}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP kernels)")
    return found


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only target feature; that is harmless.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [OBJ_DIR / (s.stem + ".o") for s in sources]

    def compile_one(pair):
        src, obj = pair
        _run([hipcc, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)], verbose)

    with ThreadPoolExecutor(max_workers=min(len(sources), os.cpu_count() or 4)) as ex:
        list(ex.map(compile_one, zip(sources, objs)))

    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)], verbose)
    os.replace(tmp, LIB_PATH)
    build_host(verbose)
    return LIB_PATH


def build_host(verbose: bool = False) -> Path:
    """The torch-tensor binding of the decode call (csrc/host/gqa_host.cpp):
    host-only C++ built with g++ against torch's headers, linked to
    libgqa_hip.so beside it (rpath $ORIGIN), as gqa_kernels/_gqa_host.so."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    src = CSRC / "host" / "gqa_host.cpp"
    tmp = HOST_PATH.with_suffix(".so.tmp")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O3", "-std=c++17", "-fPIC", "-shared", str(src), "-o", str(tmp),
           f"-I{REPO_ROOT / 'include'}", f"-I{sysconfig.get_paths()['include']}",
           *[f"-I{p}" for p in cpp_extension.include_paths()],
           f"-I{os.environ.get('ROCM_PATH', '/opt/rocm')}/include",
           # the HIP runtime headers, included through torch's, select the
           # AMD platform from this macro when not compiled by hipcc
           "-D__HIP_PLATFORM_AMD__", "-DTORCH_EXTENSION_NAME=_gqa_host", "-DTORCH_API_INCLUDE_EXTENSION_H",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-L{p}" for p in cpp_extension.library_paths()], "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-ltorch_python", f"-L{LIB_PATH.parent}", "-lgqa_hip", "-Wl,-rpath,$ORIGIN"]
    _run(cmd, verbose)
    os.replace(tmp, HOST_PATH)
    return HOST_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(f"built {path}")
