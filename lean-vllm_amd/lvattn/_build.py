"""Builds ``liblvattn.so`` (the C-ABI library of HIP kernels for gfx950) in-tree with hipcc.

Each source compiles separately (in parallel), then one link. The library lands next to this file, where
``lvattn._capi`` loads it. ``python -m lvattn._build`` runs it from the command line.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR.parent / "csrc"
INCLUDE = PACKAGE_DIR.parent.parent / "include"
LIBRARY = PACKAGE_DIR / "liblvattn.so"
BUILD_DIR = PACKAGE_DIR.parent / "_build"
SOURCES = ("capi.hip", "store.hip", "pack.hip", "paged_attention.hip", "merge.hip", "mla_decode.hip", "varlen.hip")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the lvattn kernels need ROCm's hipcc to build")


def compile_flags(debug: bool = False) -> list[str]:
    flags = [
        f"--offload-arch={ARCH}",
        "-std=c++17",
        "-fPIC",
        "-O3",
        f"-I{INCLUDE}",
        f"-I{CSRC}",
        # Packed fp32 VALU forms are kept out of the code object.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
    ]
    if debug:
        flags += ["-g"]
    return flags


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source and link ``liblvattn.so``; returns its path. Always rebuilds."""
    cc = hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = [CSRC / s for s in SOURCES if (CSRC / s).exists()]
    objects = [BUILD_DIR / (s.stem + ".o") for s in sources]

    def compile_one(pair):
        src, obj = pair
        cmd = [cc, *compile_flags(), "-c", str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stderr[-4000:]}")
        if verbose:
            print(f"compiled {src.name}", flush=True)

    with ThreadPoolExecutor(max_workers=jobs or min(8, len(sources))) as pool:
        list(pool.map(compile_one, zip(sources, objects)))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of liblvattn.so failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}", flush=True)
    build_host_stage(verbose)
    return LIBRARY


def build_host_stage(verbose: bool = False) -> Path:
    """Compile the CPython extension that lays the packing inputs out on the host (``lvattn._hoststage``)."""
    cxx = shutil.which("g++") or shutil.which("c++")
    if not cxx:
        raise RuntimeError("g++ not found; lvattn._hoststage needs a host C++ compiler")
    out = PACKAGE_DIR / ("_hoststage" + sysconfig.get_config_var("EXT_SUFFIX"))
    tmp = out.with_suffix(".tmp")
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", f"-I{sysconfig.get_paths()['include']}",
           str(CSRC / "host_stage.cpp"), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed on host_stage.cpp:\n{res.stderr[-4000:]}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}", flush=True)
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
