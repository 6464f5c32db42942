"""Builds ``libddpm_hip.so`` in-tree from ``csrc/*.hip`` with hipcc for gfx950.

Usage: ``python -m dynamicconvolutionoperator_amd.build`` (or ``build()``).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libddpm_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
OBJ_DIR = os.path.join(HERE, "_build")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # ROCm 7.0's runtime (bundled with the torch wheel) loads code object v5
    "-mcode-object-version=5",
    # keep packed fp32 instructions out of the device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *FLAGS, "-I", CSRC, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def _undefined_library_symbols(path: str) -> list[str]:
    """Undefined dynamic symbols of `path` in this library's namespace (needs nm)."""
    nm = shutil.which("nm")
    if nm is None:
        return []
    res = subprocess.run([nm, "-D", "--undefined-only", path], capture_output=True, text=True)
    return [ln.split()[-1] for ln in res.stdout.splitlines() if "ddpm" in ln]


def build(verbose: bool = False) -> str:
    """Compile every csrc/*.hip for gfx950 and link libddpm_hip.so (always rebuilds)."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc link failed:\n{res.stderr}")
    # a kernel whose host stub the compiler failed to emit shows up only as an
    # undefined symbol at load time: refuse to install such a library
    undefined = _undefined_library_symbols(tmp)
    if undefined:
        os.remove(tmp)
        raise RuntimeError("libddpm_hip.so references undefined library symbols:\n  " + "\n  ".join(undefined))
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


def clean() -> None:
    shutil.rmtree(OBJ_DIR, ignore_errors=True)
    if os.path.exists(LIB_PATH):
        os.remove(LIB_PATH)


if __name__ == "__main__":
    build(verbose=True)
