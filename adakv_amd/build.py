"""Compile libadakv_amd.so (the C-ABI HIP library) in-tree for gfx950.

    python -m adakv_amd.build [-v]

Each HIP translation unit is compiled in parallel with hipcc, then linked into
``adakv_amd/_lib/libadakv_amd.so``.  Packed-fp32 instruction selection is
disabled (``-Xclang -target-feature -Xclang -packed-fp32-ops``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
OUT_DIR = os.path.join(PKG, "_lib")
BUILD_DIR = os.path.join(PKG, "_build")
LIB_NAME = "libadakv_amd.so"
SOURCES = ["centroid.hip", "plan.hip", "minmax.hip", "decode.hip", "fused.hip", "evict.hip", "capi.hip"]
ARCH = os.environ.get("ADAKV_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
    f"-I{INCLUDE}", f"-I{CSRC}",
]

# Per-source additions.  The fused step keeps its matrix-core accumulators in
# ordinary VGPRs: with the default heuristic they live in AGPRs, and the
# online-softmax rescale between tiles then copies all of them out and back.
EXTRA_FLAGS = {
    "fused.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "decode.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def flags_for(src: str) -> list:
    return [*FLAGS, *EXTRA_FLAGS.get(src, [])]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the AdaKV HIP library cannot be built")


def lib_path() -> str:
    return os.path.join(OUT_DIR, LIB_NAME)


def build(verbose: bool = False) -> str:
    """Compile every source and link the shared library; returns its path."""
    cc = hipcc()
    os.makedirs(OUT_DIR, exist_ok=True)
    os.makedirs(BUILD_DIR, exist_ok=True)

    def compile_one(src: str) -> str:
        obj = os.path.join(BUILD_DIR, src.replace(".hip", ".o"))
        cmd = [cc, *flags_for(src), "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
        if verbose and r.stderr.strip():
            print(r.stderr, flush=True)
        return obj

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = lib_path() + ".tmp"
    cmd = [cc, "-shared", f"--offload-arch={ARCH}", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, lib_path())
    return lib_path()


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
