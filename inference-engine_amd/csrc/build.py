"""Build the gfx950 shared library of the paged-KV hot path.

    python inference-engine_amd/csrc/build.py

compiles csrc/paged_kv.hip and csrc/fused.hip with hipcc for gfx950 into
lib/libpaged_kv.so (next to the engine package). The library links libamdhip64.so.7;
loaded after ``import torch`` it binds to the HIP runtime torch already loaded (same
SONAME), so torch's streams and device pointers are valid inside it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
REPO = os.path.dirname(PKG_ROOT)
LIB_DIR = os.path.join(PKG_ROOT, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libpaged_kv.so")
SOURCES = [os.path.join(HERE, "paged_kv.hip"), os.path.join(HERE, "fused.hip")]
INCLUDE = os.path.join(REPO, "include")

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Packed-FP32 VALU ops stay off: plain float code only.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]  # fmt: skip


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build the HIP library)")


def build(verbose: bool = False) -> str:
    """Compile every source into LIB_PATH (always recompiles) and return the path."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", *SOURCES, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    noise = "packed-fp32-ops"
    err = "\n".join(ln for ln in res.stderr.splitlines() if noise not in ln)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
