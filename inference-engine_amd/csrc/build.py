"""Build the gfx950 shared library of the paged-KV hot path.

    python inference-engine_amd/csrc/build.py

compiles csrc/kv_ops.hip, csrc/decode.hip, csrc/prefill.hip, csrc/cascade.hip (sharing
csrc/common.h and the kernel headers) and csrc/fused.hip with hipcc for gfx950 into
lib/libpaged_kv.so (next to the engine
package). The library links libamdhip64.so.7;
loaded after ``import torch`` it binds to the HIP runtime torch already loaded (same
SONAME), so torch's streams and device pointers are valid inside it.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
REPO = os.path.dirname(PKG_ROOT)
LIB_DIR = os.path.join(PKG_ROOT, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libpaged_kv.so")
SOURCES = [os.path.join(HERE, f) for f in ("kv_ops.hip", "decode.hip", "prefill.hip", "cascade.hip", "fused.hip")]
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


def _run(cmd: list[str]) -> subprocess.CompletedProcess:
    return subprocess.run(cmd, capture_output=True, text=True)


def build(verbose: bool = False) -> str:
    """Compile every source into LIB_PATH (always recompiles; the sources in parallel,
    then one link) and return the path."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    noise = "packed-fp32-ops"
    compile_flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    with tempfile.TemporaryDirectory() as objdir:
        objs = [os.path.join(objdir, os.path.basename(src) + ".o") for src in SOURCES]
        cmds = [[hipcc(), *compile_flags, f"-I{INCLUDE}", "-c", src, "-o", obj]
                for src, obj in zip(SOURCES, objs, strict=True)]  # fmt: skip
        cmds.append([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp])
        with concurrent.futures.ThreadPoolExecutor(len(SOURCES)) as pool:
            results = list(pool.map(_run, cmds[:-1]))
        results.append(_run(cmds[-1]) if all(r.returncode == 0 for r in results) else None)
        for cmd, res in zip(cmds, results, strict=True):
            if res is None:
                continue
            if verbose:
                print(" ".join(cmd), flush=True)
            err = "\n".join(ln for ln in res.stderr.splitlines() if noise not in ln)
            if res.returncode != 0:
                raise RuntimeError(f"hipcc failed ({res.returncode}):\n{err}")
            if verbose and err.strip():
                print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
