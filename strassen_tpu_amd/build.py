"""Build the gfx950 C-ABI library in-tree.

``python -m strassen_tpu_amd.build`` (or ``build()``) compiles
``csrc/strassen_gemm.hip`` with hipcc into ``libstrassen_mi355x.so`` next to
this file. hipcc cross-compiles for gfx950 without a GPU.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
SOURCE = os.path.join(HERE, "csrc", "strassen_gemm.hip")
LIBRARY = os.path.join(HERE, "libstrassen_mi355x.so")
INCLUDE = os.path.join(REPO, "include")


def hipcc_path():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    if os.path.exists(path):
        return path
    found = shutil.which("hipcc")
    if found is None:
        raise RuntimeError("hipcc not found: set ROCM_PATH or put hipcc on PATH")
    return found


def compile_command(output=LIBRARY, extra=()):
    return [
        hipcc_path(), "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
        # Code object v5 is accepted by both the ROCm 7.0 runtime bundled with
        # torch and the system ROCm 7.2 runtime.
        "-mcode-object-version=5",
        # Packed FP32 VALU ops (v_pk_add_f32 and friends) stay disabled.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", INCLUDE, *extra, SOURCE, "-o", output,
    ]


def build(verbose=False):
    """Compile the library; returns its path. Always recompiles."""
    tmp = LIBRARY + ".tmp"
    cmd = compile_command(tmp)
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    stderr = "\n".join(l for l in result.stderr.splitlines() if noise not in l)
    if result.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + stderr)
    if verbose and stderr.strip():
        print(stderr, file=sys.stderr)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
