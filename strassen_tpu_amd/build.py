"""Build the gfx950 C-ABI library in-tree.

``python -m strassen_tpu_amd.build`` (or ``build()``) compiles the C ABI's
translation unit (``csrc/strassen_gemm.hip``) and the four units that
instantiate the GEMM kernels (``csrc/gemm_*.hip``) with hipcc, in parallel,
checks each unit's device assembly, and links ``libstrassen_mi355x.so`` next
to this file. hipcc cross-compiles for gfx950 without a GPU.
"""

from __future__ import annotations

import os
import re
from concurrent.futures import ThreadPoolExecutor
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
SOURCES = tuple(os.path.join(HERE, "csrc", name) for name in (
    "strassen_gemm.hip", "gemm_strassen.hip", "gemm_strassen_thin.hip", "gemm_strassen_pm.hip", "gemm_cubic.hip",
    "gemm_cubic_thin.hip"))
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


def compile_command(source, output, extra=()):
    """hipcc command compiling one translation unit to an object file."""
    return [
        hipcc_path(), "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-c",
        # Code object v5 is accepted by both the ROCm 7.0 runtime bundled with
        # torch and the system ROCm 7.2 runtime.
        "-mcode-object-version=5",
        # Packed FP32 VALU ops (v_pk_add_f32 and friends) stay disabled.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-I", INCLUDE, *extra, source, "-o", output,
    ]


def link_command(objects, output):
    return [hipcc_path(), "--offload-arch=gfx950", "-fPIC", "-shared", *objects, "-o", output]


# The pre-summed Strassen kernel issues its MFMAs through inline asm (to pin
# accumulators to AGPRs / VGPRs), so the compiler does not insert the wait
# states an MFMA result needs before a VALU, VMEM or v_accvgpr read. Such a
# kernel only reads accumulators after an explicit s_nop drain; any spill,
# AGPR copy or read the compiler places between the first MFMA and that
# drain would read a stale value. This check finds every kernel with an
# inline-asm MFMA and rejects such code.
_FUNCTION = re.compile(r"^(_Z\w+):", re.M)
_ASM_MFMA = re.compile(r";;#ASMSTART\s*\n\s*v_mfma")
_DRAIN = "s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
_CALL = re.compile(r"^\s*s_swappc_b64.*$", re.M)
_FORBIDDEN = re.compile(r"^\s*(scratch_\w+|buffer_store\w*|v_accvgpr_read\w*|v_accvgpr_mov\w*)\b", re.M)


def verify_inline_asm_kernels(asm_text):
    """Raise if a kernel with inline-asm MFMAs touches accumulators before its
    drain; returns the number of such kernels (at least one is expected)."""
    checked = 0
    labels = list(_FUNCTION.finditer(asm_text))
    for n, m in enumerate(labels):
        name = m.group(1)
        # The whole function, up to its end marker or the next function: a
        # kernel may end some waves (s_endpgm) before another wave's MFMA loop.
        end = asm_text.find(".Lfunc_end", m.end())
        if end < 0:
            end = len(asm_text)
        if n + 1 < len(labels):
            end = min(end, labels[n + 1].start())
        body = asm_text[m.end():end]
        if not _ASM_MFMA.search(body):
            continue
        checked += 1
        call = _CALL.search(body)
        if call:
            raise RuntimeError(f"{name}: calls a device function ({call.group(0).strip()}); the kernel's helpers "
                               "must inline, or their results turn divergent; refusing to build")
        if _DRAIN not in body:
            raise RuntimeError(f"{name}: inline-asm MFMAs without the drain sequence")
        # A kernel may hold several MFMA loops (one per wave role), each
        # ending in its own drain. In every stretch between drains, nothing
        # may read, copy or spill registers from the stretch's first MFMA to
        # the drain that ends it (before an MFMA no accumulator holds an MFMA
        # result yet); MFMAs after the last drain are refused.
        start = 0
        while True:
            first_mfma = body.find("v_mfma", start)
            if first_mfma < 0:
                break
            drain = body.find(_DRAIN, first_mfma)
            if drain < 0:
                raise RuntimeError(f"{name}: an MFMA after the last drain sequence")
            bad = _FORBIDDEN.search(body[first_mfma:drain])
            if bad:
                raise RuntimeError(f"{name}: '{bad.group(1)}' before the MFMA drain "
                                   "(accumulators spilled or copied); refusing to build")
            start = drain + len(_DRAIN)
    if not checked:
        raise RuntimeError("no inline-asm MFMA kernels found in the device assembly")
    return checked


# Scratch (private segment) per GEMM kernel, in bytes per lane. The Strassen
# kernels and the matched cubic keep their accumulators, fragments and
# addresses in registers: a spill there is reloaded on every tile, so the
# build refuses it. One exception carries a stated cap: the cubic that adds
# an FP32 partial product before its epilogue (the exact-panel path, off the
# hot path).
_KERNEL_DESC = re.compile(r"\.amdhsa_kernel (\S+)(.*?)\.end_amdhsa_kernel", re.S)
_SPLIT = re.compile(r"gemm_splitILi(\d+)ELi(\d+)ELb(\d)E")
_PM = re.compile(r"gemm_pmILi(\d+)EE")
_PACKED = re.compile(r"gemm_packedILi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELb(\d)E")
_QUAD_CUBIC_PARTIAL = 1
PARTIAL_SCRATCH_CAP = 1024


def scratch_limit(name):
    """Allowed scratch bytes per lane of a kernel (None: not a GEMM kernel)."""
    if _SPLIT.search(name) or _PM.search(name):
        return 0
    m = _PACKED.search(name)
    if m:
        return PARTIAL_SCRATCH_CAP if int(m.group(3)) == _QUAD_CUBIC_PARTIAL else 0
    return None


def verify_kernel_scratch(asm_text, require=True):
    """Raise if a GEMM kernel's private segment exceeds its limit; returns the
    number of GEMM kernels checked (with require, at least one)."""
    checked = 0
    for m in _KERNEL_DESC.finditer(asm_text):
        limit = scratch_limit(m.group(1))
        if limit is None:
            continue
        size = re.search(r"\.amdhsa_private_segment_fixed_size (\d+)", m.group(2))
        scratch = int(size.group(1)) if size else 0
        if scratch > limit:
            raise RuntimeError(f"{m.group(1)}: {scratch} bytes of scratch per lane (limit {limit}): "
                               "registers spill; refusing to build")
        checked += 1
    if require and not checked:
        raise RuntimeError("no GEMM kernel descriptors found in the device assembly")
    return checked


def _compile_unit(source, workdir):
    """Compiles one unit in its own directory (-save-temps keeps its device
    assembly); returns (object path, assembly text, compiler messages)."""
    os.makedirs(workdir)
    obj = os.path.join(workdir, os.path.basename(source).replace(".hip", ".o"))
    cmd = compile_command(source, obj, extra=("-save-temps",))
    result = subprocess.run(cmd, capture_output=True, text=True, cwd=workdir)
    noise = "packed-fp32-ops"
    stderr = "\n".join(l for l in result.stderr.splitlines() if noise not in l)
    if result.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + stderr)
    asm = [f for f in os.listdir(workdir) if f.endswith("gfx950.s")]
    if len(asm) != 1:
        raise RuntimeError(f"expected one gfx950 assembly file from -save-temps of {source}, found {asm}")
    with open(os.path.join(workdir, asm[0])) as f:
        return obj, f.read(), stderr


def build(verbose=False, jobs=None):
    """Compile the library; returns its path. Always recompiles."""
    tmp = LIBRARY + ".tmp"
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with tempfile.TemporaryDirectory() as scratch:
        dirs = [os.path.join(scratch, f"unit{i}") for i in range(len(SOURCES))]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            units = list(pool.map(_compile_unit, SOURCES, dirs))
        checked = gemms = 0
        for source, (_, text, stderr) in zip(SOURCES, units):
            if verbose and stderr.strip():
                print(stderr, file=sys.stderr)
            # The C ABI's unit holds the compact kernels and the packers; the
            # inline-asm MFMA kernels and the GEMM scratch limits live in the
            # kernel units, each of which must hold some.
            kernel_unit = os.path.basename(source) != "strassen_gemm.hip"
            if kernel_unit:
                checked += verify_inline_asm_kernels(text)
            gemms += verify_kernel_scratch(text, require=kernel_unit)
        cmd = link_command([obj for obj, _, _ in units], tmp)
        result = subprocess.run(cmd, capture_output=True, text=True, cwd=scratch)
        if result.returncode != 0:
            raise RuntimeError("link failed:\n" + " ".join(cmd) + "\n" + result.stderr)
    if verbose:
        print(f"verified {checked} inline-asm MFMA kernels and the scratch of {gemms} GEMM kernels", file=sys.stderr)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
