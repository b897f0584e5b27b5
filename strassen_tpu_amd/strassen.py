"""Drop-in surface of the reference's ``strassen_pallas`` GEMM path on gfx950.

``strassen_matmul`` keeps the keyword surface, argument meaning and error
messages of ``strassen_pallas.strassen_matmul`` (``strassen_pallas.py:882-1221``)
and runs the hand-written HIP kernel in ``csrc/strassen_gemm.hip`` through
the C ABI of ``include/strassen_mi355x.h``. Tensors are torch bf16 or
float32 tensors on the HIP device; the result is a new tensor of the input
dtype (or ``output_dtype``), computed asynchronously on torch's current
stream.

Differences a caller can observe, all raised as exceptions (never silent):

* FP32 inputs run the DEFAULT-precision product (the ``jnp.dot`` of
  ``strassen_pallas.py:228-232`` at its default ``dot_precision``, ``:889``,
  which makes one bf16 pass on a TPU): the packing pass forms each
  operand sum in float and rounds it once to bf16, and every product is one
  bf16 MFMA pass into FP32. ``dot_precision`` HIGH / HIGHEST run the 3- and
  6-pass bf16 products: the packing pass splits each float operand into
  bf16 parts (p0 = bf16(v), p1 = bf16(v - p0), p2 = bf16(v - p0 - p1)) and
  lays the pass pairs out along K pass-major, smallest products first
  ([p2 p0, p1 p1, p0 p2,] p1 p0, p0 p1, p0 p0), so one GEMM over 3K or 6K
  sums them in FP32 with the leading pass added last. How XLA orders and
  rounds these passes on a TPU is not visible here; the pass pairs are those
  of its published bf16_3x / bf16_6x algorithms. RoPE tables are read as
  bf16 (a float32 table is rounded once on the host).
* The exact-panel policies (``classical_panels``, ``panel_schedule``) run as
  two GEMMs: Strassen over the ordinary K panels into an FP32 partial, then
  the matched cubic over the exact panels, which adds the partial before
  the epilogue. Operands are ``SplitOperand`` s packed with the call's
  schedule (a plain weight is split for the call); a schedule held on the
  device is read back once per call. ``panel_schedule`` with the powers
  formula raises ``ValueError`` (the reference would add raw quadrant
  products into its encoded basis).
* ``norm_residual_add`` runs as the GEMM with an FP32 result followed by a
  row-norm pass (one bf16 rounding, as in the reference). So does
  ``qk_norm_rope`` for a ``rope_head_dim`` other than 128 (the fused q/k
  epilogue's head width), followed by a per-head norm and RoPE pass.
* ``formula_variant`` "dual" / "powers" and ``block_permutation`` run on
  packed operands: a plain weight is packed for the call (pack it once with
  ``strassen_weight_layout(..., formula_variant=, block_permutation=)``).
* TPU-only knobs (``allow_input_fusion`` after its validation,
  ``vmem_limit_bytes``) are accepted and have no effect, as is
  ``dot_precision`` for bf16 inputs (bf16 operands have no low-order part);
  ``interpret=True`` raises ``NotImplementedError`` (there is no CPU path).
* The kernel keeps seven persistent FP32 product accumulators and combines
  the quadrants once after the last K panel, so ``interleave_products`` and
  the ``product_aware_*`` schedules (which only reorder FP32 additions in
  the reference) are validated and accepted but select the same kernel.
* Every tile the reference's ``check_tiling`` accepts runs (bm % 16, bn % 256,
  bk % 256): the packed kernels take bm % 16, bn % 256, bk % 64. A bm whose
  half is not a multiple of 128 (decode-sized M, for one) runs their
  thin-tiling instantiations, which map output rows one by one. The compact
  kernel (``plain_weight_kernel("compact")``) needs bm % 256 and takes
  bn % 128; a tile it cannot take runs packed.
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import warnings

import numpy as np
import torch

from . import _lib
from .layouts import is_k_contiguous
from .packing import (PackedOperand, SplitOperand, exact_schedule, pack_operand, pack_weight_for_call,
                      packed_weight_cache_info, precision_passes)

__all__ = [
    "strassen_matmul", "strassen_matmul_lhs_transposed", "cubic_matmul", "native_matmul", "check_tiling",
    "TUNED_BM", "TUNED_BN", "TUNED_BK", "VMEM_PROFILE", "PROFILE_INFO", "plain_weight_kernel", "strassen_kernel",
]

LANE = 128
SUBLANE = 8

# The reference's default tile (``compact16``, strassen_pallas.py:20-24).
TUNED_BM, TUNED_BN, TUNED_BK = 1024, 1024, 512
VMEM_PROFILE = "compact16"
PROFILE_INFO = {
    "profile": VMEM_PROFILE,
    "tile": (TUNED_BM, TUNED_BN, TUNED_BK),
    "device": "gfx950",
}

_EPILOGUES = ("swiglu", "geglu", "residual_add", "bias_add", "qk_norm_rope", "norm_residual_add")


def check_tiling(bm, bn, bk):
    """The reference's alignment rule (``strassen_pallas.py:127-140``)."""
    requirements = (
        ("bm", bm, 2 * SUBLANE),
        ("bn", bn, 2 * LANE),
        ("bk", bk, 2 * LANE),
    )
    errors = [
        f"{name}={value} must be a multiple of {multiple}"
        for name, value, multiple in requirements
        if value % multiple
    ]
    if errors:
        raise ValueError("tile breaks TPU v5e alignment:\n  " + "\n  ".join(errors))


def _check_device_tiling(algo, epilogue, bm, bn, bk, b_layout):
    tm, tn, tk = _lib.tile_requirements(algo, epilogue, b_layout)
    errors = [
        f"{name}={value} must be a multiple of {multiple}"
        for name, value, multiple in (("bm", bm, 2 * tm), ("bn", bn, 2 * tn), ("bk", bk, 2 * tk))
        if value % multiple
    ]
    if errors:
        raise ValueError("tile breaks the gfx950 kernel tiling:\n  " + "\n  ".join(errors))


# Kernel for a plain (unpacked) weight: "pack" packs both operands for the
# call and runs the packed kernel whenever the tile suits it (the packing
# passes are bandwidth-bound and far cheaper than the compact kernel's
# in-register operand sums); "compact" always runs the compact kernel.
# SMX_PLAIN_WEIGHTS sets the default; plain_weight_kernel() switches it.
PLAIN_WEIGHTS = os.environ.get("SMX_PLAIN_WEIGHTS", "pack")


@contextlib.contextmanager
def plain_weight_kernel(kind):
    """Run plain-weight calls inside the block on ``kind`` ("pack" or
    "compact"). Process-wide; not for concurrent use."""
    global PLAIN_WEIGHTS
    if kind not in ("pack", "compact"):
        raise ValueError("plain-weight kernel must be 'pack' or 'compact'")
    previous, PLAIN_WEIGHTS = PLAIN_WEIGHTS, kind
    try:
        yield
    finally:
        PLAIN_WEIGHTS = previous


# Strassen kernel for packed operands: "split" (the seven products of a
# 128 x 128 product tile in registers, gemm_split), "product_major" (the
# products of a 128 x 256 tile one after another into three register sets,
# SMX_FLAG_PRODUCT_MAJOR; calls that kernel cannot take run "split") or
# "product_major_rounds" (the product-major kernel on the leading tile
# columns that fill whole rounds of the CUs, "split" on the rest,
# SMX_FLAG_PRODUCT_MAJOR_ROUNDS). The default is "product_major_rounds":
# on whole rounds the product-major kernel does the same work in 2-10% less
# time than "split" (most where the packed operands overflow the MALL), but
# its last, partly filled round runs as long as a full one, which the split
# kernel's K split avoids; calls with no whole round of its tiles run
# "split" alone. Its head parks 256 KB per product-major tile in the call's
# workspace.
STRASSEN_KERNELS = ("split", "product_major", "product_major_rounds")
STRASSEN_KERNEL = "product_major_rounds"


@contextlib.contextmanager
def strassen_kernel(kind):
    """Run packed Strassen calls inside the block on ``kind`` (one of
    STRASSEN_KERNELS). Process-wide; not for concurrent use."""
    global STRASSEN_KERNEL
    if kind not in STRASSEN_KERNELS:
        raise ValueError(f"Strassen kernel must be one of {STRASSEN_KERNELS}")
    previous, STRASSEN_KERNEL = STRASSEN_KERNEL, kind
    try:
        yield
    finally:
        STRASSEN_KERNEL = previous


def _fits(algo, epilogue, bm, bn, bk, b_layout):
    tm, tn, tk = _lib.tile_requirements(algo, epilogue, b_layout)
    return bm % (2 * tm) == 0 and bn % (2 * tn) == 0 and bk % (2 * tk) == 0


def _fits_packed(algo, epilogue, bm, bn, bk):
    return _fits(algo, epilogue, bm, bn, bk, _lib.SMX_B_PACKED)


class PlainWeightPackWarning(UserWarning):
    """A call packed an ordinary weight for itself (no packed-weight cache)."""


_PLAIN_PACK_WARNED = False
_PLAIN_PACK_EXPECTED = 0


@contextlib.contextmanager
def per_call_packing_expected():
    """Calls inside pack plain weights per call on purpose (a measurement of
    that cost): they neither warn nor use up the once-per-process warning."""
    global _PLAIN_PACK_EXPECTED
    _PLAIN_PACK_EXPECTED += 1
    try:
        yield
    finally:
        _PLAIN_PACK_EXPECTED -= 1


def _plain_weight(b, **packing):
    """The packed form of a plain weight for one call (through the
    packed-weight cache when enabled). The first per-call pack of a process
    without a cache warns once: it repeats on every call."""
    global _PLAIN_PACK_WARNED
    if (not _PLAIN_PACK_WARNED and not _PLAIN_PACK_EXPECTED
            and packed_weight_cache_info()["capacity"] <= 0):
        _PLAIN_PACK_WARNED = True
        warnings.warn("a plain weight is packed on every call (a Strassen weight packs to 7/4 of its bytes): "
                      "pack it once with strassen_weight_layout / cubic_weight_layout, or keep packed weights "
                      "with cache_packed_weights(capacity_bytes)", PlainWeightPackWarning, stacklevel=4)
    return pack_weight_for_call(b, **packing)


# Head width of the fused q/k epilogue: a head's half (64 columns) is two of
# the kernels' 32-column accumulator blocks. Other widths run the GEMM with an
# FP32 result and the per-head pass smx_qk_norm_rope.
FUSED_QK_HEAD_DIM = 128


def _is_dtype(x, dtype):
    return x.dtype == dtype


def _check_epilogue_name(epilogue):
    if epilogue not in _EPILOGUES:
        raise ValueError(
            f"unknown epilogue {epilogue!r}; choose 'swiglu' or "
            "'residual_add' or 'bias_add'")


def _check_epilogue_operands(m, n, bn, *, epilogue, residual, bias, rope_cos, rope_sin, rope_scale,
                             rope_head_dim, norm_scale):
    """Presence, pairing and shapes of the epilogue operands for an [m, n]
    output (the checks of ``strassen_pallas.py:927-1047`` that concern
    them). The kernels read these operands by address only, so both the
    Strassen and the cubic entry run these checks before any launch."""
    if epilogue in ("swiglu", "geglu") and bn % 2:
        raise ValueError(f"{epilogue} epilogue needs an even bn, got {bn}")
    if epilogue == "residual_add" and residual is None:
        raise ValueError("residual_add epilogue requires residual=")
    if epilogue == "bias_add" and bias is None:
        raise ValueError("bias_add epilogue requires bias=")
    if residual is not None and epilogue not in ("residual_add", "norm_residual_add"):
        raise ValueError(
            "residual= is only used by the residual_add and "
            "norm_residual_add epilogues")
    if bias is not None and epilogue != "bias_add":
        raise ValueError("bias= is only used by the bias_add epilogue")
    if epilogue == "norm_residual_add":
        if residual is None or norm_scale is None:
            raise ValueError("norm_residual_add requires residual= and norm_scale=")
        if bn != n:
            raise ValueError(
                "norm_residual_add normalises over the whole output row, so "
                f"the tile must span it: bn={bn} must equal n={n}")
        if tuple(residual.shape) != (m, n):
            raise ValueError(f"residual shape {tuple(residual.shape)} != output {(m, n)}")
        if tuple(norm_scale.shape) != (n,):
            raise ValueError(f"norm_scale shape {tuple(norm_scale.shape)} != output width {(n,)}")
    if epilogue == "qk_norm_rope":
        if rope_cos is None or rope_sin is None or rope_scale is None:
            raise ValueError(
                "qk_norm_rope epilogue requires rope_cos=, rope_sin= and "
                "rope_scale= (use rope_layout_tables and rope_scale_layout)")
        if bn % (2 * rope_head_dim):
            raise ValueError(
                f"qk_norm_rope needs bn a multiple of 2*head_dim="
                f"{2 * rope_head_dim} so a tile half holds whole heads, "
                f"got bn={bn}")
        if tuple(rope_cos.shape) != (m, bn // 2) or tuple(rope_sin.shape) != (m, bn // 2):
            raise ValueError(
                f"rope tables must be {(m, bn // 2)}, got "
                f"{tuple(rope_cos.shape)} and {tuple(rope_sin.shape)}")
        if tuple(rope_scale.shape) != (bn,):
            raise ValueError(
                f"rope_scale must be laid out to {(bn,)}, got "
                f"{tuple(rope_scale.shape)}")
    if rope_cos is not None and epilogue != "qk_norm_rope":
        raise ValueError("rope_* are only used by the qk_norm_rope epilogue")
    if epilogue == "bias_add" and tuple(bias.shape) != (n,):
        raise ValueError(f"bias shape {tuple(bias.shape)} != output width {(n,)}")
    if epilogue == "residual_add" and tuple(residual.shape) != (m, n):
        raise ValueError(f"residual shape {tuple(residual.shape)} != output shape {(m, n)}")


def _validate(a, b, *, bm, bn, bk, block_permutation, formula_variant,
              classical_panels, panel_schedule, epilogue, residual, bias,
              rope_cos, rope_sin, rope_scale, rope_head_dim, norm_scale,
              output_dtype, allow_input_fusion, product_aware_swiglu,
              product_aware_residual):
    """Argument checks in the order and wording of ``strassen_pallas.py:927-1047``."""
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError("strassen_matmul expects two rank-2 matrices")
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError(f"inner dimensions disagree: {k} vs {k2}")
    if a.dtype != b.dtype:
        raise ValueError(f"input dtypes disagree: {a.dtype} vs {b.dtype}")
    if a.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("inputs must be BF16 or FP32")
    if not isinstance(block_permutation, int) or not 0 <= block_permutation < 8:
        raise ValueError("block_permutation must be an integer from 0 through 7")
    if formula_variant not in ("classical", "dual", "powers"):
        raise ValueError("formula_variant must be 'classical', 'dual', or 'powers'")
    classical_panels = tuple(sorted({int(p) for p in classical_panels}))
    if epilogue is not None:
        _check_epilogue_name(epilogue)
        if formula_variant == "powers":
            raise ValueError("fused epilogues require a quadrant-basis formula")
        if output_dtype is not None and output_dtype != torch.bfloat16:
            raise ValueError("fused epilogues write a BF16 output tile")
    _check_epilogue_operands(m, n, bn, epilogue=epilogue, residual=residual, bias=bias, rope_cos=rope_cos,
                             rope_sin=rope_sin, rope_scale=rope_scale, rope_head_dim=rope_head_dim,
                             norm_scale=norm_scale)
    if product_aware_swiglu and epilogue not in ("swiglu", "geglu"):
        raise ValueError(
            "product_aware_swiglu is only valid with epilogue='swiglu' or 'geglu'")
    if product_aware_residual and epilogue != "residual_add":
        raise ValueError(
            "product_aware_residual is only valid with epilogue='residual_add'")
    operand_count = 3 if epilogue in ("residual_add", "bias_add") else 2
    if epilogue == "norm_residual_add":
        operand_count = 4
    if epilogue == "qk_norm_rope":
        operand_count = 6
    if allow_input_fusion is not None:
        allow_input_fusion = tuple(allow_input_fusion)
        if len(allow_input_fusion) != operand_count:
            raise ValueError(
                "allow_input_fusion must contain one boolean per operand: "
                f"expected {operand_count}, got {len(allow_input_fusion)}")
        if not all(isinstance(value, bool) for value in allow_input_fusion):
            raise TypeError("allow_input_fusion entries must be bool")
    if panel_schedule is not None and classical_panels:
        raise ValueError(
            "pass either classical_panels (static) or panel_schedule "
            "(prefetched), not both")
    if classical_panels:
        if formula_variant == "powers":
            raise ValueError("classical_panels requires a quadrant-basis formula")
        if classical_panels[0] < 0 or classical_panels[-1] >= k // bk:
            raise ValueError(f"classical_panels {classical_panels} outside 0..{k // bk - 1}")
    for name, dimension, block in (("M", m, bm), ("N", n, bn), ("K", k, bk)):
        if dimension % block:
            raise ValueError(f"{name}={dimension} is not divisible by {block}")
    check_tiling(bm, bn, bk)
    out = a.dtype if output_dtype is None else output_dtype
    if out not in (torch.bfloat16, torch.float32):
        raise ValueError("output_dtype must be BF16 or FP32")
    nk = k // bk
    if panel_schedule is not None:
        # strassen_pallas.py:1079-1090
        if epilogue is not None:
            raise ValueError("panel_schedule does not support fused epilogues")
        shape = tuple(panel_schedule.shape) if hasattr(panel_schedule, "shape") else np.shape(panel_schedule)
        if shape != (nk,):
            raise ValueError(f"panel_schedule must have shape ({nk},), got {shape}")
        if formula_variant == "powers":
            raise ValueError("panel_schedule requires a quadrant-basis formula")
    # The kernel's product-aware checks (strassen_pallas.py:299-322).
    if product_aware_swiglu and (formula_variant != "classical" or block_permutation != 0
                                 or (nk - 1) in classical_panels or panel_schedule is not None):
        raise ValueError(
            "product-aware SwiGLU requires unpermuted classical Strassen "
            "with quadrant accumulators; exact panels are allowed except on "
            "the final K panel, whose product order the schedule owns")
    if product_aware_residual and (formula_variant != "classical" or block_permutation != 0
                                   or (nk - 1) in classical_panels or panel_schedule is not None):
        raise ValueError(
            "product-aware residual requires unpermuted classical Strassen "
            "with quadrant accumulators and the residual_add epilogue; exact "
            "panels are allowed except on the final K panel")
    return m, k, n, classical_panels, out


def _unsupported(dtype, interpret, dot_precision=None):
    if interpret:
        raise NotImplementedError("interpret=True: the gfx950 kernel has no CPU interpreter path")
    precision_passes(dot_precision, dtype)  # an unknown precision raises here


def _require_device(*tensors):
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError("the gfx950 kernel needs tensors on the HIP device "
                             f"(got a tensor on {t.device})")


def _check_passes(x, name, passes):
    if x.passes != passes:
        raise ValueError(f"{name} was packed for {x.passes} bf16 pass(es) per product; the call's dot_precision "
                         f"needs {passes} (pack it with the call's dot_precision)")


def _check_packed(x, algo, side, tile_rows, bk, formula="classical", block_permutation=0, passes=1):
    name = "a" if side == "lhs" else "b"
    _check_passes(x, name, passes)
    if x.algo != algo or x.side != side:
        raise ValueError(f"{name} was packed as {x!r}, not as the {side} of this algorithm")
    if (x.tile_rows, x.bk) != (tile_rows, bk):
        raise ValueError(f"{name} was packed for the tile ({x.tile_rows}, bk={x.bk}), "
                         f"called with ({tile_rows}, bk={bk})")
    if (x.formula, x.block_permutation) != (formula, block_permutation):
        raise ValueError(f"{name} was packed for formula_variant={x.formula!r}, "
                         f"block_permutation={x.block_permutation}; called with "
                         f"formula_variant={formula!r}, block_permutation={block_permutation}")
    if x.schedule is not None:
        raise ValueError(f"{name} was packed for the exact panels {x.schedule.exact}; called without exact "
                         "panels")


def _aux_tensor(x):
    """An epilogue operand as bf16 or float32 (other dtypes become float32,
    as the reference casts them to float32 in the kernel)."""
    return x if x.dtype in (torch.bfloat16, torch.float32) else x.to(torch.float32)


def _norm_residual_add(algo, a, b, *, residual, norm_scale, norm_eps, **kw):
    """``norm_residual_add`` (``strassen_pallas.py:836-866``) in two passes:
    the GEMM stores its FP32 result, then ``smx_norm_residual_add`` applies
    the row RMSNorm, the scale and the residual with one bf16 rounding (the
    row's sum of squares spans every column tile of the output)."""
    out_dtype = kw.pop("out_dtype", torch.bfloat16)
    product = _run(algo, a, b, out_dtype=torch.float32, **kw)
    m, n = product.shape
    _require_device(residual, norm_scale)
    residual = _aux_tensor(residual)
    if residual.stride(1) != 1:
        residual = residual.contiguous()
    scale = _aux_tensor(norm_scale.contiguous())
    out = torch.empty((m, n), dtype=out_dtype, device=product.device)
    dtypes = ((_lib.SMX_NRA_SCALE_F32 if scale.dtype == torch.float32 else 0)
              | (_lib.SMX_NRA_RESIDUAL_F32 if residual.dtype == torch.float32 else 0)
              | (_lib.SMX_NRA_OUT_F32 if out_dtype == torch.float32 else 0))
    stream = torch.cuda.current_stream(product.device).cuda_stream
    rc = _lib.load().smx_norm_residual_add(m, n, _lib.ptr(product), product.stride(0), _lib.ptr(residual),
                                           residual.stride(0), _lib.ptr(scale), dtypes,
                                           float(norm_eps), _lib.ptr(out), out.stride(0), stream)
    _lib.check(rc)
    return out


def _qk_norm_rope(algo, a, b, *, rope_cos, rope_sin, rope_scale, rope_head_dim, rope_eps, **kw):
    """``qk_norm_rope`` (``strassen_pallas.py:793-835``) for head widths the
    fused epilogue does not take, in two passes: the GEMM stores its FP32
    result, then ``smx_qk_norm_rope`` applies each head's RMSNorm (over its
    columns in both tile halves) and the rotation, rounding once."""
    out_dtype = kw.pop("out_dtype", torch.bfloat16)
    product = _run(algo, a, b, out_dtype=torch.float32, **kw)
    m, n = product.shape
    _require_device(rope_cos, rope_sin, rope_scale)
    cos = rope_cos.to(torch.bfloat16).contiguous()
    sin = rope_sin.to(torch.bfloat16).contiguous()
    scale = _aux_tensor(rope_scale.contiguous())
    out = torch.empty((m, n), dtype=out_dtype, device=product.device)
    dtypes = ((_lib.SMX_QK_SCALE_F32 if scale.dtype == torch.float32 else 0)
              | (_lib.SMX_QK_OUT_F32 if out_dtype == torch.float32 else 0))
    stream = torch.cuda.current_stream(product.device).cuda_stream
    rc = _lib.load().smx_qk_norm_rope(m, n, _lib.ptr(product), product.stride(0), _lib.ptr(cos), _lib.ptr(sin),
                                      _lib.ptr(scale), dtypes, kw["bn"], rope_head_dim, float(rope_eps),
                                      _lib.ptr(out), out.stride(0), stream)
    _lib.check(rc)
    return out


def _run(algo, a, b, *, bm, bn, bk, epilogue=None, residual=None, bias=None,
         rope_cos=None, rope_sin=None, rope_scale=None, rope_head_dim=128,
         rope_eps=1e-6, out_dtype=torch.bfloat16, formula="classical", block_permutation=0,
         norm_scale=None, norm_eps=1e-6, schedule=None, partial=None, dot_precision=None):
    if epilogue == "qk_norm_rope" and rope_head_dim != FUSED_QK_HEAD_DIM:
        return _qk_norm_rope(algo, a, b, rope_cos=rope_cos, rope_sin=rope_sin, rope_scale=rope_scale,
                             rope_head_dim=rope_head_dim, rope_eps=rope_eps, bm=bm, bn=bn, bk=bk,
                             out_dtype=out_dtype, formula=formula, block_permutation=block_permutation,
                             schedule=schedule, partial=partial, dot_precision=dot_precision)
    if epilogue == "norm_residual_add":
        return _norm_residual_add(algo, a, b, residual=residual, norm_scale=norm_scale, norm_eps=norm_eps,
                                  bm=bm, bn=bn, bk=bk, formula=formula, block_permutation=block_permutation,
                                  schedule=schedule, out_dtype=out_dtype, dot_precision=dot_precision)
    if schedule is not None:
        return _run_split(a, b, bm=bm, bn=bn, bk=bk, schedule=schedule, formula=formula,
                          block_permutation=block_permutation, epilogue=epilogue, residual=residual, bias=bias,
                          rope_cos=rope_cos, rope_sin=rope_sin, rope_scale=rope_scale,
                          rope_head_dim=rope_head_dim, rope_eps=rope_eps, out_dtype=out_dtype,
                          dot_precision=dot_precision)
    lib = _lib.load()
    m, k = a.shape
    n = b.shape[1]
    # bf16 passes per product: the packed operands hold passes * k columns
    passes = precision_passes(dot_precision, a.dtype)
    variant = dict(formula=formula, block_permutation=block_permutation)
    # Formula variants and block permutations run on packed operands; a
    # plain weight is packed for the call, as is any plain weight whose tile
    # suits the packed kernel unless the compact kernel is selected.
    packed = isinstance(b, PackedOperand) or formula != "classical" or block_permutation != 0
    if not packed and PLAIN_WEIGHTS == "pack" and _fits_packed(algo, epilogue, bm, bn, bk):
        packed = True
    if not packed and not _fits(algo, epilogue, bm, bn, bk, _lib.SMX_B_KCONTIG) and _fits_packed(
            algo, epilogue, bm, bn, bk):
        packed = True  # a tile the compact kernel cannot take (a thin bm, for one)
    if not packed and (a.dtype == torch.float32 or b.dtype == torch.float32):
        packed = True  # FP32 inputs reach the kernels through the packing pass only
    if isinstance(a, PackedOperand) and not packed:
        raise ValueError("a packed activation needs a packed weight (strassen_weight_layout / "
                         "cubic_weight_layout)")
    b_layout = _lib.SMX_B_PACKED if packed else _lib.SMX_B_KCONTIG
    if isinstance(b, PackedOperand):
        _check_packed(b, algo, "rhs", bn, bk, passes=passes, **variant)
    if isinstance(a, PackedOperand):
        _check_packed(a, algo, "lhs", bm, bk, passes=passes, **variant)
    _check_device_tiling(algo, epilogue, bm, bn, bk, b_layout)
    _require_device(a.data if isinstance(a, PackedOperand) else a,
                    b.data if isinstance(b, PackedOperand) else b,
                    residual, bias, rope_cos, rope_sin, rope_scale)
    if packed:
        if not isinstance(b, PackedOperand):
            b = _plain_weight(b, algo=algo, bn=bn, bk=bk, dot_precision=dot_precision, **variant)
        if not isinstance(a, PackedOperand):
            a = pack_operand(a, algo=algo, side="lhs", tile_rows=bm, bk=bk, dot_precision=dot_precision, **variant)
        a_ptr, b_ptr, lda, ldb = a.data, b.data, k * passes, k * passes
    else:
        if a.stride(1) != 1 or a.stride(0) % 8 or a.data_ptr() % 16:
            a = a.contiguous()
        if not is_k_contiguous(b) or b.stride(1) % 8 or b.data_ptr() % 16:
            b = b.t().contiguous().t()
        bt = b.t()  # [N, K], rows contiguous
        a_ptr, b_ptr, lda, ldb = a, bt, a.stride(0), bt.stride(0)
    out_cols = n // 2 if epilogue in ("swiglu", "geglu") else n
    c = torch.empty((m, out_cols), dtype=out_dtype, device=a.device)
    desc = _lib.SmxGemmDesc()
    desc.m, desc.n, desc.k = m, n, k * passes
    desc.lda, desc.ldb, desc.ldc = lda, ldb, c.stride(0)
    desc.bm, desc.bn, desc.bk = bm, bn, bk
    desc.algo = algo
    desc.epilogue = _lib.SMX_EPI[epilogue]
    desc.a_layout = _lib.SMX_A_PACKED if packed else _lib.SMX_A_ROWMAJOR
    desc.b_layout = b_layout
    desc.flags = _lib.SMX_FLAG_OUT_F32 if out_dtype == torch.float32 else 0
    if algo == 7 and packed and STRASSEN_KERNEL == "product_major":
        desc.flags |= _lib.SMX_FLAG_PRODUCT_MAJOR
    if algo == 7 and packed and STRASSEN_KERNEL == "product_major_rounds":
        desc.flags |= _lib.SMX_FLAG_PRODUCT_MAJOR_ROUNDS
    desc.formula = _lib.SMX_FORMULA[formula]
    desc.block_permutation = block_permutation
    if partial is not None:
        desc.partial, desc.ldp = partial.data_ptr(), partial.stride(0)
    desc.rope_head_dim = rope_head_dim
    desc.rope_eps = rope_eps
    aux = 0
    if residual is not None:
        residual = _aux_tensor(residual)
        # the kernels read residual rows in 16-byte chunks
        if residual.stride(1) != 1 or (residual.stride(0) * residual.element_size()) % 16 or residual.data_ptr() % 16:
            residual = residual.contiguous()
        if residual.dtype == torch.float32:
            aux |= _lib.SMX_AUX_RESIDUAL_F32
        desc.ldr = residual.stride(0)
    if bias is not None:
        bias = _aux_tensor(bias.contiguous())
        if bias.dtype == torch.float32:
            aux |= _lib.SMX_AUX_BIAS_F32
    if rope_cos is not None:
        # The kernels read bf16 tables (rope_values builds them in bf16);
        # float32 tables are rounded to bf16 here.
        rope_cos = rope_cos.to(torch.bfloat16).contiguous()
        rope_sin = rope_sin.to(torch.bfloat16).contiguous()
        # the kernels read the tables and the scale 16 bytes at a time
        rope_cos = rope_cos if rope_cos.data_ptr() % 16 == 0 else rope_cos.clone()
        rope_sin = rope_sin if rope_sin.data_ptr() % 16 == 0 else rope_sin.clone()
        rope_scale = _aux_tensor(rope_scale.contiguous())
        rope_scale = rope_scale if rope_scale.data_ptr() % 16 == 0 else rope_scale.clone()
        if rope_scale.dtype == torch.float32:
            aux |= _lib.SMX_AUX_SCALE_F32
    desc.aux_f32 = aux
    # The library asks for a workspace when the tiles of a partly filled last
    # round run as K shares (FP32 shares of the output, summed by a second
    # pass) or when the product-major kernel takes the call (its two parked
    # FP32 sets per tile).
    need = ctypes.c_int64()
    _lib.check(lib.smx_gemm_workspace_bytes(desc, ctypes.byref(need)))
    workspace = None
    if need.value:
        workspace = torch.empty(need.value, dtype=torch.uint8, device=a.device)
        desc.workspace, desc.workspace_bytes = workspace.data_ptr(), need.value
    stream = torch.cuda.current_stream(a.device).cuda_stream
    rc = lib.smx_gemm(desc, _lib.ptr(a_ptr), _lib.ptr(b_ptr), _lib.ptr(c), _lib.ptr(residual),
                      _lib.ptr(bias), _lib.ptr(rope_cos), _lib.ptr(rope_sin),
                      _lib.ptr(rope_scale), stream)
    _lib.check(rc)
    return c


def _run_split(a, b, *, bm, bn, bk, schedule, formula, block_permutation, out_dtype, dot_precision=None,
               **epilogue_args):
    """An exact-panel schedule (``strassen_pallas.py:575-586``, ``:713-735``):
    Strassen over the ordinary K panels with an FP32 result, then the
    matched cubic over the exact panels (the eight products of
    ``run_exact_panel`` on raw quadrants), which adds that result to its
    quadrants before the epilogue. Products are summed in FP32 either way;
    only the order of the FP32 additions differs from the reference's
    panel-by-panel accumulation."""
    variant = dict(formula=formula, block_permutation=block_permutation)
    for x, name, side, tile_rows in ((a, "a", "lhs", bm), (b, "b", "rhs", bn)):
        if not isinstance(x, PackedOperand):
            continue
        if not isinstance(x, SplitOperand):
            raise ValueError(f"{name} was packed without exact panels; called with exact panels {schedule.exact} "
                             "(pack it with the call's classical_panels / panel_schedule)")
        if x.side != side or (x.tile_rows, x.bk) != (tile_rows, bk):
            raise ValueError(f"{name} was packed as {x!r}, not as the {side} of this call's tile")
        if x.schedule != schedule:
            raise ValueError(f"{name} was packed for the exact panels {x.schedule.exact}; called with "
                             f"{schedule.exact}")
        _check_passes(x, name, precision_passes(dot_precision, x.dtype))
        if (x.formula, x.block_permutation) != (formula, block_permutation):
            raise ValueError(f"{name} was packed for formula_variant={x.formula!r}, "
                             f"block_permutation={x.block_permutation}; called with "
                             f"formula_variant={formula!r}, block_permutation={block_permutation}")
    _check_device_tiling(_lib.SMX_ALGO_STRASSEN, epilogue_args.get("epilogue"), bm, bn, bk, _lib.SMX_B_PACKED)
    _require_device(a.data if isinstance(a, PackedOperand) else a, b.data if isinstance(b, PackedOperand) else b)
    if not isinstance(a, SplitOperand):
        a = pack_operand(a, algo=_lib.SMX_ALGO_STRASSEN, side="lhs", tile_rows=bm, bk=bk, panel_schedule=schedule,
                         dot_precision=dot_precision, **variant)
    if not isinstance(b, SplitOperand):
        b = _plain_weight(b, algo=_lib.SMX_ALGO_STRASSEN, bn=bn, bk=bk, panel_schedule=schedule,
                          dot_precision=dot_precision, **variant)
    partial = None
    if a.ordinary is not None:
        partial = _run(_lib.SMX_ALGO_STRASSEN, a.ordinary, b.ordinary, bm=bm, bn=bn, bk=bk,
                       out_dtype=torch.float32, dot_precision=dot_precision, **variant)
    return _run(_lib.SMX_ALGO_CUBIC, a.exact, b.exact, bm=bm, bn=bn, bk=bk, out_dtype=out_dtype, partial=partial,
                dot_precision=dot_precision, **epilogue_args)


def strassen_matmul(
    a,
    b,
    *,
    bm=TUNED_BM,
    bn=TUNED_BN,
    bk=TUNED_BK,
    dot_precision=None,
    interleave_products=False,
    block_permutation=0,
    formula_variant="classical",
    classical_panels=(),
    panel_schedule=None,
    epilogue=None,
    residual=None,
    bias=None,
    rope_cos=None,
    rope_sin=None,
    rope_scale=None,
    rope_head_dim=128,
    rope_eps=1e-6,
    norm_scale=None,
    norm_eps=1e-6,
    output_dtype=None,
    allow_input_fusion=None,
    product_aware_swiglu=False,
    product_aware_residual=False,
    interpret=False,
    vmem_limit_bytes=None,
):
    """Compute ``a @ b`` with one tile-local classical Strassen level.

    ``a`` is ``[M, K]`` and ``b`` is ``[K, N]``, both bf16 on the HIP device.
    ``b`` is either a tensor, read directly when K-contiguous (``w.t()`` of a
    ``[N, K]`` weight, see ``layouts.k_contiguous``; otherwise transposed on
    each call) and served by the kernel that forms both operand sums in
    registers; or a packed weight from ``strassen_weight_layout(b, bn, bk)``
    (pre-summed B operands), served by the packed kernel after ``a`` is
    packed with its A sums (or pass ``a`` already packed by
    ``pack_activation``). Epilogues and their operands follow
    ``strassen_pallas.py:739-879``:
    ``swiglu`` returns ``[M, N/2]`` from a ``swiglu_weight_layout`` weight,
    ``residual_add`` adds ``residual`` ``[M, N]``, ``bias_add`` adds
    ``bias`` ``[N]``, ``qk_norm_rope`` applies per-head RMSNorm and RoPE with
    ``rope_layout_tables`` / ``rope_scale_layout`` operands.
    """
    m, k, n, classical_panels, out_dtype = _validate(
        a, b, bm=bm, bn=bn, bk=bk, block_permutation=block_permutation,
        formula_variant=formula_variant, classical_panels=classical_panels,
        panel_schedule=panel_schedule, epilogue=epilogue, residual=residual,
        bias=bias, rope_cos=rope_cos, rope_sin=rope_sin, rope_scale=rope_scale,
        rope_head_dim=rope_head_dim, norm_scale=norm_scale,
        output_dtype=output_dtype, allow_input_fusion=allow_input_fusion,
        product_aware_swiglu=product_aware_swiglu,
        product_aware_residual=product_aware_residual)
    _unsupported(a.dtype, interpret, dot_precision)
    schedule = exact_schedule(k // bk, classical_panels=classical_panels, panel_schedule=panel_schedule)
    return _run(_lib.SMX_ALGO_STRASSEN, a, b, bm=bm, bn=bn, bk=bk, epilogue=epilogue,
                residual=residual, bias=bias, rope_cos=rope_cos, rope_sin=rope_sin,
                rope_scale=rope_scale, rope_head_dim=rope_head_dim, rope_eps=rope_eps,
                out_dtype=out_dtype, formula=formula_variant, block_permutation=block_permutation,
                norm_scale=norm_scale, norm_eps=norm_eps, schedule=schedule, dot_precision=dot_precision)


def strassen_matmul_lhs_transposed(a, b, *, bm=TUNED_BM, bn=TUNED_BN, bk=TUNED_BK, dot_precision=None,
                                   interleave_products=False, output_dtype=None, allow_input_fusion=None,
                                   interpret=False, vmem_limit_bytes=None):
    """``a.T @ b`` with ``a`` kept in its producer layout ``[K, M]``
    (``strassen_pallas.py:1224-1312``), for weight-gradient products.

    The packing pass reads ``a`` transposed tile by tile (no ``[M, K]`` copy is
    materialised) while forming the A operand sums; ``b`` is a ``[K, N]``
    tensor (packed on each call) or a ``strassen_weight_layout`` weight.
    Arguments, checks and messages follow ``:1250-1267``; FP32 inputs run
    the product of ``dot_precision`` (one pass at DEFAULT, 3 / 6 bf16 passes
    at HIGH / HIGHEST) and ``interpret=True`` raises ``NotImplementedError``.
    """
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError("strassen_matmul_lhs_transposed expects rank-2 inputs")
    k, m = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError(f"contracting dimensions disagree: {k} vs {k2}")
    if a.dtype != b.dtype:
        raise ValueError(f"input dtypes disagree: {a.dtype} vs {b.dtype}")
    if a.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("inputs must be BF16 or FP32")
    for name, dimension, block in (("M", m, bm), ("N", n, bn), ("K", k, bk)):
        if dimension % block:
            raise ValueError(f"{name}={dimension} is not divisible by {block}")
    check_tiling(bm, bn, bk)
    if allow_input_fusion is not None:
        allow_input_fusion = tuple(allow_input_fusion)
        if len(allow_input_fusion) != 2:
            raise ValueError("allow_input_fusion must contain two booleans")
    out_dtype = a.dtype if output_dtype is None else output_dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("output_dtype must be BF16 or FP32")
    _unsupported(a.dtype, interpret, dot_precision)
    _check_device_tiling(_lib.SMX_ALGO_STRASSEN, None, bm, bn, bk, _lib.SMX_B_PACKED)
    _require_device(a, b.data if isinstance(b, PackedOperand) else b)
    packed_a = pack_operand(a, algo=_lib.SMX_ALGO_STRASSEN, side="lhs_t", tile_rows=bm, bk=bk,
                            dot_precision=dot_precision)
    if not isinstance(b, PackedOperand):
        b = _plain_weight(b, algo=_lib.SMX_ALGO_STRASSEN, bn=bn, bk=bk, dot_precision=dot_precision)
    return _run(_lib.SMX_ALGO_STRASSEN, packed_a, b, bm=bm, bn=bn, bk=bk, out_dtype=out_dtype,
                dot_precision=dot_precision)


def cubic_matmul(a, b, *, variant="blocked", bm=TUNED_BM, bn=TUNED_BN, bk=TUNED_BK,
                 dot_precision=None, allow_input_fusion=None, interpret=False,
                 vmem_limit_bytes=None, epilogue=None, residual=None, bias=None,
                 rope_cos=None, rope_sin=None, rope_scale=None, rope_head_dim=128,
                 rope_eps=1e-6, output_dtype=None, norm_scale=None, norm_eps=1e-6):
    """Matched cubic control (``experiments/qwen3/benchmark_cubic_control.py:116-177``).

    Eight half-size products per K panel into four FP32 quadrant
    accumulators, with the Strassen kernel's tiling, LDS staging and
    epilogues. ``variant="full"`` (one full-tile product per panel) computes
    the same cubic GEMM and runs the same kernel. The fused epilogues are an
    extension of the reference control, used to time fused sites against an
    identical cubic arm. A plain ``b`` runs the compact kernel that matches
    ``strassen_matmul`` with a plain weight; a ``cubic_weight_layout(b, bn,
    bk)`` weight runs the packed kernel that matches ``strassen_matmul`` with
    a ``strassen_weight_layout`` weight.
    """
    if variant not in ("full", "blocked"):
        raise ValueError(f"unknown cubic variant {variant!r}")
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError("cubic_matmul expects two rank-2 matrices")
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError(f"inner dimensions disagree: {k} vs {k2}")
    if allow_input_fusion is not None:
        allow_input_fusion = tuple(allow_input_fusion)
        if len(allow_input_fusion) != 2:
            raise ValueError("allow_input_fusion must contain one boolean per operand")
        if not all(isinstance(value, bool) for value in allow_input_fusion):
            raise TypeError("allow_input_fusion entries must be bool")
    for name, dimension, block in (("M", m, bm), ("N", n, bn), ("K", k, bk)):
        if dimension % block:
            raise ValueError(f"{name}={dimension} is not divisible by {block}")
    check_tiling(bm, bn, bk)
    if a.dtype != b.dtype:
        raise ValueError(f"input dtypes disagree: {a.dtype} vs {b.dtype}")
    if a.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("inputs must be BF16 or FP32")
    _unsupported(a.dtype, interpret, dot_precision)
    out_dtype = a.dtype if output_dtype is None else output_dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("output_dtype must be BF16 or FP32")
    if epilogue is not None:
        _check_epilogue_name(epilogue)
        if output_dtype is not None and output_dtype != torch.bfloat16:
            raise ValueError("fused epilogues write a BF16 output tile")
    _check_epilogue_operands(m, n, bn, epilogue=epilogue, residual=residual, bias=bias, rope_cos=rope_cos,
                             rope_sin=rope_sin, rope_scale=rope_scale, rope_head_dim=rope_head_dim,
                             norm_scale=norm_scale)
    return _run(_lib.SMX_ALGO_CUBIC, a, b, bm=bm, bn=bn, bk=bk, epilogue=epilogue,
                residual=residual, bias=bias, rope_cos=rope_cos, rope_sin=rope_sin,
                rope_scale=rope_scale, rope_head_dim=rope_head_dim, rope_eps=rope_eps,
                out_dtype=out_dtype, norm_scale=norm_scale, norm_eps=norm_eps, dot_precision=dot_precision)


def native_matmul(a, b):
    """Vendor arm: hipBLASLt bf16 GEMM with FP32 accumulation and bf16 output
    (``strassen_pallas.py:1414-1421``)."""
    return torch.matmul(a, b)
