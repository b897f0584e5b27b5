"""Numpy restatement of the reference's tile-local one-level Strassen path.

Test infrastructure only (see ``oracle/__init__.py``). Matrices are carried
as float32 arrays whose values are exactly representable in bfloat16 (the
"bf16 value" convention); ``bf16_round`` performs every bf16 rounding the
reference performs, and nothing else rounds.

File:line citations are relative to the reference checkout.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "bf16_round", "bf16_bits", "bits_to_f32", "silu", "gelu_tanh",
    "strassen_matmul", "strassen_matmul_lhs_transposed", "cubic_blocked_matmul", "native_matmul",
    "high_precision_reference", "device_error", "host_uniform_inputs",
    "swiglu_weight_layout_order", "swiglu_weight_layout",
    "rope_weight_layout_order", "rope_weight_layout", "rope_layout_tables",
    "rope_scale_layout", "rope_layout_to_heads", "rope_values", "rms_norm",
    "apply_rope", "strassen_products", "strassen_a_operands", "strassen_b_operands",
    "operand_planes", "packed_operand", "unpack_operand", "PACK_TILE", "PACK_STAGE",
    "dual_a_operands", "dual_b_operands", "powers_a_operands", "powers_b_operands", "powers_decode",
    "permuted_quadrants", "formula_operands", "operand_values", "DUAL_UPDATES", "POWERS_BASIS_UPDATES",
    "PRODUCT_UPDATES", "precision_passes", "bf16_part", "pass_product", "PASS_PARTS",
]


# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------

def bf16_bits(x):
    """Round float32 values to bfloat16 (ties to even) and return uint16 bits.

    Same rounding as ``x.astype(jnp.bfloat16)`` used throughout
    ``strassen_pallas.py`` (e.g. ``:327-329``): round-to-nearest-even on the
    upper 16 bits. NaN stays NaN (quiet bit set); +-inf and overflow to inf
    follow IEEE rounding.
    """
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32)
    rounding_bias = np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
    rounded = ((u + rounding_bias) >> np.uint32(16)).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded = np.where(nan, ((u >> np.uint32(16)) | np.uint32(0x0040)).astype(np.uint16), rounded)
    return rounded


def bits_to_f32(bits):
    """Widen uint16 bfloat16 bit patterns to float32 (exact)."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)
    return b.view(np.float32)


def bf16_round(x):
    """Round to the nearest bfloat16 value, returned as float32."""
    return bits_to_f32(bf16_bits(x))


def silu(x):
    """float32 ``x * sigmoid(x)`` -- ``jax.nn.silu`` (``strassen_pallas.py:153``)."""
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore"):
        return (x / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def gelu_tanh(x):
    """float32 tanh-approximate GELU -- ``jax.nn.gelu(approximate=True)``, the
    GeGLU gate (``strassen_pallas.py:143-153``):
    0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))."""
    x = np.asarray(x, dtype=np.float32)
    k = np.float32(np.sqrt(2.0 / np.pi))
    inner = k * (x + np.float32(0.044715) * x * x * x)
    return (np.float32(0.5) * x * (np.float32(1.0) + np.tanh(inner))).astype(np.float32)


# ---------------------------------------------------------------------------
# Strassen algebra
# ---------------------------------------------------------------------------

# Classical products and the quadrant updates each one makes,
# ``strassen_pallas.py:324-379``. Quadrants: 0=(top,left) 1=(top,right)
# 2=(bottom,left) 3=(bottom,right); a0..a3 / b0..b3 use the same numbering
# over (row half, K half) and (K half, column half), ``:193-204``.
PRODUCT_UPDATES = {
    1: ((0, +1), (3, +1)),   # P1=(A0+A3)(B0+B3)
    2: ((2, +1), (3, -1)),   # P2=(A2+A3)B0
    3: ((1, +1), (3, +1)),   # P3=A0(B1-B3)
    4: ((0, +1), (2, +1)),   # P4=A3(B2-B0)
    5: ((0, -1), (1, +1)),   # P5=(A0+A1)B3
    6: ((3, +1),),           # P6=(A2-A0)(B0+B1)
    7: ((0, +1),),           # P7=(A1-A3)(B2+B3)
}

PLAIN_ORDER = (1, 2, 3, 4, 5, 6, 7)                 # ``:566-573``
INTERLEAVED_ORDER = (4, 6, 5, 2, 7, 3, 1)           # ``:556-565``
PA_SWIGLU_TOP = (4, 5, 7, 3, 1)                     # ``:627-631``
PA_SWIGLU_BOTTOM = (6, 2)                           # ``:633-634``
PA_RESIDUAL_FINAL = (4, 6, 5, 2, 7, 3, 1)           # ``:679-687``


def _identity(x):
    return x


def strassen_a_operands(a_q, r=bf16_round):
    """The A operands of P1..P7 (``strassen_pallas.py:324-379``): A0+A3,
    A2+A3, A0, A3, A0+A1, A2-A0, A1-A3, every sum rounded once to bf16.

    Each add/sub is ``(x.astype(cd) + y.astype(cd)).astype(cd)`` with cd=bf16
    in the reference: the exact sum of two bf16 values rounded once to bf16.
    float32 holds that sum exactly or within half a float32 ulp, and float32
    precision (24 bits) >= 2*8+2, so rounding the float32 sum to bf16 is the
    correctly rounded bf16 sum.

    ``r`` rounds each jnp operation's result: ``bf16_round`` for bf16 inputs
    (compute dtype bf16), the identity for FP32 inputs (compute dtype f32,
    the finished operand is rounded by the product, ``operand_round``).
    """
    a0, a1, a2, a3 = a_q
    return (r(a0 + a3), r(a2 + a3), a0, a3, r(a0 + a1), r(a2 - a0), r(a1 - a3))


def strassen_b_operands(b_q, r=bf16_round):
    """The B operands of P1..P7: B0+B3, B0, B1-B3, B2-B0, B3, B0+B1, B2+B3."""
    b0, b1, b2, b3 = b_q
    return (r(b0 + b3), b0, r(b1 - b3), r(b2 - b0), b3, r(b0 + b1), r(b2 + b3))


# Dual formula (``strassen_pallas.py:461-517``): operands and quadrant updates.
DUAL_UPDATES = {
    1: ((0, +1), (3, +1)),
    2: ((1, +1), (3, -1)),
    3: ((2, +1), (3, +1)),
    4: ((0, +1), (1, +1)),
    5: ((0, -1), (2, +1)),
    6: ((3, +1),),
    7: ((0, +1),),
}
DUAL_INTERLEAVED_ORDER = (5, 6, 4, 3, 7, 2, 1)       # ``:539-547``

# Power-of-two formula (``:381-459``): updates of the sparse output basis
# z0..z3, decoded once after the last K panel (``:744-760``).
POWERS_BASIS_UPDATES = {
    1: ((3, +1),),
    2: ((2, +1),),
    3: ((0, +1), (3, -1)),
    4: ((2, -1), (3, +1)),
    5: ((0, +1),),
    6: ((1, +1),),
    7: ((1, +1), (3, +1)),
}
POWERS_INTERLEAVED_ORDER = (3, 2, 6, 5, 4, 7, 1)     # ``:520-528``


def dual_a_operands(a_q, r=bf16_round):
    """A operands of the dual formula Q1..Q7 (``:461-517``): A0+A3, A0,
    A2-A3, A1-A0, A3, A0+A2, A1+A3."""
    a0, a1, a2, a3 = a_q
    return (r(a0 + a3), a0, r(a2 - a3), r(a1 - a0), a3, r(a0 + a2), r(a1 + a3))


def dual_b_operands(b_q, r=bf16_round):
    """B operands of Q1..Q7: B0+B3, B1+B3, B0, B3, B0+B2, B1-B0, B2-B3."""
    b0, b1, b2, b3 = b_q
    return (r(b0 + b3), r(b1 + b3), b0, b3, r(b0 + b2), r(b1 - b0), r(b2 - b3))


def powers_a_operands(a_q, r=bf16_round):
    """A operands of R1..R7 (``:398-459``). Every jnp bf16 operation rounds
    its result to bf16 (the HLO semantics of the traced expressions);
    scaling by 1/2 and 1/4 is exact, so each two-term sum rounds once and
    each balanced four-term expression rounds its two halves and their sum."""
    a0, a1, a2, a3 = a_q
    h, q = np.float32(0.5), np.float32(0.25)
    return (r(a2 - a1),
            r(r(a0 - a2 * h) + r(a1 * h - a3 * q)),
            r(a2 - a3 * h),
            r(a1 - a3 * h),
            r(a2 + a3 * h),
            r(r(a0 - a1 * h) + r(a2 * h - a3 * q)),
            r(a1 + a3 * h))


def powers_b_operands(b_q, r=bf16_round):
    """B operands of R1..R7 (``:398-459``), rounded as ``powers_a_operands``."""
    b0, b1, b2, b3 = b_q
    h, q = np.float32(0.5), np.float32(0.25)
    return (r(b0 - b3),
            r(b0 + b1 * h),
            r(b1 * h - b3),
            r(r(b0 * h - b2) + r(b1 * q - b3 * h)),
            r(b1 * h + b3),
            r(b0 - b1 * h),
            r(r(b0 * h + b2) - r(b1 * q + b3 * h)))


def powers_decode(z):
    """Quadrants from the basis (``:744-760``): C3 = z0, C2 = z3 + z0/2,
    C0 = (z1 + z2)/2 + z0/4, C1 = (z2 - z1) + z3 + z0/2."""
    z0, z1, z2, z3 = z
    h, q = np.float32(0.5), np.float32(0.25)
    return [((z1 + z2) * h + z0 * q).astype(np.float32),
            (((z2 - z1) + z3) + z0 * h).astype(np.float32),
            (z3 + z0 * h).astype(np.float32),
            z0.astype(np.float32)]


def permuted_quadrants(quads, swap_rows, swap_cols):
    """``transformed_index`` (``:209-226``): quadrant (row, col) reads the
    original quadrant (row ^ swap_rows, col ^ swap_cols)."""
    return tuple(quads[2 * (row ^ swap_rows) + (col ^ swap_cols)] for row in range(2) for col in range(2))


def operation_round(input_dtype):
    """Rounding of each jnp operation in the kernel: the compute dtype is the
    input dtype (``compute_dtype=a.dtype``, ``strassen_pallas.py:1062``)."""
    if input_dtype == "bfloat16":
        return bf16_round
    if input_dtype == "float32":
        return _identity
    raise ValueError(f"input_dtype must be 'bfloat16' or 'float32', got {input_dtype!r}")


def operand_round(x):
    """What the product sees of an operand: ``jnp.dot`` at DEFAULT precision
    multiplies one bf16 pass on the TPU (``:228-232``), so a float32 operand
    is rounded to bf16 (bf16 operands are unchanged)."""
    return bf16_round(x)


# ``dot_precision`` (``:228-232``, default ``:889``) for FP32 operands: the
# jax.lax.Precision names and string aliases -> bf16 passes per product.
# DEFAULT multiplies one bf16 pass; HIGH is XLA's 3-pass bf16 product
# (bf16_3x) and HIGHEST its 6-pass product (bf16_6x).
_PRECISION_PASSES = {"DEFAULT": 1, "FASTEST": 1, "BFLOAT16": 1, "HIGH": 3, "BFLOAT16_3X": 3,
                     "TENSORFLOAT32": 3, "HIGHEST": 6, "FLOAT32": 6}

# Parts (of the A operand, of the B operand) multiplied by each pass: the
# bf16 expansion v = p0 + p1 + p2 of each operand, and every pass pair whose
# parts' orders sum to at most 1 (HIGH) or 2 (HIGHEST), smallest products
# first: p1*p0, p0*p1, p0*p0; p2*p0, p1*p1, p0*p2, p1*p0, p0*p1, p0*p0.
PASS_PARTS = {1: ((0,), (0,)), 3: ((1, 0, 0), (0, 1, 0)), 6: ((2, 1, 0, 1, 0, 0), (0, 1, 2, 0, 1, 0))}


def precision_passes(dot_precision, input_dtype="float32"):
    """bf16 passes per product: 1 for bf16 inputs (their operands are bf16
    values, whose low-order parts are zero), else by ``dot_precision``."""
    if dot_precision is None:
        passes = 1
    else:
        name = str(getattr(dot_precision, "name", dot_precision)).upper().rsplit(".", 1)[-1]
        if name not in _PRECISION_PASSES:
            raise ValueError(f"unknown dot_precision {dot_precision!r}")
        passes = _PRECISION_PASSES[name]
    return passes if input_dtype == "float32" else 1


def bf16_part(x, part):
    """Part ``part`` of the bf16 expansion of float32 ``x``: p0 = bf16(x),
    p1 = bf16(x - p0), p2 = bf16(x - p0 - p1), remainders in float32 (they
    are exact there)."""
    x = np.asarray(x, dtype=np.float32)
    p = bf16_round(x)
    for _ in range(part):
        x = (x - p).astype(np.float32)
        p = bf16_round(x)
    return p


def pass_product(s, t, passes=1):
    """``jnp.dot(s, t, preferred_element_type=float32)`` at ``passes`` bf16
    passes: the sum over the pass pairs of the bf16-part products, each an
    exact product summed in FP32. One pass is the DEFAULT product
    ``bf16(s) @ bf16(t)``."""
    parts_a, parts_b = PASS_PARTS[passes]
    value = np.zeros((s.shape[0], t.shape[1]), dtype=np.float32)
    for i, j in zip(parts_a, parts_b):
        value += np.matmul(bf16_part(s, i), bf16_part(t, j), dtype=np.float32)
    return value


def operand_values(formula, a_q, b_q, input_dtype="bfloat16"):
    """{p: (S_p, T_p)} of products 1..7 of ``formula`` in the compute dtype
    (each jnp operation rounded for bf16 inputs), before the product's own
    bf16 rounding."""
    r = operation_round(input_dtype)
    if formula == "classical":
        return strassen_products(a_q, b_q, r)
    if formula == "dual":
        sa, tb = dual_a_operands(a_q, r), dual_b_operands(b_q, r)
    elif formula == "powers":
        sa, tb = powers_a_operands(a_q, r), powers_b_operands(b_q, r)
    else:
        raise ValueError(f"unknown formula {formula!r}")
    return {p: (sa[p - 1], tb[p - 1]) for p in range(1, 8)}


def formula_operands(formula, a_q, b_q, input_dtype="bfloat16"):
    """(A operand, B operand) of products 1..7 of ``formula``, each operand
    as the one-pass product sees it."""
    return {p: (operand_round(s_), operand_round(t_))
            for p, (s_, t_) in operand_values(formula, a_q, b_q, input_dtype).items()}


# The eight half-size cubic products (A quadrant, B quadrant, C quadrant) in
# the matched control's order (benchmark_cubic_control.py:96-106), which is
# also the exact-panel order (strassen_pallas.py:575-586).
CUBIC_PAIRS = ((0, 0, 0), (0, 1, 1), (2, 0, 2), (2, 1, 3), (1, 2, 0), (1, 3, 1), (3, 2, 2), (3, 3, 3))


def strassen_products(a_q, b_q, r=bf16_round):
    """The seven classical operand pairs {p: (S_p, T_p)}."""
    sa = strassen_a_operands(a_q, r)
    tb = strassen_b_operands(b_q, r)
    return {p: (sa[p - 1], tb[p - 1]) for p in range(1, 8)}


def _split_a(a, bm, bk, step):
    """Quadrants of every A tile in K panel ``step`` stacked over row tiles.

    Returns four (M/2, bk/2) arrays whose row index is (row tile, local row).
    Quadrant slicing follows ``strassen_pallas.py:193-198``.
    """
    m = a.shape[0]
    hm, hk = bm // 2, bk // 2
    panel = a[:, step * bk:(step + 1) * bk].reshape(m // bm, 2, hm, 2, hk)
    return tuple(
        np.ascontiguousarray(panel[:, r, :, c, :].reshape(m // 2, hk))
        for r in range(2) for c in range(2))


def _split_b(b, bn, bk, step):
    """Quadrants of every B tile in K panel ``step`` stacked over column tiles.

    Returns four (bk/2, N/2) arrays (``strassen_pallas.py:199-204``).
    """
    n = b.shape[1]
    hn, hk = bn // 2, bk // 2
    panel = b[step * bk:(step + 1) * bk, :].reshape(2, hk, n // bn, 2, hn)
    return tuple(
        np.ascontiguousarray(panel[r, :, :, c, :].reshape(hk, n // 2))
        for r in range(2) for c in range(2))


def _quadrants_of(x, bm, bn):
    """Split an (M, N) output-shaped array into its four quadrant planes."""
    m, n = x.shape
    hm, hn = bm // 2, bn // 2
    v = x.reshape(m // bm, 2, hm, n // bn, 2, hn)
    return tuple(
        np.ascontiguousarray(v[:, r, :, :, c, :].reshape(m // 2, n // 2))
        for r in range(2) for c in range(2))


def _assemble(quads, m, n, bm, bn):
    """Inverse of ``_quadrants_of``: four (M/2, N/2) planes -> (M, N)."""
    hm, hn = bm // 2, bn // 2
    out = np.empty((m // bm, 2, hm, n // bn, 2, hn), dtype=np.float32)
    for q in range(4):
        r, c = divmod(q, 2)
        out[:, r, :, :, c, :] = quads[q].reshape(m // bm, hm, n // bn, hn)
    return out.reshape(m, n)


def _column_vector_quadrants(v, bn):
    """Split a length-N per-column vector into its (left, right) halves."""
    n = v.shape[0]
    hn = bn // 2
    w = v.reshape(n // bn, 2, hn)
    return (np.ascontiguousarray(w[:, 0, :].reshape(n // 2)),
            np.ascontiguousarray(w[:, 1, :].reshape(n // 2)))


PACK_TILE = 128  # product rows per packed tile (the kernel's workgroup tile)
PACK_STAGE = 16  # product depth per packed stage (one MFMA k step)


def operand_planes(x, algo, side, tile_rows, bk, formula="classical", block_permutation=0,
                   input_dtype="bfloat16", dot_precision=None):
    """The GEMM operands of every tile as (nops, R, K/2) product-space planes.

    ``side="lhs"``: x is A [M, K], R = M/2 product rows (row tile, local row).
    ``side="rhs"``: x is B [K, N], R = N/2 product columns (column tile,
    local column). Depth k' = (K panel, local k < bk/2). Strassen (algo 7)
    gives the seven operand sums of ``strassen_a_operands`` /
    ``strassen_b_operands``; the cubic (algo 8) the four quadrants. Every
    operand is as the product sees it (``operand_round``; FP32 inputs form
    the sums in float32 first). A multi-pass ``dot_precision`` (FP32
    inputs) lays the passes out pass-major: depth (pass, K panel, local k),
    the pass taking the operand's bf16 part of ``PASS_PARTS``.
    """
    r = operation_round(input_dtype)
    x = np.asarray(x, dtype=np.float32)
    sm, sk, sn = block_permutation & 1, (block_permutation >> 1) & 1, (block_permutation >> 2) & 1
    a_ops = {"classical": strassen_a_operands, "dual": dual_a_operands, "powers": powers_a_operands}[formula]
    b_ops = {"classical": strassen_b_operands, "dual": dual_b_operands, "powers": powers_b_operands}[formula]
    passes = precision_passes(dot_precision, input_dtype)
    if side == "lhs":
        panels = [_split_a(x, tile_rows, bk, s) for s in range(x.shape[1] // bk)]
        ops_of = (lambda q: a_ops(permuted_quadrants(q, sm, sk), r)) if algo == 7 else list
        parts = PASS_PARTS[passes][0]
    elif side == "rhs":
        panels = [[q.T for q in _split_b(x, tile_rows, bk, s)] for s in range(x.shape[0] // bk)]
        ops_of = (lambda q: b_ops(permuted_quadrants(q, sk, sn), r)) if algo == 7 else list
        parts = PASS_PARTS[passes][1]
    else:
        raise ValueError("side must be 'lhs' or 'rhs'")
    ops = [np.stack(ops_of(quads)) for quads in panels]
    return np.concatenate([bf16_part(o, part) for part in parts for o in ops], axis=2)


def packed_operand(x, algo, side, tile_rows, bk, formula="classical", block_permutation=0,
                   input_dtype="bfloat16", dot_precision=None):
    """``smx_pack_operand``'s output as a flat float32 array of bf16 values:
    ``[R/128][K/32][nops][4][64][8]``, lane l of a fragment holding product
    row l%32 of its 32-row block and depth 8*(l//32)..+8 of its stage; R is
    the product rows rounded up to 128, the rows past them zeros."""
    planes = operand_planes(x, algo, side, tile_rows, bk, formula, block_permutation, input_dtype, dot_precision)
    nops, rows, depth = planes.shape
    # A thin tiling (tile_rows/2 not a multiple of 128) leaves a partial last
    # product tile: its missing rows are zeros (smx_packed_bytes counts them).
    padded = -(-rows // PACK_TILE) * PACK_TILE
    if padded != rows:
        planes = np.concatenate([planes, np.zeros((nops, padded - rows, depth), np.float32)], axis=1)
        rows = padded
    v = planes.reshape(nops, rows // PACK_TILE, 4, 32, depth // PACK_STAGE, 2, 8)
    # (op, tile, block, row32, stage, half, e) -> (tile, stage, op, block, half, row32, e)
    return np.ascontiguousarray(v.transpose(1, 4, 0, 2, 5, 3, 6)).reshape(-1)


def unpack_operand(flat, nops, rows, depth):
    """Inverse of the packing order: flat -> (nops, R, K/2) planes."""
    v = np.asarray(flat).reshape(rows // PACK_TILE, depth // PACK_STAGE, nops, 4, 2, 32, 8)
    return np.ascontiguousarray(v.transpose(2, 0, 3, 5, 1, 4, 6)).reshape(nops, rows, depth)


def _check_common(a, b, bm, bn, bk):
    if a.ndim != 2 or b.ndim != 2:
        raise ValueError("strassen_matmul expects two rank-2 matrices")
    m, k = a.shape
    k2, n = b.shape
    if k != k2:
        raise ValueError(f"inner dimensions disagree: {k} vs {k2}")
    for name, dimension, block in (("M", m, bm), ("N", n, bn), ("K", k, bk)):
        if dimension % block:
            raise ValueError(f"{name}={dimension} is not divisible by {block}")
    if bm % 2 or bn % 2 or bk % 2:
        raise ValueError("tile dimensions must be even")
    return m, k, n


def strassen_matmul(a, b, *, bm, bn, bk, interleave_products=False,
                    epilogue=None, residual=None, bias=None, rope_cos=None,
                    rope_sin=None, rope_scale=None, rope_head_dim=128,
                    rope_eps=1e-6, product_aware_swiglu=False,
                    product_aware_residual=False, output_dtype="bfloat16",
                    formula_variant="classical", block_permutation=0, norm_scale=None,
                    norm_eps=1e-6, classical_panels=(), panel_schedule=None, input_dtype="bfloat16",
                    dot_precision=None):
    """``a @ b`` with one tile-local classical Strassen level.

    Restates ``_classical_strassen_kernel`` (``strassen_pallas.py:156-879``)
    under the plumbing of ``strassen_matmul`` (``:882-1221``):

    * ``formula_variant`` "classical" (``:324-379``), "dual" (``:461-517``)
      or "powers" (``:381-459``, sparse output basis decoded after the last
      panel, ``:744-760``; no fused epilogues);
    * ``block_permutation`` bits swap the row / K / column halves of the
      operand and output quadrants (``:205-226``);
    * ``classical_panels`` / ``panel_schedule`` (nonzero entries) mark K
      panels that run the exact eight-product cubic update of the quadrant
      accumulators instead (``run_exact_panel``, ``:575-586``, ``:713-735``);
    * grid ``(M/bm, N/bn, K/bk)``; per K panel the seven half-size products
      update four FP32 quadrant accumulators in the reference's order
      (plain ``:566-573`` or interleaved ``:556-565``; product-aware final
      panels ``:593-689``);
    * the epilogue runs on the FP32 accumulators after the last panel and
      the result is rounded once to bf16 (``:739-879``);
    * ``output_dtype="float32"`` returns the accumulators unrounded
      (the reference's output-as-accumulator mode ``:1054-1057`` sums the
      same values in the same order).

    With ``input_dtype="bfloat16"`` the inputs must hold bf16 values (use
    ``bf16_round`` first); with ``"float32"`` they are FP32 inputs: the
    operand sums are formed in float32 and every operand is rounded once to
    bf16 by the one-pass DEFAULT-precision product (``operand_round``).
    Returns float32 arrays holding bf16 values (or raw FP32 for
    ``output_dtype="float32"``).
    """
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    m, k, n = _check_common(a, b, bm, bn, bk)
    nk = k // bk
    hm, hn = bm // 2, bn // 2
    if product_aware_swiglu and epilogue not in ("swiglu", "geglu"):
        raise ValueError("product_aware_swiglu is only valid with epilogue='swiglu' or 'geglu'")
    if product_aware_residual and epilogue != "residual_add":
        raise ValueError("product_aware_residual is only valid with epilogue='residual_add'")
    if formula_variant not in ("classical", "dual", "powers"):
        raise ValueError(f"unknown formula_variant {formula_variant!r}")
    if not 0 <= block_permutation < 8:
        raise ValueError("block_permutation must be 0..7")
    if (product_aware_swiglu or product_aware_residual) and (formula_variant != "classical" or block_permutation):
        raise ValueError("product-aware schedules require unpermuted classical Strassen")
    if formula_variant == "powers" and epilogue is not None:
        raise ValueError("fused epilogues require a quadrant-basis formula")
    swap_m, swap_k, swap_n = block_permutation & 1, (block_permutation >> 1) & 1, (block_permutation >> 2) & 1
    output_index = [2 * ((q >> 1) ^ swap_m) + ((q & 1) ^ swap_n) for q in range(4)]
    updates = {"classical": PRODUCT_UPDATES, "dual": DUAL_UPDATES, "powers": POWERS_BASIS_UPDATES}[formula_variant]
    interleaved = {"classical": INTERLEAVED_ORDER, "dual": DUAL_INTERLEAVED_ORDER,
                   "powers": POWERS_INTERLEAVED_ORDER}[formula_variant]
    order = interleaved if interleave_products else PLAIN_ORDER
    # classical / dual accumulate physical quadrants (``update``, :241-266);
    # powers accumulates the unpermuted basis (``update_basis``, :268-273)
    basis = formula_variant == "powers"
    exact = set(int(p) for p in classical_panels)
    if panel_schedule is not None:
        exact |= {i for i, v in enumerate(np.asarray(panel_schedule).tolist()) if v}
    if exact and basis:
        raise ValueError("exact panels require a quadrant-basis formula")

    acc = [np.zeros((m // 2, n // 2), dtype=np.float32) for _ in range(4)]
    passes = precision_passes(dot_precision, input_dtype)

    def run(products, sequence):
        for p in sequence:
            s, t = products[p]
            value = pass_product(s, t, passes)
            for q, sign in updates[p]:
                idx = q if basis else output_index[q]
                if sign > 0:
                    acc[idx] += value
                else:
                    acc[idx] -= value

    for step in range(nk):
        a_q = permuted_quadrants(_split_a(a, bm, bk, step), swap_m, swap_k)
        b_q = permuted_quadrants(_split_b(b, bn, bk, step), swap_k, swap_n)
        if step in exact:
            for ia, ib, q in CUBIC_PAIRS:
                acc[output_index[q]] += pass_product(a_q[ia], b_q[ib], passes)
            continue
        products = operand_values(formula_variant, a_q, b_q, input_dtype)
        last = step == nk - 1
        if last and product_aware_swiglu:
            run(products, PA_SWIGLU_TOP)
            run(products, PA_SWIGLU_BOTTOM)
        elif last and product_aware_residual:
            run(products, PA_RESIDUAL_FINAL)
        else:
            run(products, order)
    if basis:
        decoded = powers_decode(acc)
        acc = [None] * 4
        for q in range(4):
            acc[output_index[q]] = decoded[q]
    return _epilogue(acc, m, n, bm, bn, epilogue=epilogue, residual=residual,
                     bias=bias, rope_cos=rope_cos, rope_sin=rope_sin,
                     rope_scale=rope_scale, rope_head_dim=rope_head_dim,
                     rope_eps=rope_eps, output_dtype=output_dtype, norm_scale=norm_scale,
                     norm_eps=norm_eps)


def strassen_matmul_lhs_transposed(a_t, b, *, bm, bn, bk, interleave_products=False,
                                   output_dtype="bfloat16", input_dtype="bfloat16", dot_precision=None):
    """``a_t.T @ b`` (``strassen_pallas.py:1224-1312``): the kernel transposes
    each resident ``(bk, bm)`` tile of ``a_t`` and runs the ordinary classical
    Strassen body on it (``:1273-1289``), so the result is ``strassen_matmul``
    of the transposed matrix."""
    return strassen_matmul(np.asarray(a_t, dtype=np.float32).T, b, bm=bm, bn=bn, bk=bk,
                           interleave_products=interleave_products, output_dtype=output_dtype,
                           input_dtype=input_dtype, dot_precision=dot_precision)


def cubic_blocked_matmul(a, b, *, bm, bn, bk, epilogue=None, residual=None,
                         bias=None, rope_cos=None, rope_sin=None,
                         rope_scale=None, rope_head_dim=128, rope_eps=1e-6,
                         output_dtype="bfloat16", norm_scale=None, norm_eps=1e-6, dot_precision=None):
    """The matched cubic control: eight half-size products per K panel.

    ``dot_precision`` HIGH / HIGHEST multiplies the bf16 parts of each
    quadrant in 3 / 6 passes (``pass_product``); bf16 values have zero
    low-order parts, so bf16 inputs give the one-pass result.

    FP32 inputs (float32 values that are not bf16) take the same one-pass
    bf16 product as Strassen: each quadrant is rounded to bf16 at the
    product (``operand_round``; a no-op on bf16 values).

    ``_cubic_blocked_kernel`` (``experiments/qwen3/benchmark_cubic_control.py
    :76-113``): same quadrant split and four FP32 accumulators as Strassen,
    products (a0b0, a0b1, a2b0, a2b1, a1b2, a1b3, a3b2, a3b3) into quadrants
    (0, 1, 2, 3, 0, 1, 2, 3), no operand pre-adds. The reference control has
    no epilogues; the same epilogue code as Strassen is applied here so the
    fused sites can be compared against an identical cubic arm.
    """
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    m, k, n = _check_common(a, b, bm, bn, bk)
    passes = precision_passes(dot_precision)
    acc = [np.zeros((m // 2, n // 2), dtype=np.float32) for _ in range(4)]
    for step in range(k // bk):
        aq = _split_a(a, bm, bk, step)
        bq = _split_b(b, bn, bk, step)
        for ia, ib, q in CUBIC_PAIRS:
            acc[q] += pass_product(aq[ia], bq[ib], passes)
    return _epilogue(acc, m, n, bm, bn, epilogue=epilogue, residual=residual,
                     bias=bias, rope_cos=rope_cos, rope_sin=rope_sin,
                     rope_scale=rope_scale, rope_head_dim=rope_head_dim,
                     rope_eps=rope_eps, output_dtype=output_dtype, norm_scale=norm_scale,
                     norm_eps=norm_eps)


def _epilogue(acc, m, n, bm, bn, *, epilogue, residual, bias, rope_cos,
              rope_sin, rope_scale, rope_head_dim, rope_eps, output_dtype,
              norm_scale=None, norm_eps=1e-6):
    """Epilogues on the FP32 accumulators, then one bf16 rounding.

    ``strassen_pallas.py:739-879``: swiglu / geglu ``:762-777`` with the gate
    of ``:143-153``, residual_add
    ``:778-792``, qk_norm_rope ``:793-835``, bias_add ``:867-874``, plain
    store ``:875-879``.
    """
    hm, hn = bm // 2, bn // 2
    to_out = (lambda x: x.astype(np.float32)) if output_dtype == "float32" else bf16_round
    if epilogue is None:
        return to_out(_assemble(acc, m, n, bm, bn))
    if epilogue in ("swiglu", "geglu"):
        gate = silu if epilogue == "swiglu" else gelu_tanh
        top = gate(acc[0]) * acc[1]
        bottom = gate(acc[2]) * acc[3]
        # Output tile (bm, bn/2): rows [0,hm) from the top pair, [hm,bm) bottom.
        out = np.empty((m // bm, 2, hm, n // bn, hn), dtype=np.float32)
        out[:, 0] = top.reshape(m // bm, hm, n // bn, hn)
        out[:, 1] = bottom.reshape(m // bm, hm, n // bn, hn)
        return to_out(out.reshape(m, n // 2))
    if epilogue == "residual_add":
        res = _quadrants_of(np.asarray(residual, dtype=np.float32), bm, bn)
        return to_out(_assemble([acc[q] + res[q] for q in range(4)], m, n, bm, bn))
    if epilogue == "bias_add":
        left, right = _column_vector_quadrants(np.asarray(bias, dtype=np.float32), bn)
        quads = [acc[0] + left, acc[1] + right, acc[2] + left, acc[3] + right]
        return to_out(_assemble(quads, m, n, bm, bn))
    if epilogue == "qk_norm_rope":
        return to_out(_qk_norm_rope(acc, m, n, bm, bn, rope_cos, rope_sin,
                                    rope_scale, rope_head_dim, rope_eps))
    if epilogue == "norm_residual_add":
        # ``:836-866`` (bn == n): per row, recip = rsqrt((sum(left^2) +
        # sum(right^2)) / n + eps); out = half * recip * scale + residual.
        full = _assemble(acc, m, n, bm, bn)
        left, right = full[:, :n // 2], full[:, n // 2:]
        squares = (np.sum(left * left, axis=1, keepdims=True, dtype=np.float32)
                   + np.sum(right * right, axis=1, keepdims=True, dtype=np.float32))
        recip = (np.float32(1.0) / np.sqrt(squares * np.float32(1.0 / n) + np.float32(norm_eps))).astype(np.float32)
        scale = np.asarray(norm_scale, np.float32)
        return to_out(full * recip * scale + np.asarray(residual, np.float32))
    raise ValueError(f"unknown epilogue {epilogue!r}")


def _qk_norm_rope(acc, m, n, bm, bn, cos, sin, scale, head_dim, eps):
    """Per-head RMSNorm then RoPE on laid-out quadrants (``:793-835``).

    Within each (bm, bn) tile, quadrants 0/2 hold each head's first-half
    channels and 1/3 the matching second halves (``rope_weight_layout``), in
    contiguous head_dim/2-wide segments. Per row and head:
    ``sums = sum(a^2) + sum(b^2)`` over the segment (two separate segmented
    sums, ``:815-820``), ``recip = rsqrt(sums/head_dim + eps)``,
    ``a' = a*recip*gamma_a``, ``b' = b*recip*gamma_b``,
    ``out_a = a'cos - b'sin``, ``out_b = b'cos + a'sin`` with cos/sin read
    by output row (``:812-827``).
    """
    hm, hn = bm // 2, bn // 2
    seg = head_dim // 2
    cos = np.asarray(cos, dtype=np.float32)
    sin = np.asarray(sin, dtype=np.float32)
    scale = np.asarray(scale, dtype=np.float32)
    scale_a, scale_b = scale[:hn], scale[hn:]
    inverse_width = np.float32(1.0 / head_dim)
    eps = np.float32(eps)
    # Row-indexed tables for the top / bottom quadrant rows of every tile.
    rows = cos.reshape(m // bm, 2, hm, hn)
    srows = sin.reshape(m // bm, 2, hm, hn)
    outs = []
    for half in range(2):
        first = acc[2 * half].reshape(m // bm, hm, n // bn, hn)
        second = acc[2 * half + 1].reshape(m // bm, hm, n // bn, hn)
        c = rows[:, half][:, :, None, :]
        s = srows[:, half][:, :, None, :]
        fsq = (first * first).reshape(m // bm, hm, n // bn, hn // seg, seg)
        ssq = (second * second).reshape(m // bm, hm, n // bn, hn // seg, seg)
        sums = fsq.sum(axis=-1, dtype=np.float32) + ssq.sum(axis=-1, dtype=np.float32)
        recip = (np.float32(1.0) / np.sqrt(sums * inverse_width + eps)).astype(np.float32)
        recip = np.repeat(recip, seg, axis=-1)
        na = first * recip * scale_a
        nb = second * recip * scale_b
        out_a = na * c - nb * s
        out_b = nb * c + na * s
        outs.append((out_a.reshape(m // 2, n // 2), out_b.reshape(m // 2, n // 2)))
    quads = [outs[0][0], outs[0][1], outs[1][0], outs[1][1]]
    return _assemble(quads, m, n, bm, bn)


def native_matmul(a, b):
    """bf16 x bf16 with FP32 accumulation, one bf16 rounding.

    ``strassen_pallas.py:1414-1421`` / ``benchmark_common.py:17-24``.
    """
    return bf16_round(np.matmul(np.asarray(a, np.float32), np.asarray(b, np.float32)))


def high_precision_reference(a, b):
    """The FP32 HIGHEST oracle of ``benchmark_common.py:27-33``.

    Computed in float64 and rounded to float32 (at least as accurate as an
    FP32 HIGHEST product of the same bf16-valued inputs).
    """
    return np.matmul(np.asarray(a, np.float64), np.asarray(b, np.float64)).astype(np.float32)


def device_error(got, reference):
    """Error metrics of ``benchmark_common.py:36-60``."""
    got = np.asarray(got, dtype=np.float64)
    reference = np.asarray(reference, dtype=np.float64)
    delta = got - reference
    tiny = float(np.finfo(np.float32).tiny)
    max_abs = float(np.max(np.abs(delta))) if delta.size else 0.0
    return {
        "max_abs": max_abs,
        "rmse": float(np.sqrt(np.mean(delta * delta))) if delta.size else 0.0,
        "maxnorm_relative": max_abs / max(float(np.max(np.abs(reference))) if delta.size else 0.0, tiny),
        "l2_relative": float(np.linalg.norm(delta)) / max(float(np.linalg.norm(reference)), tiny),
    }


def host_uniform_inputs(shape, seed):
    """uniform[-1, 1] inputs of ``benchmark_common.py:63-69``, rounded to bf16
    as ``jnp.asarray(..., dtype=bfloat16)`` does (``:72-74``)."""
    m, k, n = shape
    rng = np.random.default_rng(seed)
    a = rng.uniform(-1.0, 1.0, (m, k)).astype(np.float32)
    b = rng.uniform(-1.0, 1.0, (k, n)).astype(np.float32)
    return bf16_round(a), bf16_round(b)


# ---------------------------------------------------------------------------
# Relayouts (pure column permutations) and unfused Qwen3 semantics
# ---------------------------------------------------------------------------

def swiglu_weight_layout_order(two_i, bn):
    """Column order of ``swiglu_weight_layout`` (``strassen_pallas.py:1381-1411``)."""
    if two_i % 2:
        raise ValueError(f"combined gate/up width {two_i} is not even")
    intermediate = two_i // 2
    half = bn // 2
    if intermediate % half:
        raise ValueError(f"intermediate {intermediate} is not divisible by bn//2={half}")
    order = []
    for block in range(intermediate // half):
        start = block * half
        order.extend(range(start, start + half))
        order.extend(range(intermediate + start, intermediate + start + half))
    return np.asarray(order, dtype=np.int64)


def swiglu_weight_layout(gate_up, bn):
    return np.asarray(gate_up)[:, swiglu_weight_layout_order(np.asarray(gate_up).shape[1], bn)]


def rope_weight_layout_order(n, bn, head_dim=128):
    """Column order of ``rope_weight_layout`` (``strassen_pallas.py:1315-1349``)."""
    if n % head_dim:
        raise ValueError(f"width {n} is not a multiple of head_dim {head_dim}")
    if bn % (2 * head_dim):
        raise ValueError(f"bn={bn} must be a multiple of 2*head_dim={2 * head_dim}")
    half_head = head_dim // 2
    heads = n // head_dim
    a_cols = [h * head_dim + j for h in range(heads) for j in range(half_head)]
    b_cols = [h * head_dim + half_head + j for h in range(heads) for j in range(half_head)]
    half = bn // 2
    if (n // 2) % half:
        raise ValueError(f"half width {n // 2} is not divisible by bn//2={half}")
    order = []
    for block in range((n // 2) // half):
        lo, hi = block * half, (block + 1) * half
        order.extend(a_cols[lo:hi])
        order.extend(b_cols[lo:hi])
    return np.asarray(order, dtype=np.int64)


def rope_weight_layout(weight, bn, head_dim=128):
    weight = np.asarray(weight)
    return weight[:, rope_weight_layout_order(weight.shape[1], bn, head_dim)]


def rope_layout_tables(cos, sin, half_width, head_dim=128):
    """``strassen_pallas.py:1352-1368``."""
    half_head = head_dim // 2
    if half_width % half_head:
        raise ValueError(f"half_width {half_width} is not a multiple of {half_head}")
    repeats = half_width // half_head
    return (np.tile(np.asarray(cos)[:, :half_head], (1, repeats)),
            np.tile(np.asarray(sin)[:, :half_head], (1, repeats)))


def rope_scale_layout(scale, bn, head_dim=128):
    """``strassen_pallas.py:1371-1378``."""
    half_head = head_dim // 2
    repeats = (bn // 2) // half_head
    scale = np.asarray(scale)
    return np.concatenate((np.tile(scale[:half_head], repeats),
                           np.tile(scale[half_head:], repeats)))


def rope_layout_to_heads(flat, heads, bn, batch, seq, head_dim=128):
    """Inverse regroup of a qk_norm_rope output
    (``experiments/qwen3/benchmark_qwen3_32b_layer.py:322-341``)."""
    half_head = head_dim // 2
    heads_per_half = (bn // 2) // half_head
    blocks = (heads * head_dim) // bn
    tokens = batch * seq
    return (np.asarray(flat).reshape(tokens, blocks, 2, heads_per_half, half_head)
            .transpose(0, 1, 3, 2, 4).reshape(batch, seq, heads, head_dim))


def rope_values(seq, head_dim=128, theta=1e6):
    """bf16 cos/sin tables (``benchmark_qwen3_32b_layer.py:258-267``)."""
    positions = np.arange(seq, dtype=np.float32)[:, None]
    inverse = (np.float32(1.0) / (np.float32(theta) ** (np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)))).astype(np.float32)
    angles = np.concatenate((positions * inverse[None, :],) * 2, axis=-1).astype(np.float32)
    return bf16_round(np.cos(angles)), bf16_round(np.sin(angles))


def rms_norm(x, scale, eps=1e-6):
    """``benchmark_qwen3_32b_layer.py:270-276`` (FP32 math, bf16 output)."""
    x32 = np.asarray(x, dtype=np.float32)
    mean = np.mean(x32 * x32, axis=-1, keepdims=True, dtype=np.float32)
    return bf16_round(x32 * (np.float32(1.0) / np.sqrt(mean + np.float32(eps))) * np.asarray(scale, np.float32))


def apply_rope(x, cos, sin):
    """``benchmark_qwen3_32b_layer.py:279-284``: x (B,S,H,D), cos/sin (S,D)."""
    x32 = np.asarray(x, dtype=np.float32)
    first, second = np.split(x32, 2, axis=-1)
    rotated = np.concatenate((-second, first), axis=-1)
    c = np.asarray(cos, np.float32)[None, :, None, :]
    s = np.asarray(sin, np.float32)[None, :, None, :]
    return bf16_round(x32 * c + rotated * s)
