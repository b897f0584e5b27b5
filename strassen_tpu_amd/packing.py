"""Packed operands: the layout the packed gfx950 kernel streams into LDS.

A projection weight is static, so the classical B operand sums of
``strassen_pallas.py:324-379`` (B0+B3, B0, B1-B3, B2-B0, B3, B0+B1, B2+B3,
each rounded once to bf16) are formed once, offline, like the reference's
``swiglu_weight_layout`` / ``rope_weight_layout`` relayouts
(``strassen_pallas.py:1315-1411``); the activation's A sums (A0+A3, A2+A3,
A0, A3, A0+A1, A2-A0, A1-A3) are formed once per call by a bandwidth-bound
pass. The cubic control packs the raw quadrants (four operands) the same
way, so both arms stream identical fragment layouts. Results are identical
to forming the sums inside the GEMM.

Storage (``smx_pack_operand``): for ``R`` product rows (``M/2`` of A,
``N/2`` of B) and product depth ``K/2``, ``[R/128][K/32][nops][4][64][8]``
bf16, i.e. 1 KB MFMA operand fragments in lane order; ``nops`` is 7
(Strassen) or 4 (cubic), so a packed operand holds ``nops/4`` times the
elements of the original.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

__all__ = ["PackedOperand", "pack_operand", "strassen_weight_layout", "cubic_weight_layout",
           "pack_activation"]

_ALGOS = {_lib.SMX_ALGO_STRASSEN: "strassen", _lib.SMX_ALGO_CUBIC: "cubic"}


class PackedOperand:
    """A bf16 operand packed for one algorithm and quadrant tile.

    ``side`` is ``"lhs"`` for an activation ``a [M, K]`` (``tile_rows`` =
    bm) or ``"rhs"`` for a weight ``b [K, N]`` (``tile_rows`` = bn). Pass it
    to ``strassen_matmul`` / ``cubic_matmul`` in place of the tensor, with
    the same tile.
    """

    def __init__(self, data, *, algo, side, rows, k, tile_rows, bk, formula="classical", block_permutation=0):
        self.data = data
        self.algo, self.side = int(algo), side
        self.rows, self.k, self.tile_rows, self.bk = int(rows), int(k), int(tile_rows), int(bk)
        self.formula, self.block_permutation = formula, int(block_permutation)

    # The parts of the tensor interface the callers' argument checks use.
    @property
    def shape(self):
        return torch.Size((self.rows, self.k) if self.side == "lhs" else (self.k, self.rows))

    @property
    def dtype(self):
        return self.data.dtype

    @property
    def device(self):
        return self.data.device

    def dim(self):
        return 2

    def __repr__(self):
        variant = "" if self.algo != _lib.SMX_ALGO_STRASSEN else \
            f", formula={self.formula}, block_permutation={self.block_permutation}"
        return (f"PackedOperand({_ALGOS[self.algo]}, {self.side}, shape={tuple(self.shape)}, "
                f"tile_rows={self.tile_rows}, bk={self.bk}{variant}, device={self.device})")


def packed_bytes(algo, rows, k):
    out = ctypes.c_int64()
    _lib.check(_lib.load().smx_packed_bytes(algo, rows, k, ctypes.byref(out)))
    return out.value


def pack_operand(x, *, algo, side, tile_rows, bk, formula="classical", block_permutation=0):
    """Pack ``x`` (bf16 on the HIP device): ``a [M, K]`` for ``side="lhs"``,
    the same ``a`` stored transposed as ``[K, M]`` for ``side="lhs_t"``, or a
    weight ``b [K, N]`` for ``side="rhs"`` (any strides; a K-contiguous view
    of ``[N, K]`` storage is read in place). Runs asynchronously on torch's
    current stream. Strassen operands carry the operand sums of
    ``formula`` ("classical", "dual" or "powers") after the quadrant swaps of
    ``block_permutation``; both operands of a GEMM must be packed alike."""
    if formula not in _lib.SMX_FORMULA:
        raise ValueError("formula_variant must be 'classical', 'dual', or 'powers'")
    if side not in ("lhs", "rhs", "lhs_t"):
        raise ValueError("side must be 'lhs', 'lhs_t' or 'rhs'")
    if algo not in _ALGOS:
        raise ValueError(f"algo must be {_lib.SMX_ALGO_STRASSEN} or {_lib.SMX_ALGO_CUBIC}")
    if x.dim() != 2:
        raise ValueError("pack_operand expects a rank-2 matrix")
    if x.dtype != torch.bfloat16:
        raise ValueError("pack_operand expects bf16")
    if x.device.type != "cuda":
        raise ValueError("pack_operand runs on the HIP device")
    if side == "lhs_t":
        src = x  # [K, rows], rows contiguous
        k, rows = src.shape
        if src.stride(1) != 1 or src.data_ptr() % 16:
            src = src.contiguous()
    else:
        src = x if side == "lhs" else x.t()  # rows x K, K contiguous
        rows, k = src.shape
        if src.stride(1) != 1 or src.stride(0) % 8 or src.data_ptr() % 16:
            src = src.contiguous()
    if rows % tile_rows or k % bk:
        raise ValueError(f"operand [{rows}, {k}] (rows x K) does not tile by ({tile_rows}, {bk})")
    nbytes = packed_bytes(algo, rows, k)
    data = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=x.device)
    side_id = {"lhs": _lib.SMX_SIDE_LHS, "rhs": _lib.SMX_SIDE_RHS, "lhs_t": _lib.SMX_SIDE_LHS_T}[side]
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = _lib.load().smx_pack_operand(algo, _lib.SMX_FORMULA[formula], block_permutation, side_id, rows, k,
                                      _lib.ptr(src), src.stride(0), tile_rows, bk, _lib.ptr(data), stream)
    _lib.check(rc)
    return PackedOperand(data, algo=algo, side="rhs" if side == "rhs" else "lhs", rows=rows, k=k,
                         tile_rows=tile_rows, bk=bk, formula=formula, block_permutation=block_permutation)


def strassen_weight_layout(b, bn, bk, *, formula_variant="classical", block_permutation=0):
    """Pre-sum and pack a bf16 ``[K, N]`` weight for ``strassen_matmul``
    with the tile ``(bn, bk)`` (and the formula / block permutation the
    calls will use)."""
    return pack_operand(b, algo=_lib.SMX_ALGO_STRASSEN, side="rhs", tile_rows=bn, bk=bk,
                        formula=formula_variant, block_permutation=block_permutation)


def cubic_weight_layout(b, bn, bk):
    """Pack a bf16 ``[K, N]`` weight's quadrants for ``cubic_matmul`` with
    the tile ``(bn, bk)``."""
    return pack_operand(b, algo=_lib.SMX_ALGO_CUBIC, side="rhs", tile_rows=bn, bk=bk)


def pack_activation(a, algo, bm, bk, *, formula_variant="classical", block_permutation=0):
    """Pack an activation ``a [M, K]`` once for several GEMMs that share it
    (e.g. the q, k and v projections)."""
    return pack_operand(a, algo=algo, side="lhs", tile_rows=bm, bk=bk, formula=formula_variant,
                        block_permutation=block_permutation)
