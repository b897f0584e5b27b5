"""Pre-summed Strassen weights: the seven B operands of every (bk, bn) tile.

A projection weight is static, so the classical B operand sums of
``strassen_pallas.py:324-379`` (B0+B3, B0, B1-B3, B2-B0, B3, B0+B1, B2+B3,
each rounded once to bf16) can be formed once, offline, exactly like the
reference's ``swiglu_weight_layout`` / ``rope_weight_layout`` relayouts
(``strassen_pallas.py:1315-1411``). The GEMM then forms only the A sums at run
time. Storage is ``[N/2 * 7, K/2]`` bf16 (7/4 of the weight): row
``p*7 + o`` holds operand ``o`` of product-space column ``p`` over the
product-space depth. The result is identical to forming the sums in-kernel.
"""

from __future__ import annotations

import torch

from . import _lib

__all__ = ["StrassenWeight", "strassen_weight_layout"]


class StrassenWeight:
    """A ``[K, N]`` weight stored as its seven pre-summed Strassen operands
    for the quadrant tile ``(bn, bk)``. Pass it to ``strassen_matmul`` in
    place of ``b`` (with the same ``bn`` and ``bk``)."""

    def __init__(self, data, k, n, bn, bk):
        self.data = data
        self.k, self.n, self.bn, self.bk = int(k), int(n), int(bn), int(bk)

    # The parts of the tensor interface strassen_matmul's checks use.
    @property
    def shape(self):
        return torch.Size((self.k, self.n))

    @property
    def dtype(self):
        return self.data.dtype

    @property
    def device(self):
        return self.data.device

    def dim(self):
        return 2

    def __repr__(self):
        return (f"StrassenWeight(k={self.k}, n={self.n}, bn={self.bn}, bk={self.bk}, "
                f"device={self.device}, storage={tuple(self.data.shape)})")


def strassen_weight_layout(b, bn, bk):
    """Pre-sum a bf16 ``[K, N]`` weight (any strides; a K-contiguous view of
    ``[N, K]`` storage is read in place) for the tile ``(bn, bk)``.

    Runs on the weight's HIP device (``smx_strassen_weight_layout``) on
    torch's current stream.
    """
    if b.dim() != 2:
        raise ValueError("strassen_weight_layout expects a rank-2 [K, N] weight")
    if b.dtype != torch.bfloat16:
        raise ValueError("strassen_weight_layout expects a bf16 weight")
    if b.device.type != "cuda":
        raise ValueError("strassen_weight_layout runs on the HIP device")
    k, n = b.shape
    if n % bn or k % bk or bn % 2 or bk % 16:
        raise ValueError(f"weight [{k}, {n}] does not tile by (bk={bk}, bn={bn}) "
                         "with even bn and bk a multiple of 16")
    bt = b.t()
    if bt.stride(1) != 1 or bt.stride(0) % 8:
        bt = bt.contiguous()
    out = torch.empty((n // 2 * 7, k // 2), dtype=torch.bfloat16, device=b.device)
    lib = _lib.load()
    stream = torch.cuda.current_stream(b.device).cuda_stream
    rc = lib.smx_strassen_weight_layout(n, k, _lib.ptr(bt), bt.stride(0), bn, bk, _lib.ptr(out),
                                        out.stride(0), stream)
    _lib.check(rc)
    return StrassenWeight(out, k, n, bn, bk)
