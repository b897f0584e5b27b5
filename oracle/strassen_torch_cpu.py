"""Torch-CPU restatement of the reference's tile-local classical Strassen GEMM.

TEST INFRASTRUCTURE ONLY: the timed CPU baseline of ``bench.py`` (the
reference's own JAX-CPU path cannot run where the GPU is) and nothing else.
The product package never imports it.

It computes what ``oracle.strassen_ref.strassen_matmul`` computes for the
classical formula with no epilogue, with torch's CPU kernels instead of
numpy's, so that the baseline runs on the same BLAS-threaded library the
rest of the host stack uses:

* every (bm, bn, bk) tile is split into 2x2 quadrants
  (``strassen_pallas.py:188-204``), stacked over tiles into one
  (M/2 x K/2) by (K/2 x N/2) product per quadrant pair;
* the seven operand sums are formed in bf16, each the exact sum rounded once
  to bf16 (``:324-379``);
* products are FP32 matmuls, added to four FP32 quadrant accumulators in the
  reference's order (plain ``:566-573`` or interleaved ``:556-565``);
* the result is rounded once to bf16.

Pinned by ``tests/test_oracle.py``: exact-integer known answers (the result
equals ``A @ B`` bit for bit) and agreement with the numpy oracle on random
bf16 inputs to within the FP32 summation-order difference of the two BLAS
libraries (one bf16 ulp).
"""

from __future__ import annotations

import torch

from .strassen_ref import INTERLEAVED_ORDER, PLAIN_ORDER, PRODUCT_UPDATES


def _quadrant_planes(x, rows_per_tile, cols_per_tile):
    """Four quadrant planes of every (rows_per_tile x cols_per_tile) tile of
    x, each stacked over the tiles: plane (r, c) has shape (R/2, C/2)."""
    rows, cols = x.shape
    hr, hc = rows_per_tile // 2, cols_per_tile // 2
    v = x.reshape(rows // rows_per_tile, 2, hr, cols // cols_per_tile, 2, hc)
    return tuple(v[:, r, :, :, c, :].reshape(rows // 2, cols // 2) for r in range(2) for c in range(2))


def strassen_matmul(a, b, *, bm, bn, bk, interleave_products=True):
    """``a @ b`` (bf16 CPU tensors) with one tile-local classical Strassen
    level; returns a bf16 tensor."""
    m, k = a.shape
    k2, n = b.shape
    if k != k2 or m % bm or n % bn or k % bk or bm % 2 or bn % 2 or bk % 2:
        raise ValueError("shapes must agree and divide into even tiles")
    a = a.to(torch.bfloat16)
    b = b.to(torch.bfloat16)
    order = INTERLEAVED_ORDER if interleave_products else PLAIN_ORDER
    acc = [torch.zeros(m // 2, n // 2, dtype=torch.float32) for _ in range(4)]
    for step in range(k // bk):
        # A quadrants: (row half, K half) of each bm x bk tile of the panel.
        a0, a1, a2, a3 = _quadrant_planes(a[:, step * bk:(step + 1) * bk], bm, bk)
        # B quadrants: (K half, column half) of each bk x bn tile.
        b0, b1, b2, b3 = _quadrant_planes(b[step * bk:(step + 1) * bk, :], bk, bn)
        # bf16 + bf16 in torch rounds the exact sum once to bf16.
        ops = {
            1: (a0 + a3, b0 + b3), 2: (a2 + a3, b0), 3: (a0, b1 - b3), 4: (a3, b2 - b0),
            5: (a0 + a1, b3), 6: (a2 - a0, b0 + b1), 7: (a1 - a3, b2 + b3),
        }
        for p in order:
            s, t = ops[p]
            value = torch.matmul(s.float(), t.float())
            for q, sign in PRODUCT_UPDATES[p]:
                if sign > 0:
                    acc[q] += value
                else:
                    acc[q] -= value
    out = torch.empty(m, n, dtype=torch.float32)
    view = out.view(m // bm, 2, bm // 2, n // bn, 2, bn // 2)
    for q in range(4):
        view[:, q >> 1, :, :, q & 1, :] = acc[q].view(m // bm, bm // 2, n // bn, bn // 2)
    return out.to(torch.bfloat16)
