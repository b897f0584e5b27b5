"""Offline weight and table relayouts for the fused epilogues (torch).

Same index maps as the reference's ``strassen_pallas.py:1315-1411`` and the
inverse regroup of ``experiments/qwen3/benchmark_qwen3_32b_layer.py:322-341``.
Column permutations preserve a K-contiguous weight layout (a ``[K, N]`` view
of ``[N, K]`` storage), which is the layout the gfx950 kernel reads directly.
"""

from __future__ import annotations

import torch

__all__ = [
    "swiglu_weight_layout", "rope_weight_layout", "rope_layout_tables",
    "rope_scale_layout", "rope_layout_to_heads", "swiglu_layout_order",
    "rope_layout_order", "k_contiguous", "is_k_contiguous",
]


def is_k_contiguous(b):
    """True when ``b`` ([K, N]) is a transposed view of contiguous [N, K]."""
    return b.dim() == 2 and b.stride(0) == 1 and (b.shape[1] <= 1 or b.stride(1) >= b.shape[0])


def k_contiguous(b):
    """Return ``b`` ([K, N]) as a K-contiguous view of ``[N, K]`` storage.

    Projection weights stored ``[out, in]`` already are (``w.t()``); a
    row-major ``[K, N]`` weight is transposed once here. Do this offline,
    like the other relayouts: ``strassen_matmul`` would otherwise repeat it
    on every call.
    """
    if is_k_contiguous(b):
        return b
    return b.t().contiguous().t()


def _permute_columns(w, order):
    order = torch.as_tensor(order, dtype=torch.long, device=w.device)
    if is_k_contiguous(w):
        return w.t().index_select(0, order).t()
    return w.index_select(1, order)


def swiglu_layout_order(two_i, bn):
    """``strassen_pallas.py:1397-1411``: blocks ``gate[h*b:h*(b+1)] | up[...]``
    with ``h = bn // 2``."""
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
    return order


def swiglu_weight_layout(gate_up, bn):
    """Reorder a combined ``[gate | up]`` weight so SwiGLU fuses in-kernel
    (``strassen_pallas.py:1381-1411``): quadrants 0/2 of every output tile
    become gate channels and 1/3 the matching up channels."""
    return _permute_columns(gate_up, swiglu_layout_order(gate_up.shape[1], bn))


def rope_layout_order(n, bn, head_dim=128):
    """``strassen_pallas.py:1329-1349``."""
    if n % head_dim:
        raise ValueError(f"width {n} is not a multiple of head_dim {head_dim}")
    if bn % (2 * head_dim):
        raise ValueError(
            f"bn={bn} must be a multiple of 2*head_dim={2 * head_dim} so each "
            "tile half holds whole heads")
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
    return order


def rope_weight_layout(weight, bn, head_dim=128):
    """Reorder a q/k projection weight so q_norm+RoPE fuses in-kernel
    (``strassen_pallas.py:1315-1349``): every tile holds ``a`` halves of whole
    heads in quadrants 0/2 and the matching ``b`` halves in 1/3."""
    return _permute_columns(weight, rope_layout_order(weight.shape[1], bn, head_dim))


def rope_layout_tables(cos, sin, half_width, head_dim=128):
    """Half-width RoPE tables matching ``rope_weight_layout``
    (``strassen_pallas.py:1352-1368``)."""
    half_head = head_dim // 2
    if half_width % half_head:
        raise ValueError(f"half_width {half_width} is not a multiple of {half_head}")
    repeats = half_width // half_head
    return (cos[:, :half_head].repeat(1, repeats).contiguous(),
            sin[:, :half_head].repeat(1, repeats).contiguous())


def rope_scale_layout(scale, bn, head_dim=128):
    """Per-head RMSNorm scale reordered to match ``rope_weight_layout``
    (``strassen_pallas.py:1371-1378``)."""
    half_head = head_dim // 2
    repeats = (bn // 2) // half_head
    return torch.cat((scale[:half_head].repeat(repeats), scale[half_head:].repeat(repeats)))


def rope_layout_to_heads(flat, heads, bn, batch, seq, head_dim=128):
    """Regroup a ``qk_norm_rope`` output ``[tokens, heads*head_dim]`` into
    ``(batch, seq, heads, head_dim)`` head order
    (``experiments/qwen3/benchmark_qwen3_32b_layer.py:322-341``)."""
    half_head = head_dim // 2
    heads_per_half = (bn // 2) // half_head
    blocks = (heads * head_dim) // bn
    return (flat.reshape(batch * seq, blocks, 2, heads_per_half, half_head)
            .transpose(2, 3).reshape(batch, seq, heads, head_dim))
