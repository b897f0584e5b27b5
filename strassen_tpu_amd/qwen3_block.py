"""A Qwen3 decoder block whose GEMM sites run on the gfx950 kernels.

Mirrors the reference's layer (``experiments/qwen3/benchmark_qwen3_32b_layer.py``:
``rms_norm`` :270-276, ``apply_rope`` :279-284, ``rope_values`` :258-267,
``attention_prefix`` :344-377, ``make_layer`` :380-398) and the fused arm of
``benchmark_qwen3_32b_full_layer_product_inference.py:119-176``. In the
``"strassen"`` and ``"cubic"`` arms:

* q and k carry their per-head RMSNorm and RoPE in the ``qk_norm_rope`` epilogue,
  and share one packed activation;
* o and down fold the residual add into ``residual_add``;
* gate|up folds SwiGLU into ``swiglu``.

v runs on hipBLASLt (``torch.matmul``), and attention on torch's fused SDPA
kernels. The ``"hipblaslt"`` arm is the reference's unfused native layer:
``torch.matmul`` GEMMs with the norms, RoPE, SwiGLU and residual adds as
separate torch ops. The ``"cubic_unfused"`` arm is the cubic arm of the
reference's published block run (``cubic_pallas`` with extended sites o and
down, :63-76, :146-170): the cubic kernel for o, gate|up and down with no
fused epilogue (the reference's ``cubic_matmul`` takes none), SwiGLU and the
residual adds as torch ops, and q, k and v on hipBLASLt with torch's norms
and RoPE. Weights are random-init (there is no network to fetch
checkpoints); a caller may supply real ones through ``BlockWeights``.
"""

from __future__ import annotations

import dataclasses

import torch

from . import _lib
from .layouts import (rope_layout_tables, rope_layout_to_heads, rope_scale_layout, rope_weight_layout,
                      swiglu_weight_layout)
from .packing import cubic_weight_layout, pack_activation, strassen_weight_layout
from .strassen import cubic_matmul, strassen_matmul

__all__ = ["Qwen3Dims", "QWEN3_32B", "BlockWeights", "PreparedBlock", "rms_norm", "apply_rope", "rope_values",
           "attention", "block_forward", "ARMS"]

ARMS = ("strassen", "cubic", "hipblaslt", "cubic_unfused")


@dataclasses.dataclass(frozen=True)
class Qwen3Dims:
    hidden: int
    ffn: int
    heads: int
    kv_heads: int
    head_dim: int = 128
    eps: float = 1e-6
    theta: float = 1e6


# Qwen/Qwen3-32B (``benchmark_qwen3_32b_layer.py:43-82``).
QWEN3_32B = Qwen3Dims(hidden=5120, ffn=25600, heads=64, kv_heads=8)


@dataclasses.dataclass
class BlockWeights:
    """One block's parameters, GEMM weights stored ``[in, out]`` (the
    reference's transposed checkpoint tensors, ``:401-431``); ``gate_up`` is
    ``[gate | up]`` along the output axis."""

    attention_norm: torch.Tensor
    query: torch.Tensor
    query_norm: torch.Tensor
    key: torch.Tensor
    key_norm: torch.Tensor
    value: torch.Tensor
    attention_output: torch.Tensor
    mlp_norm: torch.Tensor
    gate_up: torch.Tensor
    mlp_down: torch.Tensor

    @classmethod
    def random_init(cls, dims, device, seed=0, std=0.02):
        """Random-init bf16 weights: projections ~N(0, std), norm scales
        ~1 + N(0, 0.1). Projections are ``[in, out]`` views of ``[out, in]``
        storage, as ``nn.Linear`` keeps them."""
        g = torch.Generator(device=device).manual_seed(seed)

        def linear(fan_in, fan_out):
            return (torch.randn(fan_out, fan_in, device=device, generator=g) * std).to(torch.bfloat16).t()

        def scale(n):
            return (1.0 + 0.1 * torch.randn(n, device=device, generator=g)).to(torch.bfloat16)

        h, q, kv = dims.hidden, dims.heads * dims.head_dim, dims.kv_heads * dims.head_dim
        return cls(
            attention_norm=scale(h), query=linear(h, q), query_norm=scale(dims.head_dim),
            key=linear(h, kv), key_norm=scale(dims.head_dim), value=linear(h, kv),
            attention_output=linear(q, h), mlp_norm=scale(h), gate_up=linear(h, 2 * dims.ffn),
            mlp_down=linear(dims.ffn, h))


def rms_norm(x, scale, eps):
    """``x * rsqrt(mean(x^2) + eps) * scale`` in FP32, bf16 out (``:270-276``)."""
    x32 = x.float()
    return (x32 * torch.rsqrt(x32.square().mean(-1, keepdim=True) + eps) * scale.float()).to(torch.bfloat16)


def apply_rope(x, cos, sin):
    """RoPE on ``[batch, seq, heads, head_dim]`` with ``[seq, head_dim]``
    tables (``:279-284``)."""
    first, second = x.float().chunk(2, dim=-1)
    rotated = torch.cat((-second, first), dim=-1)
    return (x.float() * cos[None, :, None, :].float() + rotated * sin[None, :, None, :].float()).to(torch.bfloat16)


def rope_values(seq, head_dim, theta, device):
    """bf16 cos / sin tables ``[seq, head_dim]`` (``:258-267``)."""
    positions = torch.arange(seq, dtype=torch.float32, device=device)[:, None]
    inverse = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim))
    angles = torch.cat((positions * inverse[None, :],) * 2, dim=-1)
    return torch.cos(angles).to(torch.bfloat16), torch.sin(angles).to(torch.bfloat16)


def attention(query, key, value):
    """Causal grouped-query attention, ``[batch, seq, heads, head_dim]`` in
    and out (``jax.nn.dot_product_attention(..., is_causal=True)``, ``:370-372``).

    Runs on torch's fused SDPA kernels only (flash or memory-efficient); the
    math backend is excluded because its batched bf16 products on transposed
    views are not safe on this GPU, so an unsupported shape raises instead.
    """
    from torch.nn.attention import SDPBackend, sdpa_kernel

    groups = query.shape[2] // key.shape[2]
    q = query.transpose(1, 2).contiguous()
    k = key.repeat_interleave(groups, dim=2).transpose(1, 2).contiguous()
    v = value.repeat_interleave(groups, dim=2).transpose(1, 2).contiguous()
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        out = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
    return out.transpose(1, 2)


class PreparedBlock:
    """A block's weights laid out for one arm, built once and kept on the
    device (the reference caches relayouts per layer the same way)."""

    def __init__(self, weights, dims, arm, *, batch, seq, tile=(1024, 1024, 512)):
        if arm not in ARMS:
            raise ValueError(f"unknown arm {arm!r}; expected one of {ARMS}")
        self.weights, self.dims, self.arm = weights, dims, arm
        self.batch, self.seq, self.tile = batch, seq, tuple(tile)
        device = weights.query.device
        self.cos, self.sin = rope_values(seq, dims.head_dim, dims.theta, device)
        if arm == "hipblaslt":
            return
        bm, bn, bk = self.tile
        self.algo = _lib.SMX_ALGO_STRASSEN if arm == "strassen" else _lib.SMX_ALGO_CUBIC
        pack = strassen_weight_layout if arm == "strassen" else cubic_weight_layout
        if arm == "cubic_unfused":
            # plain [gate | up] columns: SwiGLU runs on the GEMM's output
            self.attention_output = pack(weights.attention_output, bn, bk)
            self.gate_up = pack(weights.gate_up, bn, bk)
            self.mlp_down = pack(weights.mlp_down, bn, bk)
            return
        self.query = pack(rope_weight_layout(weights.query, bn, dims.head_dim), bn, bk)
        self.key = pack(rope_weight_layout(weights.key, bn, dims.head_dim), bn, bk)
        self.attention_output = pack(weights.attention_output, bn, bk)
        self.gate_up = pack(swiglu_weight_layout(weights.gate_up, bn), bn, bk)
        self.mlp_down = pack(weights.mlp_down, bn, bk)
        tokens_cos = self.cos.repeat(batch, 1)
        tokens_sin = self.sin.repeat(batch, 1)
        self.rope_cos, self.rope_sin = rope_layout_tables(tokens_cos, tokens_sin, bn // 2, dims.head_dim)
        self.query_scale = rope_scale_layout(weights.query_norm, bn, dims.head_dim)
        self.key_scale = rope_scale_layout(weights.key_norm, bn, dims.head_dim)

    def gemm(self, a, b, **kw):
        bm, bn, bk = self.tile
        if self.arm == "strassen":
            return strassen_matmul(a, b, bm=bm, bn=bn, bk=bk, interleave_products=True, **kw)
        return cubic_matmul(a, b, bm=bm, bn=bn, bk=bk, **kw)


def block_forward(x, block):
    """One decoder block: ``x [batch*seq, hidden]`` bf16 -> same shape."""
    d, w = block.dims, block.weights
    batch, seq = block.batch, block.seq
    normalized = rms_norm(x, w.attention_norm, d.eps)
    if block.arm in ("hipblaslt", "cubic_unfused"):
        query = torch.matmul(normalized, w.query).view(batch, seq, d.heads, d.head_dim)
        key = torch.matmul(normalized, w.key).view(batch, seq, d.kv_heads, d.head_dim)
        query = apply_rope(rms_norm(query, w.query_norm, d.eps), block.cos, block.sin)
        key = apply_rope(rms_norm(key, w.key_norm, d.eps), block.cos, block.sin)
    else:
        bn = block.tile[1]
        shared = pack_activation(normalized, block.algo, block.tile[0], block.tile[2])
        qk = dict(epilogue="qk_norm_rope", rope_cos=block.rope_cos, rope_sin=block.rope_sin,
                  rope_head_dim=d.head_dim, rope_eps=d.eps)
        query = rope_layout_to_heads(block.gemm(shared, block.query, rope_scale=block.query_scale, **qk),
                                     d.heads, bn, batch, seq, d.head_dim)
        key = rope_layout_to_heads(block.gemm(shared, block.key, rope_scale=block.key_scale, **qk),
                                   d.kv_heads, bn, batch, seq, d.head_dim)
    value = torch.matmul(normalized, w.value).view(batch, seq, d.kv_heads, d.head_dim)
    attended = attention(query, key, value).reshape(batch * seq, d.heads * d.head_dim)
    if block.arm == "hipblaslt":
        residual = (x.float() + torch.matmul(attended, w.attention_output).float()).to(torch.bfloat16)
        normalized = rms_norm(residual, w.mlp_norm, d.eps)
        gate, up = torch.matmul(normalized, w.gate_up).chunk(2, dim=-1)
        activated = (torch.nn.functional.silu(gate.float()) * up.float()).to(torch.bfloat16)
        return (residual.float() + torch.matmul(activated, w.mlp_down).float()).to(torch.bfloat16)
    if block.arm == "cubic_unfused":
        residual = (x.float() + block.gemm(attended, block.attention_output).float()).to(torch.bfloat16)
        normalized = rms_norm(residual, w.mlp_norm, d.eps)
        gate, up = block.gemm(normalized, block.gate_up).chunk(2, dim=-1)
        activated = (torch.nn.functional.silu(gate.float()) * up.float()).to(torch.bfloat16)
        return (residual.float() + block.gemm(activated, block.mlp_down).float()).to(torch.bfloat16)
    residual = block.gemm(attended, block.attention_output, epilogue="residual_add", residual=x)
    normalized = rms_norm(residual, w.mlp_norm, d.eps)
    activated = block.gemm(normalized, block.gate_up, epilogue="swiglu")
    return block.gemm(activated, block.mlp_down, epilogue="residual_add", residual=residual)
