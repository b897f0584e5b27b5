"""Real Qwen3 weights from local safetensors files.

The reference streams one layer's tensors over HTTP range requests from a
sharded Hugging Face checkpoint (``ShardedSafetensors``,
``experiments/qwen3/benchmark_qwen3_32b_layer.py:160-224``) and assembles
the block parameters in ``load_params`` (``:401-431``). There is no network
here, so ``LocalSafetensors`` reads the same checkpoint layout from disk: a
directory holding ``model.safetensors.index.json`` and its shards, a
directory with a single ``model.safetensors``, or one ``.safetensors`` file.
Tensors are memory-mapped and only the requested ones are read.
"""

from __future__ import annotations

import hashlib
import json
import os

import torch
from safetensors import safe_open

from .qwen3_block import BlockWeights, Qwen3Dims

__all__ = ["LocalSafetensors", "load_block_weights", "dims_from_config", "TENSOR_PREFIX"]

TENSOR_PREFIX = "model"
INDEX = "model.safetensors.index.json"


class LocalSafetensors:
    """Name -> tensor access over a local (possibly sharded) checkpoint."""

    def __init__(self, path):
        if os.path.isdir(path):
            index = os.path.join(path, INDEX)
            if os.path.exists(index):
                with open(index) as f:
                    weight_map = json.load(f)["weight_map"]
                self.shard_of = {name: os.path.join(path, shard) for name, shard in weight_map.items()}
            else:
                single = os.path.join(path, "model.safetensors")
                if not os.path.exists(single):
                    raise FileNotFoundError(f"{path} holds neither {INDEX} nor model.safetensors")
                self.shard_of = self._names_of(single)
        else:
            self.shard_of = self._names_of(path)
        self._open = {}

    @staticmethod
    def _names_of(file):
        with safe_open(file, framework="pt", device="cpu") as f:
            return {name: file for name in f.keys()}

    def names(self):
        return sorted(self.shard_of)

    def tensor(self, name, *, device="cpu", digest=None):
        """The bf16 tensor ``name`` on ``device``; non-bf16 tensors are
        refused as the reference does. If ``digest`` is a dict, the SHA-256
        of the raw bytes is recorded in it under ``name``."""
        if name not in self.shard_of:
            raise KeyError(f"{name} is not in the checkpoint")
        file = self.shard_of[name]
        handle = self._open.get(file)
        if handle is None:
            handle = self._open[file] = safe_open(file, framework="pt", device="cpu")
        value = handle.get_tensor(name)
        if value.dtype != torch.bfloat16:
            raise ValueError(f"{name} has dtype {value.dtype}")
        if digest is not None:
            digest[name] = hashlib.sha256(value.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()
        return value.to(device)


def load_block_weights(checkpoint, layer, *, device, prefix=TENSOR_PREFIX, digest=None):
    """``BlockWeights`` of decoder layer ``layer``. Projections keep their
    checkpoint storage ``[out, in]`` and are viewed ``[in, out]`` (the
    reference transposes them, ``:404-406``); gate and up are stored
    stacked as ``[2*ffn, in]`` and viewed ``[in, 2*ffn] = [gate | up]``, so
    every GEMM weight is K-contiguous."""
    if not isinstance(checkpoint, LocalSafetensors):
        checkpoint = LocalSafetensors(checkpoint)
    base = f"{prefix}.layers.{layer}."

    def get(name):
        return checkpoint.tensor(base + name, device=device, digest=digest)

    gate = get("mlp.gate_proj.weight")
    up = get("mlp.up_proj.weight")
    return BlockWeights(
        attention_norm=get("input_layernorm.weight"),
        query=get("self_attn.q_proj.weight").t(),
        query_norm=get("self_attn.q_norm.weight"),
        key=get("self_attn.k_proj.weight").t(),
        key_norm=get("self_attn.k_norm.weight"),
        value=get("self_attn.v_proj.weight").t(),
        attention_output=get("self_attn.o_proj.weight").t(),
        mlp_norm=get("post_attention_layernorm.weight"),
        gate_up=torch.cat((gate, up), dim=0).t(),
        mlp_down=get("mlp.down_proj.weight").t(),
    )


def dims_from_config(path):
    """``(Qwen3Dims, num_layers, vocab)`` from a checkpoint directory's
    Hugging Face ``config.json``."""
    with open(os.path.join(path, "config.json")) as f:
        config = json.load(f)
    heads = config["num_attention_heads"]
    dims = Qwen3Dims(hidden=config["hidden_size"], ffn=config["intermediate_size"], heads=heads,
                     kv_heads=config.get("num_key_value_heads", heads),
                     head_dim=config.get("head_dim", config["hidden_size"] // heads),
                     eps=config.get("rms_norm_eps", 1e-6), theta=config.get("rope_theta", 1e6))
    return dims, config["num_hidden_layers"], config["vocab_size"]
