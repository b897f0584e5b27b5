"""Local safetensors loader: a toy sharded Qwen3-style checkpoint written
here is read back tensor by tensor and assembled into block weights with
the reference's naming and transposes (benchmark_qwen3_32b_layer.py:401-431)."""

import json

import pytest
import torch
from safetensors.torch import save_file

from strassen_tpu_amd.checkpoint import LocalSafetensors, dims_from_config, load_block_weights

H, F, HEADS, KV, HD = 64, 96, 4, 2, 16


def layer_tensors(layer, g):
    def w(out, inp):
        return torch.randn(out, inp, generator=g).to(torch.bfloat16)

    def v(n):
        return torch.randn(n, generator=g).to(torch.bfloat16)

    p = f"model.layers.{layer}."
    return {
        p + "input_layernorm.weight": v(H), p + "post_attention_layernorm.weight": v(H),
        p + "self_attn.q_proj.weight": w(HEADS * HD, H), p + "self_attn.k_proj.weight": w(KV * HD, H),
        p + "self_attn.v_proj.weight": w(KV * HD, H), p + "self_attn.o_proj.weight": w(H, HEADS * HD),
        p + "self_attn.q_norm.weight": v(HD), p + "self_attn.k_norm.weight": v(HD),
        p + "mlp.gate_proj.weight": w(F, H), p + "mlp.up_proj.weight": w(F, H), p + "mlp.down_proj.weight": w(H, F),
    }


@pytest.fixture
def checkpoint(tmp_path):
    g = torch.Generator().manual_seed(0)
    shards = [layer_tensors(0, g), layer_tensors(1, g)]
    shards[1]["model.norm.weight"] = torch.ones(H, dtype=torch.bfloat16)
    shards[1]["model.embed_tokens.weight"] = torch.randn(32, H, generator=g).to(torch.bfloat16)
    weight_map = {}
    for i, tensors in enumerate(shards):
        name = f"model-{i + 1:05d}-of-00002.safetensors"
        save_file(tensors, str(tmp_path / name))
        weight_map.update({key: name for key in tensors})
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    (tmp_path / "config.json").write_text(json.dumps({
        "hidden_size": H, "intermediate_size": F, "num_attention_heads": HEADS, "num_key_value_heads": KV,
        "head_dim": HD, "rms_norm_eps": 1e-6, "rope_theta": 1e6, "num_hidden_layers": 2, "vocab_size": 32}))
    return tmp_path, {k: v for s in shards for k, v in s.items()}


def test_sharded_checkpoint_round_trip(checkpoint):
    path, tensors = checkpoint
    ckpt = LocalSafetensors(str(path))
    assert ckpt.names() == sorted(tensors)
    for name, value in tensors.items():
        assert torch.equal(ckpt.tensor(name), value)
    with pytest.raises(KeyError):
        ckpt.tensor("model.layers.9.mlp.up_proj.weight")


def test_block_weights_layout(checkpoint):
    path, tensors = checkpoint
    digest = {}
    w = load_block_weights(str(path), 1, device="cpu", digest=digest)
    p = "model.layers.1."
    assert torch.equal(w.query, tensors[p + "self_attn.q_proj.weight"].t())
    assert torch.equal(w.mlp_down, tensors[p + "mlp.down_proj.weight"].t())
    assert w.gate_up.shape == (H, 2 * F) and w.gate_up.stride(0) == 1  # K-contiguous
    assert torch.equal(w.gate_up[:, :F], tensors[p + "mlp.gate_proj.weight"].t())
    assert torch.equal(w.gate_up[:, F:], tensors[p + "mlp.up_proj.weight"].t())
    assert torch.equal(w.key_norm, tensors[p + "self_attn.k_norm.weight"])
    assert len(digest) == 11 and all(len(h) == 64 for h in digest.values())


def test_config_and_dtype_checks(checkpoint, tmp_path):
    path, _ = checkpoint
    dims, layers, vocab = dims_from_config(str(path))
    assert (dims.hidden, dims.ffn, dims.heads, dims.kv_heads, dims.head_dim, layers, vocab) == (H, F, HEADS, KV, HD,
                                                                                                 2, 32)
    single = tmp_path / "single"
    single.mkdir()
    save_file({"x": torch.zeros(4, dtype=torch.float32)}, str(single / "model.safetensors"))
    with pytest.raises(ValueError, match="dtype"):
        LocalSafetensors(str(single)).tensor("x")
    empty = tmp_path / "empty"
    empty.mkdir()
    with pytest.raises(FileNotFoundError):
        LocalSafetensors(str(empty))
