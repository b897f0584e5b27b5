"""The streamed decoder on the GPU at reduced width: three layers through the
three arms, finite, each arm's drift against the native arm bounded, Strassen
drift comparable to the cubic arm's."""

import pytest

from strassen_tpu_amd import qwen3_block as qb
from strassen_tpu_amd import streamed_decoder as sd

pytestmark = pytest.mark.gpu


def test_streamed_decoder_small():
    records = []
    dims = qb.Qwen3Dims(hidden=1024, ffn=2048, heads=8, kv_heads=2)
    summary = sd.run(3, dims=dims, batch=2, seq=256, vocab=4096, warmups=1, runs=2, tile=(256, 256, 256),
                     emit=records.append)
    print(summary, flush=True)
    assert summary["all_finite"]
    layers = [r for r in records if r["kind"] == "layer"]
    assert len(layers) == 3
    for r in layers:
        for arm in ("cubic", "strassen"):
            assert r["errors_vs_hipblaslt"][arm]["l2_relative"] < 5e-2, (r["layer"], arm)
        assert all(v > 0 for v in r["mean_ms"].values())
    final = summary["final_errors_vs_hipblaslt"]
    assert final["strassen"]["l2_relative"] <= 2 * final["cubic"]["l2_relative"] + 1e-2
    logits = summary["logit_metrics"]
    assert logits["strassen"]["positions"] == 2 * 255
    assert logits["strassen"]["mean_kl_nats"] < 0.05


def test_streamed_decoder_from_local_checkpoint(tmp_path):
    """Two layers read from a toy safetensors checkpoint written here (the
    naming of a Hugging Face Qwen3 checkpoint) run through the same path."""
    import json

    import torch
    from safetensors.torch import save_file

    from strassen_tpu_amd.checkpoint import LocalSafetensors, dims_from_config

    hidden, ffn, heads, kv, hd, vocab = 1024, 2048, 8, 2, 128, 4096
    g = torch.Generator().manual_seed(3)

    def w(out, inp):
        return (torch.randn(out, inp, generator=g) * 0.02).to(torch.bfloat16)

    def scale(n):
        return (1 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)

    tensors = {"model.embed_tokens.weight": torch.randn(vocab, hidden, generator=g).to(torch.bfloat16),
               "model.norm.weight": scale(hidden)}
    for layer in range(2):
        p = f"model.layers.{layer}."
        tensors.update({
            p + "input_layernorm.weight": scale(hidden), p + "post_attention_layernorm.weight": scale(hidden),
            p + "self_attn.q_proj.weight": w(heads * hd, hidden), p + "self_attn.k_proj.weight": w(kv * hd, hidden),
            p + "self_attn.v_proj.weight": w(kv * hd, hidden), p + "self_attn.o_proj.weight": w(hidden, heads * hd),
            p + "self_attn.q_norm.weight": scale(hd), p + "self_attn.k_norm.weight": scale(hd),
            p + "mlp.gate_proj.weight": w(ffn, hidden), p + "mlp.up_proj.weight": w(ffn, hidden),
            p + "mlp.down_proj.weight": w(hidden, ffn)})
    save_file(tensors, str(tmp_path / "model.safetensors"))
    (tmp_path / "config.json").write_text(json.dumps({
        "hidden_size": hidden, "intermediate_size": ffn, "num_attention_heads": heads, "num_key_value_heads": kv,
        "head_dim": hd, "num_hidden_layers": 2, "vocab_size": vocab}))
    dims, layers, vocab = dims_from_config(str(tmp_path))
    records = []
    summary = sd.run(layers, dims=dims, batch=2, seq=256, vocab=vocab, warmups=1, runs=2, tile=(256, 256, 256),
                     emit=records.append, checkpoint=LocalSafetensors(str(tmp_path)))
    assert summary["all_finite"]
    assert records[0]["data"].startswith("local checkpoint")
    for r in (r for r in records if r["kind"] == "layer"):
        for arm in ("cubic", "strassen"):
            assert r["errors_vs_hipblaslt"][arm]["l2_relative"] < 5e-2, (r["layer"], arm)
