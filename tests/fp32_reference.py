"""FP32 restatements used by the GPU tests as references (not collected).

``fp32_block`` restates one Qwen3 decoder layer of the reference
(``experiments/qwen3/benchmark_qwen3_32b_layer.py:344-398``) in float32 (on
the CPU, or on the GPU for full-size layers): the same sites and epilogue
semantics, no bf16 rounding after the inputs. ``fp32_decoder`` composes it over layers, and ``logit_metrics``
computes the reference's task metrics
(``benchmark_qwen3_32b_streamed_inference.py:343-378``) of a candidate's
logits against reference logits.
"""

import torch

from strassen_tpu_amd import qwen3_block as qb


def fp32_block(x, w, dims, batch, seq, device="cpu"):
    f = lambda t: t.detach().float().to(device)
    x, eps = f(x), dims.eps

    def norm(v, g):
        return v * torch.rsqrt(v.square().mean(-1, keepdim=True) + eps) * f(g)

    cos, sin = (t.float().to(device) for t in qb.rope_values(seq, dims.head_dim, dims.theta, "cpu"))

    def rope(v):
        a, b = v.chunk(2, dim=-1)
        return v * cos[None, :, None, :] + torch.cat((-b, a), -1) * sin[None, :, None, :]

    h = norm(x, w.attention_norm)
    q = rope(norm((h @ f(w.query)).view(batch, seq, dims.heads, dims.head_dim), w.query_norm))
    k = rope(norm((h @ f(w.key)).view(batch, seq, dims.kv_heads, dims.head_dim), w.key_norm))
    v = (h @ f(w.value)).view(batch, seq, dims.kv_heads, dims.head_dim)
    groups = dims.heads // dims.kv_heads
    att = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(1, 2), k.repeat_interleave(groups, 2).transpose(1, 2),
        v.repeat_interleave(groups, 2).transpose(1, 2), is_causal=True).transpose(1, 2)
    r = x + att.reshape(batch * seq, -1) @ f(w.attention_output)
    h2 = norm(r, w.mlp_norm)
    gate, up = (h2 @ f(w.gate_up)).chunk(2, dim=-1)
    return r + (torch.nn.functional.silu(gate) * up) @ f(w.mlp_down)


def fp32_decoder(initial, layer_weights, dims, batch, seq):
    """The FP32 layers applied in turn to the bf16 initial hidden state;
    ``layer_weights`` yields each layer's BlockWeights."""
    x = initial.detach().float().cpu()
    for w in layer_weights:
        x = fp32_block(x, w, dims, batch, seq)
    return x


def fp32_logits(hidden, final_norm, lm_head, eps, batch, seq):
    """Final RMSNorm and LM head in float32 over every position but each
    sequence's last (the rows the next-token metrics use)."""
    h = hidden.detach().float().cpu()
    h = h * torch.rsqrt(h.square().mean(-1, keepdim=True) + eps) * final_norm.detach().float().cpu()
    h = h.view(batch, seq, -1)[:, :-1].reshape(-1, h.shape[-1])
    return h @ lm_head.detach().float().cpu()


def logit_metrics(candidate, reference, targets):
    """Next-token loss delta, mean KL(reference || candidate) in nats and
    top-1 agreement of float32 logits [positions, vocab]."""
    lp_c = torch.log_softmax(candidate.double(), -1)
    lp_r = torch.log_softmax(reference.double(), -1)
    t = targets.detach().cpu().long()[:, None]
    loss_c = float(-lp_c.gather(1, t).mean())
    loss_r = float(-lp_r.gather(1, t).mean())
    kl = float((lp_r.exp() * (lp_r - lp_c)).sum(-1).mean())
    top1 = float((candidate.argmax(-1) == reference.argmax(-1)).double().mean())
    return {"absolute_loss_delta": abs(loss_c - loss_r), "mean_kl_nats": kl, "top1_agreement": top1}
