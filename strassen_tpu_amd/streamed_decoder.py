"""Streamed Qwen3-32B decoder: every layer on the three arms, one layer resident.

Restates the scope of the reference's streamed harness
(``experiments/qwen3/benchmark_qwen3_32b_streamed_inference.py:452-560``).
There is no network to stream a checkpoint: each layer's weights are either
generated on the device (random init) or read from a local safetensors
checkpoint (``--checkpoint DIR``, ``checkpoint.LocalSafetensors``). Timing
is "summed resident layer compute", not end-to-end latency; layer
generation, relayout / packing, embeddings and the final logits are excluded
(``docs/COLAB_RUNBOOK.md:121-127``).

For every layer, in order:
1. Build the layer's weights, then the arms' relayouts: packed Strassen and
   packed cubic weights, or plain weights for hipBLASLt.
2. Run ``warmups`` + ``runs`` forwards per arm, rotating the arm order per run
   as the reference does (``:505-516``), each timed with HIP events.
3. Carry each arm's own hidden state to the next layer.
4. Check finiteness and record each arm's drift against the native arm
   (``device_error``, ``benchmark_common.py:36-60``), plus Strassen against
   the cubic arm.

After the last layer the final RMSNorm and LM head produce logits per arm.
The next-token loss, KL to the native arm, top-1 agreement and logit error
are accumulated over chunks of 256 positions (``:343-378``), and each
candidate arm gets the reference's task gate (``:444-448``): |loss delta|
<= 0.01, top-1 agreement >= 0.99, KL <= 0.005 nats. ``main`` exits with 2
when an arm fails it. With random weights and random tokens these are drift
measures, not model quality.

``python -m strassen_tpu_amd.streamed_decoder --layers 64`` prints one JSON
record per layer and a summary record.
"""

from __future__ import annotations

import argparse
import dataclasses
import gc
import json
import math
import statistics
import sys
import time

import numpy as np
import torch

from . import qwen3_block as qb
from .checkpoint import TENSOR_PREFIX, LocalSafetensors, dims_from_config, load_block_weights

__all__ = ["ARMS", "device_error", "logit_chunk_metrics", "passes_task_gate", "run"]

# The reference's arms: regular_xla -> hipBLASLt, gated_cubic, gated_strassen.
ARMS = ("hipblaslt", "cubic", "strassen")
LOGIT_CHUNK = 256


def device_error(got, reference):
    """max_abs, rmse, maxnorm_relative and l2_relative of ``got`` against
    ``reference`` (``benchmark_common.py:36-60``), computed on the device."""
    got, reference = got.float(), reference.float()
    delta = got - reference
    tiny = torch.finfo(torch.float32).tiny
    max_abs = delta.abs().max()
    values = torch.stack([
        max_abs, delta.square().mean().sqrt(),
        max_abs / reference.abs().max().clamp_min(tiny),
        torch.linalg.vector_norm(delta) / torch.linalg.vector_norm(reference).clamp_min(tiny),
    ]).tolist()
    return dict(zip(("max_abs", "rmse", "maxnorm_relative", "l2_relative"), values))


def logit_chunk_metrics(native_h, cubic_h, strassen_h, lm_head, targets, mask):
    """Per-chunk sums of ``:343-378``: native loss, native logit square sum and
    max; for cubic and Strassen (loss, KL to native, top-1 agreement, logit
    delta square sum, max |delta|); the position count."""
    logits = [torch.matmul(h, lm_head).float() for h in (native_h, cubic_h, strassen_h)]
    log_probs = [torch.log_softmax(v, dim=-1) for v in logits]
    selected = [lp.gather(1, targets[:, None])[:, 0] for lp in log_probs]
    m32 = mask.float()
    native_probs = log_probs[0].exp()

    def candidate(i):
        delta = logits[i] - logits[0]
        return (float(-(selected[i] * m32).sum()),
                float(((native_probs * (log_probs[0] - log_probs[i])).sum(1) * m32).sum()),
                float(((logits[i].argmax(1) == logits[0].argmax(1)).float() * m32).sum()),
                float((delta.square() * m32[:, None]).sum()),
                float((delta.abs() * m32[:, None]).max()))

    return (float(-(selected[0] * m32).sum()), float((logits[0].square() * m32[:, None]).sum()),
            float((logits[0].abs() * m32[:, None]).max()), candidate(1), candidate(2), float(m32.sum()))


def bootstrap_sum_interval(deltas, seed):
    """95% bootstrap interval of a sum of per-layer deltas (``:334-340``)."""
    values = np.asarray(deltas, np.float64)
    rng = np.random.default_rng(seed)
    sums = rng.choice(values, size=(20000, len(values)), replace=True).sum(axis=1)
    low, high = np.quantile(sums, [0.025, 0.975])
    return {"sum_ms": float(values.sum()), "ci95_ms": [float(low), float(high)]}


def _time_forward(x, block):
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    out = qb.block_forward(x, block)
    stop.record()
    return out, (start, stop)


# The reference's task gate (benchmark_qwen3_32b_streamed_inference.py:444-448).
GATE_LOSS_DELTA = 0.01
GATE_TOP1 = 0.99
GATE_KL_NATS = 0.005


def passes_task_gate(record):
    """|loss delta| <= 0.01, top-1 agreement >= 0.99 and mean KL <= 0.005
    nats against the native arm (``:444-448``)."""
    return bool(record["absolute_loss_delta"] <= GATE_LOSS_DELTA and record["top1_agreement"] >= GATE_TOP1
                and record["mean_kl_nats"] <= GATE_KL_NATS)


def run(num_layers, *, dims=qb.QWEN3_32B, batch=8, seq=1024, vocab=151936, warmups=1, runs=3, seed=0,
        tile=(1024, 1024, 512), device="cuda:0", emit=None, checkpoint=None, capture=None):
    """Stream ``num_layers`` layers through the three arms; returns the
    summary record (and passes every record to ``emit``). Weights are
    random-init, or read layer by layer from ``checkpoint`` (a
    ``LocalSafetensors`` whose layers match ``dims``); token ids are random
    either way. A ``capture`` dict receives the token ids, the initial
    hidden state, each arm's final hidden state, the final norm scale and
    the LM head, for a caller that recomputes the forward another way."""
    emit = emit or (lambda record: None)
    dev = torch.device(device)
    gen = torch.Generator(device=dev).manual_seed(seed)
    token_ids = torch.randint(0, vocab, (batch, seq), device=dev, generator=gen)
    if checkpoint is not None:
        embeddings = checkpoint.tensor(f"{TENSOR_PREFIX}.embed_tokens.weight", device=dev)
    else:
        embeddings = (torch.randn(vocab, dims.hidden, device=dev, generator=gen)).to(torch.bfloat16)
    initial = embeddings[token_ids.reshape(-1)]
    del embeddings
    if capture is not None:
        capture["token_ids"], capture["initial"] = token_ids, initial.clone()
    hidden = {arm: initial.clone() for arm in ARMS}
    del initial
    emit({"kind": "metadata", "layers": num_layers, "dims": dataclasses.asdict(dims), "batch": batch, "seq": seq,
          "vocab": vocab, "tile": list(tile), "arms": list(ARMS), "warmups_per_layer": warmups, "runs_per_layer": runs,
          "performance_scope": "aggregate resident layer compute; layer generation and relayout excluded",
          "data": ("local checkpoint bf16 weights" if checkpoint is not None else "random-init bf16 weights")
          + ", random token ids"})

    per_layer = {arm: [] for arm in ARMS}
    all_finite = True
    for index in range(num_layers):
        started = time.perf_counter()
        if checkpoint is not None:
            weights = load_block_weights(checkpoint, index, device=dev)
        else:
            weights = qb.BlockWeights.random_init(dims, dev, seed=seed * 1000 + index + 1)
        blocks = {arm: qb.PreparedBlock(weights, dims, arm, batch=batch, seq=seq, tile=tile) for arm in ARMS}
        torch.cuda.synchronize()
        prepare_s = time.perf_counter() - started
        for warmup in range(warmups):
            order = ARMS[(index + warmup) % 3:] + ARMS[:(index + warmup) % 3]
            for arm in order:
                qb.block_forward(hidden[arm], blocks[arm])
        torch.cuda.synchronize()
        events = {arm: [] for arm in ARMS}
        next_hidden = {}
        for r in range(runs):
            order = ARMS[(index + r) % 3:] + ARMS[:(index + r) % 3]
            if r % 2:
                order = tuple(reversed(order))
            for arm in order:
                next_hidden[arm], ev = _time_forward(hidden[arm], blocks[arm])
                events[arm].append(ev)
        torch.cuda.synchronize()
        samples = {arm: [a.elapsed_time(b) for a, b in events[arm]] for arm in ARMS}
        hidden = next_hidden
        finite = all(bool(torch.isfinite(v).all()) for v in hidden.values())
        all_finite = all_finite and finite
        errors = {arm: device_error(hidden[arm], hidden["hipblaslt"]) for arm in ("cubic", "strassen")}
        strassen_vs_cubic = device_error(hidden["strassen"], hidden["cubic"])
        means = {arm: statistics.fmean(v) for arm, v in samples.items()}
        for arm in ARMS:
            per_layer[arm].append(means[arm])
        emit({"kind": "layer", "layer": index, "prepare_s": prepare_s, "mean_ms": means, "samples_ms": samples,
              "errors_vs_hipblaslt": errors, "strassen_vs_cubic": strassen_vs_cubic, "finite": finite})
        del blocks, weights
        gc.collect()

    aggregate = {arm: float(sum(v)) for arm, v in per_layer.items()}
    performance = {
        "aggregate_ms": aggregate,
        "speedup_strassen_vs_hipblaslt": aggregate["hipblaslt"] / aggregate["strassen"],
        "speedup_strassen_vs_cubic": aggregate["cubic"] / aggregate["strassen"],
        "strassen_minus_hipblaslt": bootstrap_sum_interval(
            [s - x for x, s in zip(per_layer["hipblaslt"], per_layer["strassen"])], seed=1),
        "strassen_minus_cubic": bootstrap_sum_interval(
            [s - c for c, s in zip(per_layer["cubic"], per_layer["strassen"])], seed=2),
    }

    # Final norm and LM head (excluded from timing), chunked like the reference.
    if checkpoint is not None:
        final_norm = checkpoint.tensor(f"{TENSOR_PREFIX}.norm.weight", device=dev)
        head_name = "lm_head.weight" if "lm_head.weight" in checkpoint.shard_of else \
            f"{TENSOR_PREFIX}.embed_tokens.weight"  # tied embeddings
        lm_head = checkpoint.tensor(head_name, device=dev).t()
    else:
        final_norm = (1.0 + 0.1 * torch.randn(dims.hidden, device=dev, generator=gen)).to(torch.bfloat16)
        lm_head = (torch.randn(vocab, dims.hidden, device=dev, generator=gen) * 0.02).to(torch.bfloat16).t()
    rows = {arm: qb.rms_norm(h, final_norm, dims.eps).view(batch, seq, dims.hidden)[:, :-1]
            .reshape(-1, dims.hidden) for arm, h in hidden.items()}
    targets = token_ids[:, 1:].reshape(-1)
    totals = {"native_loss": 0.0, "native_sq": 0.0, "native_max": 0.0, "count": 0.0,
              "cubic": [0.0] * 5, "strassen": [0.0] * 5}
    for start in range(0, targets.numel(), LOGIT_CHUNK):
        stop = min(start + LOGIT_CHUNK, targets.numel())
        mask = torch.ones(stop - start, device=dev)
        nl, nsq, nmax, cub, stra, count = logit_chunk_metrics(
            rows["hipblaslt"][start:stop], rows["cubic"][start:stop], rows["strassen"][start:stop], lm_head,
            targets[start:stop], mask)
        totals["native_loss"] += nl
        totals["native_sq"] += nsq
        totals["native_max"] = max(totals["native_max"], nmax)
        totals["count"] += count
        for name, values in (("cubic", cub), ("strassen", stra)):
            for i, v in enumerate(values):
                totals[name][i] = max(totals[name][i], v) if i == 4 else totals[name][i] + v
    count = totals["count"]
    task = {}
    for name in ("cubic", "strassen"):
        loss, kl, top1, delta_sq, max_delta = totals[name]
        task[name] = {
            "native_loss": totals["native_loss"] / count, "candidate_loss": loss / count,
            "absolute_loss_delta": abs(loss - totals["native_loss"]) / count, "mean_kl_nats": kl / count,
            "top1_agreement": top1 / count,
            "logit_l2_relative": math.sqrt(delta_sq / max(totals["native_sq"], 1e-30)),
            "logit_maxnorm_relative": max_delta / max(totals["native_max"], 1e-30), "positions": int(count),
        }
        task[name]["passes_task_gate"] = passes_task_gate(task[name])
    if capture is not None:
        capture.update(hidden=hidden, final_norm=final_norm, lm_head=lm_head)
    summary = {"kind": "summary", "layers": num_layers, "all_finite": all_finite, "performance": performance,
               "final_errors_vs_hipblaslt": {arm: device_error(hidden[arm], hidden["hipblaslt"])
                                             for arm in ("cubic", "strassen")},
               "logit_metrics": task}
    emit(summary)
    return summary


def main(argv=None):
    ap = argparse.ArgumentParser(description="Streamed Qwen3-32B decoder, random-init weights, three arms")
    ap.add_argument("--layers", type=int, default=64)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--seq", type=int, default=1024)
    ap.add_argument("--warmups", type=int, default=1)
    ap.add_argument("--runs", type=int, default=3)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--out", default=None, help="also write the records to this JSONL file")
    ap.add_argument("--checkpoint", default=None,
                    help="local Hugging Face checkpoint directory (config.json + safetensors) instead of random init")
    args = ap.parse_args(argv)
    sink = open(args.out, "w") if args.out else None

    def emit(record):
        line = json.dumps(record)
        print(line, flush=True)
        if sink:
            sink.write(line + "\n")
            sink.flush()

    extra = {}
    if args.checkpoint:
        dims, layers, vocab = dims_from_config(args.checkpoint)
        extra = dict(dims=dims, vocab=vocab, checkpoint=LocalSafetensors(args.checkpoint))
        args.layers = min(args.layers, layers)
    summary = run(args.layers, batch=args.batch, seq=args.seq, warmups=args.warmups, runs=args.runs,
                  seed=args.seed, emit=emit, **extra)
    if not summary["all_finite"]:
        return 1
    failed = [arm for arm, record in summary["logit_metrics"].items() if not record["passes_task_gate"]]
    if failed:
        print(f"task gate failed for {failed} (|loss delta| <= {GATE_LOSS_DELTA}, top-1 >= {GATE_TOP1}, "
              f"KL <= {GATE_KL_NATS} nats against the hipBLASLt arm)", file=sys.stderr)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main())
