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
