"""Host logic of the Qwen3 block (CPU): the torch norm / RoPE helpers against
the oracle's restatement of ``benchmark_qwen3_32b_layer.py:258-284``."""

import numpy as np
import pytest
import torch

import oracle as o
from strassen_tpu_amd import qwen3_block as qb


def bf16(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)


def test_rope_values_match_oracle():
    cos, sin = qb.rope_values(64, 128, 1e6, "cpu")
    want_cos, want_sin = o.rope_values(64, 128, 1e6)
    assert np.array_equal(cos.float().numpy(), want_cos)
    assert np.array_equal(sin.float().numpy(), want_sin)


def test_rms_norm_matches_oracle():
    rng = np.random.default_rng(3)
    x = o.bf16_round(rng.standard_normal((32, 256)).astype(np.float32))
    g = o.bf16_round((1 + 0.1 * rng.standard_normal(256)).astype(np.float32))
    got = qb.rms_norm(bf16(x), bf16(g), 1e-6).float().numpy()
    want = o.rms_norm(x, g, 1e-6)
    # rsqrt vs 1/sqrt may differ by an FP32 ulp before the bf16 rounding
    assert np.mean(got != want) < 0.01
    assert np.max(np.abs(got - want)) <= np.max(np.abs(want)) * 2 ** -7


def test_apply_rope_matches_oracle():
    rng = np.random.default_rng(4)
    x = o.bf16_round(rng.standard_normal((2, 16, 4, 128)).astype(np.float32))
    cos, sin = o.rope_values(16, 128, 1e6)
    got = qb.apply_rope(bf16(x), bf16(cos), bf16(sin)).float().numpy()
    assert np.array_equal(got, o.apply_rope(x, cos, sin))


def test_block_surface_checks():
    dims = qb.Qwen3Dims(hidden=256, ffn=512, heads=2, kv_heads=1)
    w = qb.BlockWeights.random_init(dims, "cpu")
    assert tuple(w.query.shape) == (256, 256) and tuple(w.gate_up.shape) == (256, 1024)
    assert w.query.stride(0) == 1  # [in, out] view of [out, in] storage
    with pytest.raises(ValueError, match="unknown arm"):
        qb.PreparedBlock(w, dims, "xla", batch=1, seq=256)
    # the native arm needs no relayout and builds on any device
    block = qb.PreparedBlock(w, dims, "hipblaslt", batch=1, seq=256)
    assert tuple(block.cos.shape) == (256, 128)


def test_decoder_metrics_on_cpu_tensors():
    """The streamed decoder's metrics (device-agnostic torch) against numpy."""
    from strassen_tpu_amd import streamed_decoder as sd

    rng = np.random.default_rng(6)
    ref = rng.standard_normal((64, 32)).astype(np.float32)
    got = ref + 1e-3 * rng.standard_normal((64, 32)).astype(np.float32)
    e = sd.device_error(torch.from_numpy(got), torch.from_numpy(ref))
    want = o.device_error(got, ref)
    for key in ("max_abs", "rmse", "maxnorm_relative", "l2_relative"):
        assert e[key] == pytest.approx(want[key], rel=1e-5), key
    # logit metrics: identical candidates have zero KL, full agreement, zero delta
    h = torch.randn(8, 16).to(torch.bfloat16)
    head = torch.randn(16, 40).to(torch.bfloat16)
    targets = torch.randint(0, 40, (8,))
    nl, nsq, nmax, cub, stra, count = sd.logit_chunk_metrics(h, h, h, head, targets, torch.ones(8))
    assert count == 8 and cub[0] == pytest.approx(nl) and cub[1] == pytest.approx(0, abs=1e-6)
    assert cub[2] == 8 and cub[3] == 0 and cub[4] == 0
    # the native loss is the summed negative log-likelihood of the targets
    logp = torch.log_softmax(torch.matmul(h, head).float(), -1)
    assert nl == pytest.approx(float(-logp[torch.arange(8), targets].sum()), rel=1e-5)
    interval = sd.bootstrap_sum_interval([1.0, 2.0, 3.0], seed=0)
    assert interval["sum_ms"] == 6.0 and interval["ci95_ms"][0] <= 6.0 <= interval["ci95_ms"][1]
