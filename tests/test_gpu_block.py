"""The Qwen3 decoder block on the GPU: the Strassen and cubic arms (fused
epilogues, packed weights) against an FP32 restatement of the reference layer
(``experiments/qwen3/benchmark_qwen3_32b_layer.py:344-398``) computed on the
CPU, and against each other.

Bar: the block's update ``out - x`` (attention + MLP contribution) within
relative Frobenius 2e-2 of the FP32 block for every arm, and the Strassen
arm no worse than 1.5x the cubic arm's error plus 2e-3.
"""

import numpy as np
import pytest
import torch

from fp32_reference import fp32_block
from strassen_tpu_amd import qwen3_block as qb

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def say(*args):
    print(*args, flush=True)


@pytest.mark.parametrize("dims,batch,seq,tile", [
    (qb.Qwen3Dims(hidden=1024, ffn=2048, heads=8, kv_heads=2), 2, 256, (256, 256, 256)),
    (qb.Qwen3Dims(hidden=2048, ffn=4096, heads=16, kv_heads=4), 1, 512, (512, 512, 512)),
])
def test_block_arms_match_fp32_layer(dims, batch, seq, tile):
    torch.manual_seed(0)
    w = qb.BlockWeights.random_init(dims, DEV, seed=11)
    x = torch.randn(batch * seq, dims.hidden, device=DEV).to(torch.bfloat16)
    ref = fp32_block(x, w, dims, batch, seq)
    delta_ref = ref - x.float().cpu()
    errs = {}
    for arm in qb.ARMS:
        say(f"  block arm={arm} dims={dims} batch={batch} seq={seq} tile={tile}")
        block = qb.PreparedBlock(w, dims, arm, batch=batch, seq=seq, tile=tile)
        out = qb.block_forward(x, block)
        torch.cuda.synchronize()
        assert out.shape == x.shape and out.dtype == torch.bfloat16
        got = out.float().cpu()
        assert torch.isfinite(got).all()
        delta = got - x.float().cpu()
        errs[arm] = float(torch.linalg.norm(delta - delta_ref) / torch.linalg.norm(delta_ref))
    say(f"  block update rel err vs FP32: {errs}")
    for arm, e in errs.items():
        assert e <= 2e-2, arm
    assert errs["strassen"] <= 1.5 * errs["cubic"] + 2e-3


def test_block_is_deterministic_across_calls():
    dims = qb.Qwen3Dims(hidden=1024, ffn=2048, heads=8, kv_heads=2)
    w = qb.BlockWeights.random_init(dims, DEV, seed=5)
    x = torch.randn(512, 1024, device=DEV).to(torch.bfloat16)
    block = qb.PreparedBlock(w, dims, "strassen", batch=2, seq=256, tile=(256, 256, 256))
    first = qb.block_forward(x, block)
    second = qb.block_forward(x, block)
    torch.cuda.synchronize()
    assert torch.equal(first, second)
