"""The packed-weight cache on the GPU: a plain weight passed to
strassen_matmul / cubic_matmul is packed once and reused while unchanged,
with results bit-identical to packing it for every call, and an in-place
update of the weight is seen on the next call."""

import warnings

import numpy as np
import pytest
import torch

import oracle as o
import strassen_tpu_amd as smx
from strassen_tpu_amd import strassen as surface
from test_gpu_parity import DEV, assert_ulp_close, dev, dev_weight, host, say

pytestmark = pytest.mark.gpu


@pytest.fixture
def weight_cache():
    previous = smx.cache_packed_weights(256 << 20)
    yield
    smx.cache_packed_weights(0)
    smx.cache_packed_weights(previous)


def _problem(seed=31, m=512, k=1024, n=512):
    rng = np.random.default_rng(seed)
    a = o.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    b = o.bf16_round((rng.standard_normal((k, n)) * 0.05).astype(np.float32))
    return a, b


@pytest.mark.parametrize("arm", ["strassen", "cubic"])
def test_cached_weight_matches_per_call_packing(arm, weight_cache):
    a, b = _problem()
    x, w = dev(a), dev_weight(b)
    fn = smx.strassen_matmul if arm == "strassen" else smx.cubic_matmul
    kw = dict(bm=256, bn=256, bk=512)
    smx.cache_packed_weights(0)
    uncached = host(fn(x, w, **kw))
    smx.cache_packed_weights(256 << 20)
    before = smx.packed_weight_cache_info()
    first, second = host(fn(x, w, **kw)), host(fn(x, w, **kw))
    after = smx.packed_weight_cache_info()
    say(f"  {arm} cache {after}")
    assert after["misses"] == before["misses"] + 1 and after["hits"] == before["hits"] + 1
    assert np.array_equal(first, uncached) and np.array_equal(second, uncached)
    # An in-place update through the [K, N] view: the next call packs again.
    # Doubling is exact in bf16, so the result doubles exactly.
    w.mul_(2)
    doubled = host(fn(x, w, **kw))
    assert smx.packed_weight_cache_info()["stale"] == after["stale"] + 1
    assert np.array_equal(doubled, 2 * uncached)


def test_cached_weight_with_exact_panels_and_epilogue(weight_cache):
    a, b = _problem(k=2048)
    x, w = dev(a), dev_weight(b)
    res = o.bf16_round(np.random.default_rng(4).standard_normal((512, 512)).astype(np.float32))
    kw = dict(bm=256, bn=256, bk=512, classical_panels=(1, 3), epilogue="residual_add", residual=dev(res))
    got = [host(smx.strassen_matmul(x, w, **kw)) for _ in range(2)]
    want = o.strassen_matmul(a, b, bm=256, bn=256, bk=512, classical_panels=(1, 3), epilogue="residual_add",
                             residual=res)
    assert np.array_equal(got[0], got[1])
    assert_ulp_close(got[0], want, k=2048)
    assert smx.packed_weight_cache_info()["hits"] >= 1


def test_per_call_packing_warns_once():
    a, b = _problem()
    previous = smx.cache_packed_weights(0)
    surface._PLAIN_PACK_WARNED = False
    try:
        with pytest.warns(smx.PlainWeightPackWarning, match="packed on every call"):
            smx.strassen_matmul(dev(a), dev_weight(b), bm=256, bn=256, bk=512)
        assert surface._PLAIN_PACK_WARNED
    finally:
        smx.cache_packed_weights(previous)
    torch.cuda.synchronize(DEV)


def test_expected_per_call_packing_keeps_the_warning():
    """A measurement that packs per call on purpose neither warns nor uses
    up the warning of a later per-call pack."""
    a, b = _problem()
    previous = smx.cache_packed_weights(0)
    surface._PLAIN_PACK_WARNED = False
    try:
        with warnings.catch_warnings():
            warnings.simplefilter("error", smx.PlainWeightPackWarning)
            with surface.per_call_packing_expected():
                smx.strassen_matmul(dev(a), dev_weight(b), bm=256, bn=256, bk=512)
        assert not surface._PLAIN_PACK_WARNED
        with pytest.warns(smx.PlainWeightPackWarning, match="packed on every call"):
            smx.strassen_matmul(dev(a), dev_weight(b), bm=256, bn=256, bk=512)
    finally:
        smx.cache_packed_weights(previous)
    torch.cuda.synchronize(DEV)
