"""GPU parity of SMX_FLAG_PRODUCT_MAJOR_ROUNDS: the product-major kernel on
the leading tile columns whose 128 x 256 product tiles fill whole rounds of
the CUs, the default (split) kernel on the columns after them.

The two parts are column ranges of one call: the head's tiles are the ones
the product-major kernel computes on its own (bit-identical), the rest's
are the default kernel's on a call of those columns (its K split included),
so every output matches the oracle within one bf16 ulp and integer operands
are bit-exact. Checked through the surface (strassen_kernel(
"product_major_rounds")) on shapes whose head fills exactly one round of the
device's CUs and leaves a rest: every epilogue the product-major kernel
fuses, FP32 output and auxiliaries, a block permutation, the workspace the
call asks for (the larger of the head's parked sets and the rest's K
shares), and the calls with no whole round, nothing left over, or K below
4096 (the split kernel alone).
"""

import ctypes
import math

import numpy as np
import pytest
import torch

import oracle as o
import strassen_tpu_amd as smx
from strassen_tpu_amd import _lib
from test_gpu_parity import DEV, _gaussian, assert_ulp_close, dev, dev_weight, fp32_floor, host, say

pytestmark = pytest.mark.gpu

PARK_PER_TILE = 256 * 1024  # two parked FP32 sets of a 128 x 256 product tile
TILE = dict(bm=1024, bn=1024, bk=512)


@pytest.fixture(autouse=True)
def _announce(request):
    say(f"\n[gpu] {request.node.nodeid}")
    yield
    torch.cuda.synchronize()


def _cus():
    return torch.cuda.get_device_properties(DEV).multi_processor_count


def head_columns(m, k, n, bn=1024):
    """Output columns of the product-major head (the C library's
    pm_round_columns, restated): the most 256-column product tiles per row
    whose tiles fill whole rounds and end on a bn tile boundary; none below
    K = 4096."""
    if k < 4096:
        return 0
    tiles_m, tiles_n = (m // 2) // 128, (n // 2) // 256
    per_round = _cus() // math.gcd(tiles_m, _cus())
    step = math.lcm(per_round, (bn // 2) // 256)
    return 2 * 256 * (tiles_n // step * step)


def hybrid_shape(k):
    """M = 1024 (4 product-major tile rows): the head fills one round of the
    CUs with cus / 4 tile columns; two more bn tiles form the rest."""
    m = 1024
    n = 2 * 256 * (_cus() // 4) + 2 * 1024
    return m, k, n


def _workspace_bytes(m, n, k, flags, epilogue=None, tile=(1024, 1024, 512)):
    d = _lib.SmxGemmDesc()
    d.m, d.n, d.k = m, n, k
    d.lda, d.ldb = k, k
    d.ldc = n // 2 if epilogue in ("swiglu", "geglu") else n
    d.bm, d.bn, d.bk = tile
    d.algo, d.epilogue = 7, _lib.SMX_EPI[epilogue]
    d.a_layout, d.b_layout = _lib.SMX_A_PACKED, _lib.SMX_B_PACKED
    d.flags = flags
    d.rope_head_dim, d.rope_eps = 128, 1e-6
    need = ctypes.c_int64()
    _lib.check(_lib.load().smx_gemm_workspace_bytes(d, ctypes.byref(need)))
    return need.value


def rounds_matmul(a, b, **kw):
    with smx.strassen_kernel("product_major_rounds"):
        return smx.strassen_matmul(a, b, **kw)


def pm_matmul(a, b, **kw):
    with smx.strassen_kernel("product_major"):
        return smx.strassen_matmul(a, b, **kw)


def test_workspace_covers_both_parts():
    rounds = _lib.SMX_FLAG_PRODUCT_MAJOR_ROUNDS
    m, k, n = hybrid_shape(4096)
    head = head_columns(m, k, n)
    assert 0 < head < n
    head_tiles = (m // 256) * (head // 512)
    assert head_tiles == _cus()
    rest = _workspace_bytes(m, n - head, k, 0)  # the rest as a call of its own
    assert rest > 0  # its 32 split-kernel tiles split over K
    assert _workspace_bytes(m, n, k, rounds) == max(head_tiles * PARK_PER_TILE, rest)
    # Every column in whole rounds: the product-major kernel alone.
    assert _workspace_bytes(m, head, k, rounds) == head_tiles * PARK_PER_TILE
    # No whole round: the default kernel alone.
    for shape in ((1024, 2048, 2048), (2048, 4096, 4096)):
        assert _workspace_bytes(*shape, rounds) == _workspace_bytes(*shape, 0)
    # A q/k epilogue is never the product-major kernel's.
    assert _workspace_bytes(m, n, k, rounds, epilogue="qk_norm_rope") == _workspace_bytes(
        m, n, k, 0, epilogue="qk_norm_rope")
    # Below K = 4096 the split kernel runs alone.
    assert head_columns(m, 2048, n) == 0
    assert _workspace_bytes(m, n, 2048, rounds) == _workspace_bytes(m, n, 2048, 0)


@pytest.mark.parametrize("k", [4096, 6144])
def test_integer_kat_bit_exact(k):
    """The rest's tiles split over K as well."""
    m, k, n = hybrid_shape(k)
    rng = np.random.default_rng(960 + k // 1024)
    a = rng.integers(-2, 3, (m, k)).astype(np.float32)
    b = rng.integers(-2, 3, (k, n)).astype(np.float32)
    w = smx.strassen_weight_layout(dev_weight(b), 1024, 512)
    exact = a @ b
    got32 = host(rounds_matmul(dev(a), w, output_dtype=torch.float32, **TILE))
    assert np.array_equal(got32, exact)
    got = host(rounds_matmul(dev(a), w, **TILE))
    assert np.array_equal(got, o.bf16_round(exact))


@pytest.mark.parametrize("bn", [512, 2048])
def test_other_bn_tiles_bit_exact(bn):
    """bn = 512 (one product-major tile column per bn tile) and bn = 2048
    (four): the head ends on a bn tile boundary and the rest starts on one,
    with integer operands and an integer residual bit-exact."""
    m, k = 1024, 4096
    n = 2 * 256 * (_cus() // 4) + bn
    head = head_columns(m, k, n, bn=bn)
    assert head == 2 * 256 * (_cus() // 4)
    rng = np.random.default_rng(990 + bn)
    a = rng.integers(-2, 3, (m, k)).astype(np.float32)
    b = rng.integers(-2, 3, (k, n)).astype(np.float32)
    r = rng.integers(-8, 9, (m, n)).astype(np.float32)
    w = smx.strassen_weight_layout(dev_weight(b), bn, 512)
    tile = dict(bm=1024, bn=bn, bk=512)
    exact = a @ b
    assert np.array_equal(host(rounds_matmul(dev(a), w, output_dtype=torch.float32, **tile)), exact)
    got = host(rounds_matmul(dev(a), w, epilogue="residual_add", residual=dev(r), **tile))
    assert np.array_equal(got, o.bf16_round(exact + r))


def test_exact_panels_transposed_lhs_and_fp32_inputs_take_the_head():
    """The paths built on the packed Strassen call keep their results when
    it splits into a product-major head and a split rest, with integer
    operands bit-exact: exact panels (the Strassen part over 14 of 16 bk
    panels, FP32, then the cubic over the other two), a transposed A, and
    FP32 inputs at HIGHEST precision (six bf16 passes, packed K = 6 K)."""
    m, n = 1024, 2 * 256 * (_cus() // 4) + 1024
    rng = np.random.default_rng(995)
    a = rng.integers(-2, 3, (m, 8192)).astype(np.float32)
    b = rng.integers(-2, 3, (8192, n)).astype(np.float32)
    got = smx.strassen_matmul(dev(a), dev_weight(b), classical_panels=(1, 3), **TILE)
    assert np.array_equal(host(got), o.bf16_round(a @ b))
    a4, b4 = a[:, :4096], b[:4096]
    got = smx.strassen_matmul_lhs_transposed(dev(np.ascontiguousarray(a4.T)), dev(b4), **TILE)
    assert np.array_equal(host(got), o.bf16_round(a4 @ b4))
    a1, b1 = a[:, :1024], b[:1024]
    got = smx.strassen_matmul(torch.from_numpy(a1).to(DEV), torch.from_numpy(b1).to(DEV), dot_precision="HIGHEST",
                              output_dtype=torch.float32, **TILE)
    assert np.array_equal(host(got), a1 @ b1)


def _sample_columns(n, head, width):
    """Column blocks (one bn tile of output each) at both ends of the head
    and of the rest."""
    return sorted({0, head - width, head, n - width})


@pytest.mark.parametrize("epilogue,perm", [(None, 0), ("swiglu", 0), ("geglu", 5), ("residual_add", 3),
                                           ("bias_add", 6)])
def test_epilogues_match_oracle_and_both_kernels(epilogue, perm):
    m, k, n = hybrid_shape(4096)
    head = head_columns(m, k, n)
    rng, a, b = _gaussian(970 + perm, m, k, n)
    gated = epilogue in ("swiglu", "geglu")
    b_use = o.swiglu_weight_layout(b, 1024) if gated else b
    kw = dict(TILE, epilogue=epilogue, block_permutation=perm)
    okw = dict(TILE, epilogue=epilogue, block_permutation=perm)
    res = bias = None
    if epilogue == "residual_add":
        res = o.bf16_round(rng.standard_normal((m, n)).astype(np.float32))
        kw["residual"] = dev(res)
    if epilogue == "bias_add":
        bias = o.bf16_round(rng.standard_normal(n).astype(np.float32))
        kw["bias"] = dev(bias)
    w = smx.strassen_weight_layout(dev_weight(b_use), 1024, 512, block_permutation=perm)
    a_dev = dev(a)
    got = host(rounds_matmul(a_dev, w, **kw))
    # The head is the product-major kernel's own result, the rest the split
    # kernel's (its last round split over K, as the whole call's on the split
    # kernel alone splits other tiles: up to the order of FP32 additions).
    out_head = head // 2 if gated else head
    assert np.array_equal(got[:, :out_head], host(pm_matmul(a_dev, w, **kw))[:, :out_head])
    with smx.strassen_kernel("split"):
        split = host(smx.strassen_matmul(a_dev, w, **kw))
    assert_ulp_close(got[:, out_head:], split[:, out_head:], k=k)
    # The oracle on one bn tile of columns at each end of both parts (a
    # tile depends only on its own rows and columns).
    for c0 in _sample_columns(n, head, 1024):
        sub = dict(okw)
        if res is not None:
            sub["residual"] = res[:, c0:c0 + 1024]
        if bias is not None:
            sub["bias"] = bias[c0:c0 + 1024]
        want = o.strassen_matmul(a, b_use[:, c0:c0 + 1024], **sub)
        oc = c0 // 2 if gated else c0
        assert_ulp_close(got[:, oc:oc + want.shape[1]], want, k=k)


def test_fp32_output_and_fp32_auxiliaries():
    m, k, n = hybrid_shape(4096)
    head = head_columns(m, k, n)
    rng, a, b = _gaussian(980, m, k, n)
    w = smx.strassen_weight_layout(dev_weight(b), 1024, 512)
    a_dev = dev(a)
    r = rng.standard_normal((m, n)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    for extra in (dict(output_dtype=torch.float32),
                  dict(epilogue="residual_add", residual=torch.from_numpy(r).to(DEV)),
                  dict(epilogue="bias_add", bias=torch.from_numpy(bias).to(DEV))):
        got = host(rounds_matmul(a_dev, w, **TILE, **extra))
        assert np.array_equal(got[:, :head], host(pm_matmul(a_dev, w, **TILE, **extra))[:, :head])
        # The rest against the split kernel alone: the same tiles, their K
        # split in another place, so the FP32 sums differ only in order.
        with smx.strassen_kernel("split"):
            split = host(smx.strassen_matmul(a_dev, w, **TILE, **extra))[:, head:]
        if extra.get("output_dtype") is torch.float32:
            assert np.all(np.abs(got[:, head:] - split) <= 8 * np.abs(split) * 2.0 ** -23 + fp32_floor(split, k))
        else:
            assert_ulp_close(got[:, head:], split, k=k)
    c0 = head
    want = o.strassen_matmul(a, b[:, c0:c0 + 1024], **TILE, epilogue="residual_add", residual=r[:, c0:c0 + 1024])
    got = host(rounds_matmul(a_dev, w, **TILE, epilogue="residual_add", residual=torch.from_numpy(r).to(DEV)))
    assert_ulp_close(got[:, c0:c0 + 1024], want, k=k)


def test_both_product_major_flags_are_refused():
    m, k, n = 1024, 1024, 2048
    d = _lib.SmxGemmDesc()
    d.m, d.n, d.k = m, n, k
    d.lda, d.ldb, d.ldc = k, k, n
    d.bm, d.bn, d.bk = 1024, 1024, 512
    d.algo, d.epilogue = 7, _lib.SMX_EPI[None]
    d.a_layout, d.b_layout = _lib.SMX_A_PACKED, _lib.SMX_B_PACKED
    d.flags = _lib.SMX_FLAG_PRODUCT_MAJOR | _lib.SMX_FLAG_PRODUCT_MAJOR_ROUNDS
    need = ctypes.c_int64()
    lib = _lib.load()
    assert lib.smx_gemm_workspace_bytes(d, ctypes.byref(need)) == _lib.SMX_ERR_INVALID
    assert b"exclude each other" in lib.smx_last_error()


def test_bench_head_columns_match_the_library():
    """bench.py times the gate|up call's product-major head alone on the
    columns its head_columns names: those must be the library's head. At
    8192 x 5120 x 51200 the rest (256 split tiles, one whole round) splits
    nothing over K, so the workspace is the head's parked sets alone."""
    import bench

    m, k, n = bench.TOKENS, bench.HIDDEN, 2 * bench.FFN
    head = bench.head_columns(m, k, n, 1024, _cus())
    assert 0 < head <= n
    assert head == head_columns(m, k, n)
    need = _workspace_bytes(m, n, k, _lib.SMX_FLAG_PRODUCT_MAJOR_ROUNDS, epilogue="swiglu")
    assert need == (m // 256) * (head // 512) * PARK_PER_TILE
