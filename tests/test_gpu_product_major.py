"""GPU parity of the product-major Strassen kernel (SMX_FLAG_PRODUCT_MAJOR).

The kernel runs the seven products of a 128 x 256 product-space tile one
after another, each over the whole K range, into three FP32 register sets,
and parks two partial sets per workgroup in the workspace; the products are
the classical ones (strassen_pallas.py:324-379), so its results are the
oracle's up to the order of FP32 additions: within one bf16 ulp (plus the
FP32 floor near zero) of the oracle and of the default kernel, and bit-exact
on integer operands. Every epilogue it fuses, FP32 output, FP32 residual and
bias, every block permutation, several tile grids and tile orders, and the
calls it hands back to the default kernel (a q/k epilogue, the dual formula,
bn/2 not a multiple of 256, K not a multiple of 128) are checked through the
surface (strassen_kernel("product_major")) and the C ABI.
"""

import ctypes

import numpy as np
import pytest
import torch

import oracle as o
import strassen_tpu_amd as smx
from strassen_tpu_amd import _lib
from test_gpu_parity import DEV, _gaussian, assert_ulp_close, dev, dev_weight, fp32_floor, host, say

pytestmark = pytest.mark.gpu

PARK_PER_TILE = 256 * 1024  # two parked FP32 sets of a 128 x 256 product tile


@pytest.fixture(autouse=True)
def _announce(request):
    say(f"\n[gpu] {request.node.nodeid}")
    yield
    torch.cuda.synchronize()


def pm_matmul(a, b, **kw):
    with smx.strassen_kernel("product_major"):
        return smx.strassen_matmul(a, b, **kw)


def _workspace_bytes(m, n, k, tile, epilogue=None, flags=_lib.SMX_FLAG_PRODUCT_MAJOR, formula=0):
    d = _lib.SmxGemmDesc()
    d.m, d.n, d.k = m, n, k
    d.lda, d.ldb = k, k
    d.ldc = n // 2 if epilogue in ("swiglu", "geglu") else n
    d.bm, d.bn, d.bk = tile
    d.algo, d.epilogue = 7, _lib.SMX_EPI[epilogue]
    d.a_layout, d.b_layout = _lib.SMX_A_PACKED, _lib.SMX_B_PACKED
    d.flags, d.formula = flags, formula
    d.rope_head_dim, d.rope_eps = 128, 1e-6
    need = ctypes.c_int64()
    _lib.check(_lib.load().smx_gemm_workspace_bytes(d, ctypes.byref(need)))
    return need.value


def test_workspace_is_two_parked_sets_per_tile():
    """A call the kernel takes asks for 256 KB per 128 x 256 product tile;
    one it hands back asks for what the default kernel asks for."""
    m, n, k, tile = 2048, 4096, 2048, (1024, 1024, 512)
    tiles = (m // 2 // 128) * (n // 2 // 256)
    assert _workspace_bytes(m, n, k, tile) == tiles * PARK_PER_TILE
    assert _workspace_bytes(m, n, k, tile, epilogue="swiglu") == tiles * PARK_PER_TILE
    default = _workspace_bytes(m, n, k, tile, flags=0)
    assert _workspace_bytes(m, n, k, (1024, 256, 512)) == default  # bn/2 = 128
    assert _workspace_bytes(m, n, k, tile, formula=1) == default  # dual formula
    assert _workspace_bytes(m, n, k, tile, epilogue="qk_norm_rope") == _workspace_bytes(
        m, n, k, tile, epilogue="qk_norm_rope", flags=0)
    assert _workspace_bytes(m, n, 1152, (1024, 1024, 128)) == tiles * PARK_PER_TILE  # K % 128 == 0
    assert _workspace_bytes(m, n, 2112, (1024, 1024, 64)) == _workspace_bytes(m, n, 2112, (1024, 1024, 64),
                                                                              flags=0)  # K % 128 != 0


INT_CASES = [
    ((512, 1024, 1024), (256, 512, 512)),
    ((1024, 2048, 2048), (1024, 1024, 512)),
    ((768, 768, 1536), (256, 512, 256)),  # 3 x 3 tiles, K = 6 pipeline stages per product
]


@pytest.mark.parametrize("shape,tile", INT_CASES)
def test_integer_kat_bit_exact(shape, tile):
    m, k, n = shape
    bm, bn, bk = tile
    rng = np.random.default_rng(881)
    a = rng.integers(-2, 3, (m, k)).astype(np.float32)
    b = rng.integers(-2, 3, (k, n)).astype(np.float32)
    w = smx.strassen_weight_layout(dev_weight(b), bn, bk)
    assert _workspace_bytes(m, n, k, tile) == (m // 256) * (n // 512) * PARK_PER_TILE
    got = host(pm_matmul(dev(a), w, bm=bm, bn=bn, bk=bk))
    assert np.array_equal(got, o.bf16_round(a @ b))
    got32 = host(pm_matmul(dev(a), w, bm=bm, bn=bn, bk=bk, output_dtype=torch.float32))
    assert np.array_equal(got32, a @ b)


@pytest.mark.parametrize("epilogue", [None, "swiglu", "geglu", "residual_add", "bias_add"])
@pytest.mark.parametrize("perm", [0, 3, 5, 6])
def test_epilogues_match_oracle_and_default_kernel(epilogue, perm):
    m, k, n = 1024, 1024, 2048
    tile = bm, bn, bk = 512, 1024, 512
    rng, a, b = _gaussian(900 + perm, m, k, n)
    kw = dict(bm=bm, bn=bn, bk=bk, epilogue=epilogue, block_permutation=perm)
    okw = dict(kw)
    b_use = b
    if epilogue in ("swiglu", "geglu"):
        b_use = o.swiglu_weight_layout(b, bn)
    if epilogue == "residual_add":
        r = o.bf16_round(rng.standard_normal((m, n)).astype(np.float32))
        kw["residual"], okw["residual"] = dev(r), r
    if epilogue == "bias_add":
        bias = o.bf16_round(rng.standard_normal(n).astype(np.float32))
        kw["bias"], okw["bias"] = dev(bias), bias
    w = smx.strassen_weight_layout(dev_weight(b_use), bn, bk, block_permutation=perm)
    a_dev = dev(a)
    got = host(pm_matmul(a_dev, w, **kw))
    want = o.strassen_matmul(a, b_use, **okw)
    assert_ulp_close(got, want, k=k)
    default = host(smx.strassen_matmul(a_dev, w, **kw))
    assert_ulp_close(got, default, k=k)


def test_fp32_output_and_fp32_auxiliaries():
    m, k, n = 512, 2048, 2048
    bm, bn, bk = 256, 512, 512
    rng, a, b = _gaussian(911, m, k, n)
    w = smx.strassen_weight_layout(dev_weight(b), bn, bk)
    got = host(pm_matmul(dev(a), w, bm=bm, bn=bn, bk=bk, output_dtype=torch.float32))
    want = o.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk, output_dtype="float32")
    # FP32 summation order differs: a few FP32 ulps plus the near-zero floor.
    assert np.all(np.abs(got - want) <= 4 * np.abs(want) * 2.0 ** -23 + fp32_floor(want, k))
    r = rng.standard_normal((m, n)).astype(np.float32)
    got = host(pm_matmul(dev(a), w, bm=bm, bn=bn, bk=bk, epilogue="residual_add",
                         residual=torch.from_numpy(r).to(DEV)))
    assert_ulp_close(got, o.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk, epilogue="residual_add", residual=r), k=k)
    bias = rng.standard_normal(n).astype(np.float32)
    got = host(pm_matmul(dev(a), w, bm=bm, bn=bn, bk=bk, epilogue="bias_add", bias=torch.from_numpy(bias).to(DEV)))
    assert_ulp_close(got, o.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk, epilogue="bias_add", bias=bias), k=k)


@pytest.mark.parametrize("shape", [(2048, 1024, 4096), (4096, 512, 3072), (1536, 2560, 1536)])
def test_tile_grids_match_oracle(shape):
    """Grids of 64, 96 and 18 tiles (whole and partial XCD groups, several
    tile orders), checked tile by tile against the oracle on sampled 1024 x
    1024 blocks (a Strassen tile depends only on its own rows and columns)."""
    m, k, n = shape
    bm, bn, bk = 512, 512, 512
    _, a, b = _gaussian(920 + m // 512, m, k, n)
    w = smx.strassen_weight_layout(dev_weight(b), bn, bk)
    got = host(pm_matmul(dev(a), w, bm=bm, bn=bn, bk=bk))
    for r0, c0 in ((0, 0), (m - 512, n - 512), ((m // 1024) * 512, (n // 1024) * 512)):
        sub = o.strassen_matmul(a[r0:r0 + 512], b[:, c0:c0 + 512], bm=bm, bn=bn, bk=bk)
        assert_ulp_close(got[r0:r0 + 512, c0:c0 + 512], sub, k=k)


def test_calls_it_cannot_take_run_the_default_kernel():
    """Under strassen_kernel("product_major"), the dual formula and a bn/2
    of 128 run the default kernel and still match the oracle (the workspace
    test above covers the q/k epilogue's hand-back)."""
    m, k, n = 512, 1024, 1024
    _, a, b = _gaussian(930, m, k, n)
    a_dev = dev(a)
    w = smx.strassen_weight_layout(dev_weight(b), 256, 512)
    assert_ulp_close(host(pm_matmul(a_dev, w, bm=256, bn=256, bk=512)),
                     o.strassen_matmul(a, b, bm=256, bn=256, bk=512), k=k)
    wd = smx.strassen_weight_layout(dev_weight(b), 512, 512, formula_variant="dual")
    assert_ulp_close(host(pm_matmul(a_dev, wd, bm=256, bn=512, bk=512, formula_variant="dual")),
                     o.strassen_matmul(a, b, bm=256, bn=512, bk=512, formula_variant="dual"), k=k)


def test_short_workspace_is_refused():
    m, k, n, tile = 512, 1024, 1024, (256, 512, 512)
    rng = np.random.default_rng(940)
    a = o.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    b = o.bf16_round((rng.standard_normal((k, n)) * 0.05).astype(np.float32))
    pa = smx.packing.pack_operand(dev(a), algo=7, side="lhs", tile_rows=256, bk=512)
    pb = smx.packing.pack_operand(dev_weight(b), algo=7, side="rhs", tile_rows=512, bk=512)
    lib = _lib.load()
    d = _lib.SmxGemmDesc()
    d.m, d.n, d.k = m, n, k
    d.lda, d.ldb, d.ldc = k, k, n
    d.bm, d.bn, d.bk = tile
    d.algo, d.epilogue = 7, _lib.SMX_EPI[None]
    d.a_layout, d.b_layout = _lib.SMX_A_PACKED, _lib.SMX_B_PACKED
    d.flags = _lib.SMX_FLAG_PRODUCT_MAJOR
    need = _workspace_bytes(m, n, k, tile)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    for workspace, nbytes in ((None, 0), (ws.data_ptr(), need - 16)):
        d.workspace, d.workspace_bytes = workspace, nbytes
        rc = lib.smx_gemm(d, _lib.ptr(pa.data), _lib.ptr(pb.data), _lib.ptr(out), None, None, None, None, None,
                          stream)
        assert rc == _lib.SMX_ERR_INVALID
        assert b"workspace" in lib.smx_last_error()
    d.workspace, d.workspace_bytes = ws.data_ptr(), need
    _lib.check(lib.smx_gemm(d, _lib.ptr(pa.data), _lib.ptr(pb.data), _lib.ptr(out), None, None, None, None, None,
                            stream))
    assert_ulp_close(host(out), o.strassen_matmul(a, b, bm=256, bn=512, bk=512), k=k)


def test_repeated_calls_reuse_the_workspace():
    """Parked sets are written before they are read in every call: two calls
    in a row, the second smaller, on workspaces the caching allocator hands
    back, each match the oracle."""
    for m, seed in ((1024, 950), (512, 951)):
        _, a, b = _gaussian(seed, m, 1024, 2048)
        w = smx.strassen_weight_layout(dev_weight(b), 512, 512)
        got = host(pm_matmul(dev(a), w, bm=256, bn=512, bk=512))
        assert_ulp_close(got, o.strassen_matmul(a, b, bm=256, bn=512, bk=512), k=1024)
