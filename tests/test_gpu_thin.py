"""GPU parity of the reference-legal tiles and head widths the kernels' fast
paths do not cover directly, against the CPU oracle:

* thin tilings: bm % 16 with bm/2 not a multiple of the kernels' 128-row
  product tile (decode-sized M among them). The packed A holds product rows
  in order, zero-padded to whole tiles, and the epilogue maps every output row
  (strassen_pallas.py:127-140 allows bm % 16; :188-204 split each bm-row tile
  into row halves);
* qk_norm_rope with head_dim other than 128 (strassen_pallas.py:986-1003
  allows any head_dim with bn % (2 head_dim) == 0), which runs as the GEMM
  with an FP32 result and the per-head pass smx_qk_norm_rope.

Bars as in test_gpu_parity: exact-integer operands bit-exact; random bf16
operands within one bf16 ulp of the oracle; packed layouts byte-identical.
"""

import numpy as np
import pytest
import torch

import oracle as o
import strassen_tpu_amd as smx
from test_gpu_parity import (ARMS, DEV, _qk_problem, assert_ulp_close, dev, dev32, dev_weight, host, oracle_arm,
                             run_arm, say)

pytestmark = pytest.mark.gpu

# (m, k, n), (bm, bn, bk): product rows M/2 = 8, 24, 48, 272 (thin: none a
# multiple of 128; the last two span several product tiles or leave one
# partly padded)
THIN_CASES = [
    ((16, 512, 512), (16, 256, 256)),
    ((48, 512, 256), (16, 256, 512)),
    ((96, 1024, 512), (48, 256, 512)),
    ((544, 512, 512), (272, 256, 256)),
]


@pytest.fixture(autouse=True)
def _announce(request):
    say(f"\n[gpu] {request.node.nodeid}")
    yield
    torch.cuda.synchronize()


@pytest.mark.parametrize("algo", [7, 8])
@pytest.mark.parametrize("shape,tile", THIN_CASES)
def test_thin_pack_matches_oracle(algo, shape, tile):
    """The packers' thin-tiling output, zero padding included, for a bf16
    row-major A (pack_rows), a float32 A (pack_operand) and a transposed A."""
    (m, k, _), (bm, _, bk) = shape, tile
    rng = np.random.default_rng(41)
    a = o.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    want = o.packed_operand(a, algo, "lhs", bm, bk)
    assert want.size * 2 == smx.packing.packed_bytes(algo, m, k)
    got = smx.pack_activation(dev(a), algo, bm, bk)
    assert np.array_equal(host(got.data), want)
    got32 = smx.pack_activation(dev32(a), algo, bm, bk)
    assert np.array_equal(host(got32.data), want)
    got_t = smx.packing.pack_operand(dev(np.ascontiguousarray(a.T)), algo=algo, side="lhs_t", tile_rows=bm, bk=bk)
    assert np.array_equal(host(got_t.data), want)


@pytest.mark.parametrize("arm", ARMS)
@pytest.mark.parametrize("shape,tile", THIN_CASES)
def test_thin_integer_kat_bit_exact(arm, shape, tile):
    """Exact-integer operands: every arm (a plain weight on a thin tile runs
    packed, the compact kernel needing bm % 256) equals A @ B rounded once."""
    m, k, n = shape
    bm, bn, bk = tile
    rng = np.random.default_rng(187)
    a = rng.integers(-2, 3, (m, k)).astype(np.float32)
    b = rng.integers(-2, 3, (k, n)).astype(np.float32)
    got = host(run_arm(arm, a, b, bm=bm, bn=bn, bk=bk))
    assert np.array_equal(got, o.bf16_round(a @ b))


@pytest.mark.parametrize("shape,tile", THIN_CASES)
def test_thin_random_matches_oracle(shape, tile):
    m, k, n = shape
    bm, bn, bk = tile
    rng = np.random.default_rng(7)
    a = o.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    b = o.bf16_round((rng.standard_normal((k, n)) * 0.05).astype(np.float32))
    for arm in ("strassen_packed", "cubic_packed"):
        got = host(run_arm(arm, a, b, bm=bm, bn=bn, bk=bk))
        assert_ulp_close(got, oracle_arm(arm, a, b, bm=bm, bn=bn, bk=bk), k=k)
        got32 = host(run_arm(arm, a, b, bm=bm, bn=bn, bk=bk, output_dtype=torch.float32))
        want32 = oracle_arm(arm, a, b, bm=bm, bn=bn, bk=bk, output_dtype="float32")
        np.testing.assert_allclose(got32, want32, rtol=2e-5, atol=1e-5 * float(np.abs(want32).max()))


@pytest.mark.parametrize("shape,tile", [THIN_CASES[1], THIN_CASES[3]])
def test_thin_fused_epilogues(shape, tile):
    """SwiGLU, residual (bf16 and float32), bias and (where bn spans the
    row) norm_residual_add on thin tilings: every output row through the
    epilogue's row map."""
    m, k, n = shape
    bm, bn, bk = tile
    rng = np.random.default_rng(3)
    a = o.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    b = o.bf16_round((rng.standard_normal((k, n)) * 0.05).astype(np.float32))
    res = o.bf16_round(rng.standard_normal((m, n)).astype(np.float32))
    bias = o.bf16_round(rng.standard_normal(n).astype(np.float32))
    scale = o.bf16_round((1 + 0.1 * rng.standard_normal(n)).astype(np.float32))
    cases = [
        (dict(epilogue="swiglu"), dict(epilogue="swiglu")),
        (dict(epilogue="residual_add", residual=dev(res)), dict(epilogue="residual_add", residual=res)),
        (dict(epilogue="residual_add", residual=torch.from_numpy(res).to(DEV)),
         dict(epilogue="residual_add", residual=res)),
        (dict(epilogue="bias_add", bias=dev(bias)), dict(epilogue="bias_add", bias=bias)),
    ]
    if bn == n:  # the row norm spans the output row: the tile must span it too
        cases.append((dict(epilogue="norm_residual_add", residual=dev(res), norm_scale=dev(scale)),
                      dict(epilogue="norm_residual_add", residual=res, norm_scale=scale)))
    for arm in ("strassen_packed", "cubic_packed"):
        for kw_dev, kw_ref in cases:
            say(f"  {arm} {kw_ref['epilogue']}")
            got = host(run_arm(arm, a, b, bm=bm, bn=bn, bk=bk, **kw_dev))
            assert_ulp_close(got, oracle_arm(arm, a, b, bm=bm, bn=bn, bk=bk, **kw_ref), k=k)


def test_thin_variants_and_exact_panels():
    """The dual formula under a block permutation, and an exact-panel
    schedule (the cubic adds the Strassen panels' FP32 partial in its thin
    epilogue), on a thin tiling."""
    (m, k, n), (bm, bn, bk) = (96, 1024, 512), (48, 256, 256)
    rng = np.random.default_rng(5)
    a = o.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    b = o.bf16_round((rng.standard_normal((k, n)) * 0.05).astype(np.float32))
    res = o.bf16_round(rng.standard_normal((m, n)).astype(np.float32))
    for formula, perm in (("dual", 5), ("classical", 3)):
        w = smx.strassen_weight_layout(dev_weight(b), bn, bk, formula_variant=formula, block_permutation=perm)
        got = host(smx.strassen_matmul(dev(a), w, bm=bm, bn=bn, bk=bk, formula_variant=formula,
                                       block_permutation=perm, epilogue="residual_add", residual=dev(res)))
        want = o.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk, formula_variant=formula, block_permutation=perm,
                                 epilogue="residual_add", residual=res)
        assert_ulp_close(got, want, k=k)
    got = host(smx.strassen_matmul(dev(a), dev_weight(b), bm=bm, bn=bn, bk=bk, classical_panels=(1, 2),
                                   epilogue="swiglu"))
    want = o.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk, classical_panels=(1, 2), epilogue="swiglu")
    assert_ulp_close(got, want, k=k)


def test_thin_qk_norm_rope_fused():
    """The fused q/k epilogue (head_dim 128) on a thin tiling: its RoPE
    tables are read by mapped output row."""
    batch, seq, heads, k, bn = 3, 16, 4, 1024, 256
    x, w, laid, tcos, tsin, scale = _qk_problem(13, batch, seq, heads, k, bn)
    kw = dict(bm=16, bn=bn, bk=512, epilogue="qk_norm_rope", rope_head_dim=128, rope_eps=1e-6)
    laid_dev = smx.rope_weight_layout(dev_weight(w), bn)
    for arm in ("strassen_packed", "cubic_packed", "strassen_plain"):
        got = host(run_arm(arm, x, laid_dev, rope_cos=dev(tcos), rope_sin=dev(tsin),
                           rope_scale=torch.from_numpy(scale).to(DEV), **kw))
        want = oracle_arm(arm, x, laid, rope_cos=tcos, rope_sin=tsin, rope_scale=scale, **kw)
        assert_ulp_close(got, want, k=k)


# head_dim, bn, heads: two heads per tile half at 64, one at 256, and 48-column
# head halves that do not align with the kernels' 32-column blocks at 96
HEAD_CASES = [(64, 256, 8), (256, 512, 4), (96, 768, 8)]


@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("hd,bn,heads", HEAD_CASES)
def test_qk_norm_rope_other_head_widths(hd, bn, heads, scale_dtype):
    batch, seq, k = 2, 256, 512
    x, w, laid, tcos, tsin, scale = _qk_problem(17, batch, seq, heads, k, bn, hd)
    kw = dict(bm=256, bn=bn, bk=256, epilogue="qk_norm_rope", rope_head_dim=hd, rope_eps=1e-6)
    laid_dev = smx.rope_weight_layout(dev_weight(w), bn, hd)
    assert np.array_equal(host(laid_dev), laid)
    for arm in ARMS:
        got = host(run_arm(arm, x, laid_dev, rope_cos=dev(tcos), rope_sin=dev(tsin),
                           rope_scale=torch.from_numpy(scale).to(DEV).to(scale_dtype), **kw))
        want = oracle_arm(arm, x, laid, rope_cos=tcos, rope_sin=tsin, rope_scale=scale, **kw)
        assert_ulp_close(got, want, k=k)


def test_qk_norm_rope_thin_and_other_head_width():
    """Both at once: a decode-sized thin tiling with head_dim 64."""
    batch, seq, heads, k, bn, hd = 1, 32, 8, 512, 256, 64
    x, w, laid, tcos, tsin, scale = _qk_problem(19, batch, seq, heads, k, bn, hd)
    kw = dict(bm=16, bn=bn, bk=256, epilogue="qk_norm_rope", rope_head_dim=hd, rope_eps=1e-6)
    laid_dev = smx.rope_weight_layout(dev_weight(w), bn, hd)
    for arm in ("strassen_packed", "cubic_packed"):
        got = host(run_arm(arm, x, laid_dev, rope_cos=dev(tcos), rope_sin=dev(tsin),
                           rope_scale=torch.from_numpy(scale).to(DEV), **kw))
        want = oracle_arm(arm, x, laid, rope_cos=tcos, rope_sin=tsin, rope_scale=scale, **kw)
        assert_ulp_close(got, want, k=k)


def test_decode_sized_gate_up_swiglu():
    """16 decode tokens at the Qwen3-32B gate|up depth (K 5120; N 8192 of
    the 51200 gate|up columns) with SwiGLU, the weight packed once and
    bm = 16, against the oracle over the whole output."""
    m, k, n, bn, bk = 16, 5120, 8192, 1024, 512
    rng = np.random.default_rng(23)
    a = o.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    b = o.bf16_round((rng.standard_normal((k, n)) * 0.02).astype(np.float32))
    laid = o.swiglu_weight_layout(b, bn)
    b_dev = smx.swiglu_weight_layout(dev_weight(b), bn)
    for arm, pack, ref in (("strassen", smx.strassen_weight_layout, o.strassen_matmul),
                           ("cubic", smx.cubic_weight_layout, o.cubic_blocked_matmul)):
        say(f"  {arm}")
        fn = smx.strassen_matmul if arm == "strassen" else smx.cubic_matmul
        got = host(fn(dev(a), pack(b_dev, bn, bk), bm=16, bn=bn, bk=bk, epilogue="swiglu"))
        assert_ulp_close(got, ref(a, laid, bm=16, bn=bn, bk=bk, epilogue="swiglu"), k=k)


@pytest.mark.parametrize("out_f32,scale_f32", [(True, False), (False, True), (True, True)])
def test_qk_norm_rope_pass_through_c_abi(out_f32, scale_f32):
    """smx_qk_norm_rope on an FP32 product, through the C ABI, against the
    oracle's per-head RMSNorm + RoPE on the same FP32 values: the float32
    output agrees to float32 summation noise, the bf16 one to a bf16 ulp."""
    import ctypes

    from oracle import strassen_ref as ref
    from strassen_tpu_amd import _lib

    m, n, bn, hd, eps = 512, 1536, 768, 96, 1e-6
    rng = np.random.default_rng(29)
    x = rng.standard_normal((m, n)).astype(np.float32)
    cos, sin = o.rope_values(m, hd, 1e6)
    tcos, tsin = o.rope_layout_tables(cos, sin, bn // 2, hd)
    scale = o.rope_scale_layout(o.bf16_round((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)), bn, hd)
    quads = ref._quadrants_of(x, 256, bn)
    want = ref._qk_norm_rope(quads, m, n, 256, bn, tcos, tsin, scale, hd, eps)
    x_dev = torch.from_numpy(x).to(DEV)
    scale_dev = torch.from_numpy(scale).to(DEV)
    scale_dev = scale_dev if scale_f32 else scale_dev.to(torch.bfloat16)
    out = torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=DEV)
    dtypes = (_lib.SMX_QK_OUT_F32 if out_f32 else 0) | (_lib.SMX_QK_SCALE_F32 if scale_f32 else 0)
    # the tables live in variables until the pass has read them
    cos_dev, sin_dev = dev(tcos), dev(tsin)
    stream = ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)
    _lib.check(_lib.load().smx_qk_norm_rope(m, n, _lib.ptr(x_dev), n, _lib.ptr(cos_dev), _lib.ptr(sin_dev),
                                            _lib.ptr(scale_dev), dtypes, bn, hd, eps, _lib.ptr(out), n, stream))
    got = host(out)
    if out_f32:
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-6)
    else:
        assert_ulp_close(got, o.bf16_round(want), k=hd)


def test_thin_tiling_fp32_inputs_highest_precision():
    """A thin tiling with float32 inputs at HIGHEST precision (six bf16
    passes per product): the packed A's padding rows stay zero in every
    pass, and the FP32 result matches the oracle's."""
    from test_gpu_parity import _gaussian32, assert_f32_close, dev32_weight

    _, a, b = _gaussian32(7, 48, 1024, 512)
    kw = dict(bm=16, bn=256, bk=512, dot_precision="highest")
    for arm, fn, ref in (("strassen", smx.strassen_matmul, o.strassen_matmul),
                         ("cubic", smx.cubic_matmul, o.cubic_blocked_matmul)):
        say(f"  {arm}")
        got = host(fn(dev32(a), dev32_weight(b), **kw))
        okw = dict(kw, input_dtype="float32") if arm == "strassen" else dict(kw)
        want = ref(a, b, output_dtype="float32", **okw)
        assert_f32_close(got, want, 6 * 1024)
