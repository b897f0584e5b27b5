"""Pins for the CPU oracle (oracle/strassen_ref.py).

Each check is chosen so that a plausible mistake in the oracle fails it:
bf16 rounding against torch's conversion; Strassen/cubic algebra against
exact-integer products (reference technique,
Strassen_MM_Focus/tests/test_kernels_v001.py:59-80); operand-sum and output
rounding against the reference's published accuracy-gate errors on
regenerated inputs (archive/initial-snapshot/evidence/strassen_cubic_control.jsonl:7);
epilogues against closed forms and the unfused Qwen3 semantics.
"""

import json
import os

import numpy as np
import pytest
import torch

import oracle as o
from oracle import strassen_ref as ref

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---------------------------------------------------------------------------
# bf16 rounding
# ---------------------------------------------------------------------------

def test_bf16_round_matches_torch_conversion():
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.standard_normal(100000).astype(np.float32) * np.float32(10.0) ** rng.integers(-30, 30, 100000).astype(np.float32),
        np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, 3.3895314e38, -3.3895314e38, 1e-40, -1e-40], np.float32),
    ])
    # exact ties: bf16 value + half ulp, both parities of the kept mantissa
    base = o.bf16_round(rng.standard_normal(1000).astype(np.float32))
    ties = (base.view(np.uint32) | np.uint32(0x8000)).view(np.float32)
    x = np.concatenate([x, ties]).astype(np.float32)
    expected = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = o.bf16_bits(x)
    assert np.array_equal(got, expected)


def test_bf16_round_ties_to_even_closed_form():
    # 1 + 2^-8 is exactly halfway between 1 and 1 + 2^-7: ties to even -> 1.
    assert o.bf16_round(np.float32(1.0 + 2.0 ** -8)) == np.float32(1.0)
    # 1 + 3*2^-8 is halfway between 1+2^-7 (odd) and 1+2^-6 (even) -> 1+2^-6.
    assert o.bf16_round(np.float32(1.0 + 3 * 2.0 ** -8)) == np.float32(1.0 + 2.0 ** -6)
    assert np.isnan(o.bf16_round(np.float32(np.nan)))


# ---------------------------------------------------------------------------
# Algebra: exact-integer known answers
# ---------------------------------------------------------------------------

KAT_CASES = [
    # (m, k, n), (bm, bn, bk): several row/column tiles and K panels
    ((16, 256, 256), (16, 256, 256)),
    ((64, 1024, 512), (32, 256, 256)),
    ((48, 768, 768), (16, 256, 256)),
]


@pytest.mark.parametrize("shape,tile", KAT_CASES)
@pytest.mark.parametrize("interleave", [False, True])
def test_strassen_exact_integer_kat(shape, tile, interleave):
    rng = np.random.default_rng(187)
    m, k, n = shape
    bm, bn, bk = tile
    a = rng.integers(-2, 3, (m, k)).astype(np.float32)
    b = rng.integers(-2, 3, (k, n)).astype(np.float32)
    got = o.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk, interleave_products=interleave,
                            output_dtype="float32")
    assert np.array_equal(got, a @ b)
    got16 = o.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk, interleave_products=interleave)
    assert np.array_equal(got16, o.bf16_round(a @ b))


@pytest.mark.parametrize("shape,tile", KAT_CASES)
def test_cubic_exact_integer_kat(shape, tile):
    rng = np.random.default_rng(188)
    m, k, n = shape
    a = rng.integers(-2, 3, (m, k)).astype(np.float32)
    b = rng.integers(-2, 3, (k, n)).astype(np.float32)
    got = o.cubic_blocked_matmul(a, b, bm=tile[0], bn=tile[1], bk=tile[2], output_dtype="float32")
    assert np.array_equal(got, a @ b)


def _textbook_tile_strassen(a, b, bm, bn, bk):
    """One-level Strassen on every (bm, bn) output tile from the textbook
    formulas (M1..M7 and the four quadrant sums of Strassen 1969, as in
    Cormen et al., ch. 4.2) written on explicit per-tile slices, with every
    operand sum rounded once to bf16 as the reference's bf16 path does; the
    products and their combination in float64."""
    m, k = a.shape
    n = b.shape[1]
    hm, hn, hk = bm // 2, bn // 2, bk // 2

    def r(x):
        return o.bf16_round(x.astype(np.float32)).astype(np.float64)

    out = np.zeros((m, n))
    for i in range(m // bm):
        for j in range(n // bn):
            c11 = c12 = c21 = c22 = 0.0
            for p in range(k // bk):
                A = a[i * bm:(i + 1) * bm, p * bk:(p + 1) * bk].astype(np.float64)
                B = b[p * bk:(p + 1) * bk, j * bn:(j + 1) * bn].astype(np.float64)
                A11, A12, A21, A22 = A[:hm, :hk], A[:hm, hk:], A[hm:, :hk], A[hm:, hk:]
                B11, B12, B21, B22 = B[:hk, :hn], B[:hk, hn:], B[hk:, :hn], B[hk:, hn:]
                M1 = r(A11 + A22) @ r(B11 + B22)
                M2 = r(A21 + A22) @ B11
                M3 = A11 @ r(B12 - B22)
                M4 = A22 @ r(B21 - B11)
                M5 = r(A11 + A12) @ B22
                M6 = r(A21 - A11) @ r(B11 + B12)
                M7 = r(A12 - A22) @ r(B21 + B22)
                c11, c12 = c11 + M1 + M4 - M5 + M7, c12 + M3 + M5
                c21, c22 = c21 + M2 + M4, c22 + M1 - M2 + M3 + M6
            out[i * bm:i * bm + hm, j * bn:j * bn + hn] = c11
            out[i * bm:i * bm + hm, j * bn + hn:(j + 1) * bn] = c12
            out[i * bm + hm:(i + 1) * bm, j * bn:j * bn + hn] = c21
            out[i * bm + hm:(i + 1) * bm, j * bn + hn:(j + 1) * bn] = c22
    return out


@pytest.mark.parametrize("bm", [16, 48])
def test_thin_tile_row_pairing_against_textbook_tiles(bm):
    """Which rows meet in an operand sum (row r and r + bm/2 of each bm-row
    tile, strassen_pallas.py:188-204) changes the bf16 rounding of the sums
    only, so integer KATs cannot see it. The oracle's FP32 output agrees with
    the per-tile textbook computation to float32 summation noise (about
    1e-7), while the tilings that pair other rows differ by about 5e-3."""
    rng = np.random.default_rng(0)
    m, k, n = 96, 512, 256
    a = o.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    b = o.bf16_round((rng.standard_normal((k, n)) * 0.05).astype(np.float32))
    got = o.strassen_matmul(a, b, bm=bm, bn=256, bk=256, output_dtype="float32").astype(np.float64)

    def rel(x, y):
        return float(np.linalg.norm(x - y) / np.linalg.norm(y))

    assert rel(got, _textbook_tile_strassen(a, b, bm, 256, 256)) < 1e-6
    for other in (16, 32, 48, 96):
        if other != bm:
            assert rel(got, _textbook_tile_strassen(a, b, other, 256, 256)) > 1e-3


def test_thin_packed_operand_pads_zero_rows():
    """smx_pack_operand's layout restated for a thin tiling: the product
    rows in order (those of operand_planes), then zero rows up to a whole
    128-row tile."""
    rng = np.random.default_rng(2)
    a = o.bf16_round(rng.standard_normal((48, 512)).astype(np.float32))
    for algo, nops in ((7, 7), (8, 4)):
        planes = o.operand_planes(a, algo, "lhs", 16, 256)
        assert planes.shape == (nops, 24, 256)
        flat = o.packed_operand(a, algo, "lhs", 16, 256)
        unpacked = o.unpack_operand(flat, nops, 128, 256)
        assert np.array_equal(unpacked[:, :24], planes)
        assert not unpacked[:, 24:].any()


def test_kat_detects_planted_sign_error(monkeypatch):
    """A wrong sign in one operand sum must fail the integer KAT."""
    original = ref.strassen_products

    def broken(a_q, b_q, r=o.bf16_round):
        products = original(a_q, b_q, r)
        s, t = products[6]
        a0, a1, a2, a3 = a_q
        products[6] = (o.bf16_round(a2 + a0), t)  # should be A2 - A0
        return products

    monkeypatch.setattr(ref, "strassen_products", broken)
    rng = np.random.default_rng(187)
    a = rng.integers(-2, 3, (16, 256)).astype(np.float32)
    b = rng.integers(-2, 3, (256, 256)).astype(np.float32)
    got = o.strassen_matmul(a, b, bm=16, bn=256, bk=256, output_dtype="float32")
    assert not np.array_equal(got, a @ b)


def test_kat_detects_planted_quadrant_swap(monkeypatch):
    """Routing a product to the wrong quadrant must fail the integer KAT."""
    table = dict(ref.PRODUCT_UPDATES)
    table[3] = ((2, +1), (3, +1))  # P3 belongs to C1 and C3
    monkeypatch.setattr(ref, "PRODUCT_UPDATES", table)
    rng = np.random.default_rng(187)
    a = rng.integers(-2, 3, (16, 256)).astype(np.float32)
    b = rng.integers(-2, 3, (256, 256)).astype(np.float32)
    got = o.strassen_matmul(a, b, bm=16, bn=256, bk=256, output_dtype="float32")
    assert not np.array_equal(got, a @ b)


def test_bounded_nonzero_rounding_error():
    """Reference ``test_kernels_v001.py:82-96``: Gaussian bf16 operands give a
    Strassen error that is nonzero (operand sums are rounded) and < 0.02."""
    rng = np.random.default_rng(23)
    a = o.bf16_round(rng.normal(size=(16, 256)).astype(np.float32))
    b = o.bf16_round(rng.normal(size=(256, 256)).astype(np.float32))
    exact = a.astype(np.float64) @ b.astype(np.float64)
    got = o.strassen_matmul(a, b, bm=16, bn=256, bk=256, output_dtype="float32").astype(np.float64)
    rel = np.linalg.norm(got - exact) / np.linalg.norm(exact)
    assert 0.0 < rel < 0.02
    cubic = o.cubic_blocked_matmul(a, b, bm=16, bn=256, bk=256, output_dtype="float32").astype(np.float64)
    assert np.linalg.norm(cubic - exact) / np.linalg.norm(exact) < 1e-6 < rel


# ---------------------------------------------------------------------------
# Rounding: the reference's published accuracy gate on regenerated inputs
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def accuracy_gate_inputs():
    spec = json.load(open(os.path.join(GOLDEN, "accuracy_gate_reference.json")))
    a, b = o.host_uniform_inputs(tuple(spec["shape_mkn"]), spec["seed"])
    return spec, a, b, o.high_precision_reference(a, b)


@pytest.mark.slow
def test_oracle_reproduces_published_accuracy_gate(accuracy_gate_inputs):
    spec, a, b, reference = accuracy_gate_inputs
    bm, bn, bk = spec["tile_bm_bn_bk"]
    published = spec["errors_vs_reference"]
    strassen = o.device_error(o.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk), reference)
    cubic = o.device_error(o.cubic_blocked_matmul(a, b, bm=bm, bn=bn, bk=bk), reference)
    native = o.device_error(o.native_matmul(a, b), reference)
    # Same inputs, same operand roundings: only FP32 dot accumulation order
    # differs from the TPU, so the metrics agree to ~5 significant digits.
    for got, want in ((strassen, published["strassen"]), (cubic, published["cubic_blocked"]),
                      (native, published["native"])):
        assert got["l2_relative"] == pytest.approx(want["l2_relative"], rel=2e-4)
        assert got["rmse"] == pytest.approx(want["rmse"], rel=2e-4)
        assert got["maxnorm_relative"] == pytest.approx(want["maxnorm_relative"], rel=2e-3)


@pytest.mark.slow
def test_accuracy_gate_detects_planted_unrounded_sums(accuracy_gate_inputs, monkeypatch):
    """Dropping the bf16 rounding of the operand sums (a plausible mistake)
    moves the Strassen error far from the published value."""
    spec, a, b, reference = accuracy_gate_inputs
    monkeypatch.setattr(ref, "bf16_round", lambda x: np.asarray(x, np.float32))
    m, k, n = spec["shape_mkn"]
    a_small, b_small, r_small = a[:256], b[:, :256], reference[:256, :256]
    got = ref.strassen_matmul(a_small, b_small, bm=256, bn=256, bk=512, output_dtype="float32")
    err = o.device_error(got, r_small)["l2_relative"]
    assert err < 0.5 * spec["errors_vs_reference"]["strassen"]["l2_relative"]


# ---------------------------------------------------------------------------
# Epilogues
# ---------------------------------------------------------------------------

def _int_problem(seed, m, k, n, lo=-1, hi=2):
    rng = np.random.default_rng(seed)
    a = rng.integers(lo, hi, (m, k)).astype(np.float32)
    b = rng.integers(lo, hi, (k, n)).astype(np.float32)
    return rng, a, b


def test_residual_add_closed_form():
    rng, a, b = _int_problem(319, 32, 512, 512)
    r = rng.integers(-3, 4, (32, 512)).astype(np.float32)
    for pa in (False, True):
        got = o.strassen_matmul(a, b, bm=16, bn=256, bk=256, interleave_products=True,
                                epilogue="residual_add", residual=r, product_aware_residual=pa)
        assert np.array_equal(got, o.bf16_round(a @ b + r))


def test_bias_add_closed_form():
    rng, a, b = _int_problem(321, 32, 512, 512)
    bias = rng.integers(-3, 4, (512,)).astype(np.float32)
    got = o.strassen_matmul(a, b, bm=16, bn=256, bk=256, epilogue="bias_add", bias=bias)
    assert np.array_equal(got, o.bf16_round(a @ b + bias[None, :]))


def test_swiglu_closed_form_with_layout():
    """silu(gate) * up of the un-laid-out projection equals the fused
    epilogue on the laid-out weight (within one bf16 rounding of float32
    silu, evaluated here in float64)."""
    rng, a, b = _int_problem(318, 32, 512, 1024)
    bn = 256
    laid = o.swiglu_weight_layout(b, bn)
    exact = (a @ b).astype(np.float64)
    gate, up = np.split(exact, 2, axis=1)
    expected = gate / (1.0 + np.exp(-gate)) * up
    for pa in (False, True):
        got = o.strassen_matmul(a, laid, bm=16, bn=bn, bk=256, interleave_products=True,
                                epilogue="swiglu", product_aware_swiglu=pa)
        assert got.shape == (32, 512)
        np.testing.assert_allclose(got, expected, rtol=2 ** -7, atol=1e-6)


def test_gelu_tanh_against_torch_and_closed_form():
    """The GeGLU gate equals torch's gelu(approximate='tanh') (a separate
    implementation) and the erf GELU within the tanh approximation's error."""
    import math

    import torch

    x = np.linspace(-8, 8, 4001, dtype=np.float32)
    got = o.gelu_tanh(x)
    want = torch.nn.functional.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-6)
    exact = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in x.astype(np.float64)])
    assert np.max(np.abs(got - exact)) < 1e-3
    assert o.gelu_tanh(np.float32(0.0)) == 0.0


def test_geglu_closed_form_with_layout():
    """gelu_tanh(gate) * up of the un-laid-out projection equals the fused
    GeGLU epilogue on the laid-out weight (Strassen and cubic)."""
    rng, a, b = _int_problem(319, 32, 512, 1024)
    laid = o.swiglu_weight_layout(b, 256)
    exact = (a @ b).astype(np.float64)
    gate, up = np.split(exact, 2, axis=1)
    expected = 0.5 * gate * (1 + np.tanh(np.sqrt(2 / np.pi) * (gate + 0.044715 * gate ** 3))) * up
    for got in (o.strassen_matmul(a, laid, bm=16, bn=256, bk=256, epilogue="geglu"),
                o.cubic_blocked_matmul(a, laid, bm=16, bn=256, bk=256, epilogue="geglu")):
        assert got.shape == (32, 512)
        # float32 1 + tanh(x) cancels for very negative gates (as in the
        # reference's float32 gelu): a small absolute allowance there.
        np.testing.assert_allclose(got, expected, rtol=2 ** -7, atol=1e-5)


def test_fp32_output_is_the_unrounded_accumulator():
    """output_dtype float32 returns the FP32 quadrant values: on integer data
    exactly A @ B (no bf16 rounding), and the bf16 output is its rounding."""
    rng, a, b = _int_problem(320, 64, 512, 256)
    f32 = o.strassen_matmul(a, b, bm=32, bn=256, bk=256, output_dtype="float32")
    assert f32.dtype == np.float32 and np.array_equal(f32, a @ b)
    big = (a @ b) * 1000.5  # values no longer representable in bf16
    assert not np.array_equal(o.bf16_round(big), big)
    assert np.array_equal(o.strassen_matmul(a, b, bm=32, bn=256, bk=256), o.bf16_round(f32))


def test_product_aware_residual_bitwise_identical_to_interleaved():
    """strassen_pallas.py:640-643: same FP32 order, bitwise identical."""
    rng = np.random.default_rng(7)
    a = o.bf16_round(rng.standard_normal((64, 1024)).astype(np.float32))
    b = o.bf16_round(rng.standard_normal((1024, 512)).astype(np.float32) * np.float32(0.02))
    r = o.bf16_round(rng.standard_normal((64, 512)).astype(np.float32))
    std = o.strassen_matmul(a, b, bm=32, bn=256, bk=256, interleave_products=True,
                            epilogue="residual_add", residual=r)
    pa = o.strassen_matmul(a, b, bm=32, bn=256, bk=256, interleave_products=True,
                           epilogue="residual_add", residual=r, product_aware_residual=True)
    assert np.array_equal(std, pa)


def test_product_aware_swiglu_within_reference_gate():
    """benchmark_qwen3_32b_product_aware_inference.py:149-151: product-aware
    l2 <= standard fused l2 + 1e-3 against the unfused FP32 result."""
    rng = np.random.default_rng(20260904)
    a = o.bf16_round(rng.standard_normal((64, 1024)).astype(np.float32))
    b = o.bf16_round(rng.standard_normal((1024, 1024)).astype(np.float32) * np.float32(0.02))
    laid = o.swiglu_weight_layout(b, 256)
    exact = (a.astype(np.float64) @ b.astype(np.float64))
    gate, up = np.split(exact, 2, axis=1)
    expected = gate / (1.0 + np.exp(-gate)) * up
    std = o.strassen_matmul(a, laid, bm=32, bn=256, bk=256, interleave_products=True, epilogue="swiglu")
    pa = o.strassen_matmul(a, laid, bm=32, bn=256, bk=256, interleave_products=True, epilogue="swiglu",
                           product_aware_swiglu=True)
    e_std = o.device_error(std, expected)["l2_relative"]
    e_pa = o.device_error(pa, expected)["l2_relative"]
    assert e_pa <= e_std + 1e-3
    assert e_std < 2e-2


@pytest.mark.parametrize("hd,bn,heads", [(128, 256, 4), (64, 256, 4), (96, 768, 8), (256, 512, 4)])
def test_qk_norm_rope_matches_unfused_semantics(hd, bn, heads):
    """Fused per-head RMSNorm+RoPE on the rope layout equals the reference's
    unfused path (projection -> rms_norm per head -> apply_rope,
    benchmark_qwen3_32b_layer.py:270-284, 354-366) after rope_layout_to_heads,
    up to the bf16 roundings the unfused path adds, for head widths whose
    halves fill, share or straddle 32-column blocks."""
    rng = np.random.default_rng(11)
    batch, seq = 2, 16
    tokens, n, k = batch * seq, heads * hd, 512
    x = o.bf16_round(rng.standard_normal((tokens, k)).astype(np.float32))
    w = o.bf16_round(rng.standard_normal((k, n)).astype(np.float32) * np.float32(0.05))
    gamma = o.bf16_round((1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    cos, sin = o.rope_values(seq, hd, 1e6)
    laid = o.rope_weight_layout(w, bn, hd)
    tcos, tsin = o.rope_layout_tables(np.tile(cos, (batch, 1)), np.tile(sin, (batch, 1)), bn // 2, hd)
    scale = o.rope_scale_layout(gamma, bn, hd)
    fused = o.strassen_matmul(x, laid, bm=16, bn=bn, bk=256, epilogue="qk_norm_rope",
                              rope_cos=tcos, rope_sin=tsin, rope_scale=scale,
                              rope_head_dim=hd, rope_eps=1e-6)
    fused_heads = o.rope_layout_to_heads(fused, heads, bn, batch, seq, hd)
    # Unfused: the same Strassen projection in natural order, then the model ops.
    proj = o.strassen_matmul(x, w, bm=16, bn=bn, bk=256).reshape(batch, seq, heads, hd)
    unfused = o.apply_rope(o.rms_norm(proj, gamma), cos, sin)
    err = o.device_error(fused_heads, unfused)
    assert err["l2_relative"] < 1e-2
    # With no intermediate roundings the two paths differ by a few bf16 ulps.
    assert err["maxnorm_relative"] < 3e-2


# ---------------------------------------------------------------------------
# Relayouts: brute force and round trips
# ---------------------------------------------------------------------------

def test_swiglu_layout_brute_force():
    two_i, bn = 24, 8
    order = o.swiglu_weight_layout_order(two_i, bn)
    half, inter = bn // 2, two_i // 2
    for pos, src in enumerate(order):
        block, within = divmod(pos, bn)
        if within < half:
            assert src == block * half + within
        else:
            assert src == inter + block * half + within - half
    assert sorted(order) == list(range(two_i))


def test_rope_layout_round_trip_restores_heads():
    batch, seq, heads, hd, bn = 2, 3, 8, 16, 64
    tokens = batch * seq
    natural = np.arange(tokens * heads * hd, dtype=np.float32).reshape(tokens, heads * hd)
    laid = o.rope_weight_layout(natural, bn, hd)  # permute columns like a weight
    back = o.rope_layout_to_heads(laid, heads, bn, batch, seq, hd)
    assert np.array_equal(back, natural.reshape(batch, seq, heads, hd))


def test_rope_tables_and_scale_layout():
    cos = np.arange(5 * 16, dtype=np.float32).reshape(5, 16)
    sin = -cos
    tc, ts = o.rope_layout_tables(cos, sin, 32, 16)
    assert tc.shape == (5, 32) and np.array_equal(tc[:, 8:16], cos[:, :8])
    assert np.array_equal(ts, -tc)
    gamma = np.arange(16, dtype=np.float32)
    s = o.rope_scale_layout(gamma, 64, 16)
    assert np.array_equal(s, np.concatenate([np.tile(gamma[:8], 4), np.tile(gamma[8:], 4)]))


# ---------------------------------------------------------------------------
# Formula variants and block permutation (strassen_pallas.py:205-226, 381-517)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("formula", ["classical", "dual", "powers"])
def test_formula_variants_integer_known_answer(formula):
    """Small-integer operands keep every variant's operand expressions
    (multiples of 1/4) exact in bf16, so each formula, under every block
    permutation and both product orders, must equal A @ B bit-exactly; a
    wrong sign, operand or basis decode fails this."""
    rng, a, b = _int_problem(400, 64, 512, 256, lo=-2, hi=3)
    for perm in range(8):
        for interleave in (False, True):
            got = o.strassen_matmul(a, b, bm=32, bn=128, bk=256, formula_variant=formula,
                                    block_permutation=perm, interleave_products=interleave,
                                    output_dtype="float32")
            assert np.array_equal(got, a @ b), (formula, perm, interleave)


def _swap_tile_halves(x, tile_r, tile_c, swap_r, swap_c):
    """Physically swap the row halves / column halves of every tile."""
    r, c = x.shape
    v = x.reshape(r // tile_r, 2, tile_r // 2, c // tile_c, 2, tile_c // 2)
    if swap_r:
        v = v[:, ::-1]
    if swap_c:
        v = v[:, :, :, :, ::-1]
    return np.ascontiguousarray(v).reshape(r, c)


@pytest.mark.parametrize("formula", ["classical", "dual"])
def test_block_permutation_is_a_quadrant_relabelling(formula):
    """A permuted run equals the unpermuted formula applied to inputs whose
    tile halves were physically swapped, with the output halves swapped back
    (an independent route to the index map of :209-226), bit for bit on
    random bf16 data where roundings differ between permutations."""
    rng = np.random.default_rng(401)
    a = o.bf16_round(rng.standard_normal((64, 512)).astype(np.float32))
    b = o.bf16_round(rng.standard_normal((512, 256)).astype(np.float32))
    bm, bn, bk = 32, 128, 256
    base = o.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk, formula_variant=formula)
    distinct = 0
    for perm in range(8):
        sm, sk, sn = perm & 1, (perm >> 1) & 1, (perm >> 2) & 1
        got = o.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk, formula_variant=formula, block_permutation=perm)
        a2 = _swap_tile_halves(a, bm, bk, sm, sk)
        b2 = _swap_tile_halves(b, bk, bn, sk, sn)
        want = _swap_tile_halves(o.strassen_matmul(a2, b2, bm=bm, bn=bn, bk=bk, formula_variant=formula),
                                 bm, bn, sm, sn)
        assert np.array_equal(got, want), perm
        distinct += not np.array_equal(got, base)
    assert distinct >= 6  # permutations change the roundings


def test_formula_variants_error_band_and_rules():
    """Dual and powers stay in the classical error band on random data (no
    published figures exist for them); powers refuses fused epilogues."""
    a, b = o.host_uniform_inputs((256, 2048, 256), 20260833)
    a, b = o.bf16_round(a), o.bf16_round(b)
    ref = o.high_precision_reference(a, b).astype(np.float64)
    errs = {f: o.device_error(o.strassen_matmul(a, b, bm=128, bn=128, bk=512, formula_variant=f), ref)["l2_relative"]
            for f in ("classical", "dual", "powers")}
    cubic = o.device_error(o.cubic_blocked_matmul(a, b, bm=128, bn=128, bk=512), ref)["l2_relative"]
    for f, e in errs.items():
        assert cubic < e < 3 * errs["classical"], (f, errs, cubic)
    with pytest.raises(ValueError, match="quadrant-basis"):
        o.strassen_matmul(a, b, bm=128, bn=128, bk=512, formula_variant="powers", epilogue="bias_add",
                          bias=np.zeros(256, np.float32))


def test_norm_residual_add_closed_form():
    """norm_residual_add (strassen_pallas.py:836-866): rms_norm over the whole
    row of the exact product, times the scale, plus the residual; one bf16
    rounding. Strassen and cubic against a float64 evaluation."""
    rng, a, b = _int_problem(420, 32, 512, 256)
    r = o.bf16_round(rng.standard_normal((32, 256)).astype(np.float32))
    g = o.bf16_round((1 + 0.1 * rng.standard_normal(256)).astype(np.float32))
    exact = (a @ b).astype(np.float64)
    expected = exact / np.sqrt(np.mean(exact ** 2, axis=1, keepdims=True) + 1e-6) * g + r
    for got in (o.strassen_matmul(a, b, bm=16, bn=256, bk=256, epilogue="norm_residual_add", residual=r,
                                  norm_scale=g),
                o.cubic_blocked_matmul(a, b, bm=16, bn=256, bk=256, epilogue="norm_residual_add", residual=r,
                                       norm_scale=g)):
        np.testing.assert_allclose(got, expected, rtol=2 ** -7, atol=2 ** -7)


# Exact panels (classical_panels / panel_schedule, strassen_pallas.py:575-586,
# :713-735): the marked K panels run the eight cubic products on raw quadrants.

@pytest.mark.parametrize("formula", ["classical", "dual"])
@pytest.mark.parametrize("perm", [0, 5, 7])
def test_exact_panels_integer_known_answer(formula, perm):
    """Small integers keep every sum exact, so any schedule returns a @ b;
    an exact product sent to the wrong quadrant or dropped fails here."""
    _, a, b = _int_problem(11, 64, 1024, 256, lo=-2, hi=3)
    for panels in ((0,), (1, 3), (0, 1, 2, 3)):
        got = o.strassen_matmul(a, b, bm=32, bn=128, bk=256, formula_variant=formula, block_permutation=perm,
                                classical_panels=panels, output_dtype="float32")
        np.testing.assert_array_equal(got, a @ b)


def test_all_exact_panels_are_the_cubic_control():
    """Every panel exact: the same eight products per panel into the same
    quadrant accumulators in the same order as the matched cubic."""
    rng = np.random.default_rng(12)
    a = o.bf16_round(rng.standard_normal((64, 1024)).astype(np.float32))
    b = o.bf16_round(rng.standard_normal((1024, 256)).astype(np.float32))
    got = o.strassen_matmul(a, b, bm=32, bn=128, bk=256, classical_panels=range(4), output_dtype="float32")
    want = o.cubic_blocked_matmul(a, b, bm=32, bn=128, bk=256, output_dtype="float32")
    np.testing.assert_array_equal(got, want)


def test_exact_panel_uses_raw_quadrants_of_its_own_panel():
    """Only panel 2 of K is nonzero. Marking panel 2 exact gives the cubic
    product of that panel bit for bit (no pre-added, rounded sums); marking
    another panel leaves the Strassen rounding of panel 2 in place."""
    rng = np.random.default_rng(13)
    a = np.zeros((64, 1024), np.float32)
    b = np.zeros((1024, 256), np.float32)
    a[:, 512:768] = o.bf16_round(rng.standard_normal((64, 256)).astype(np.float32))
    b[512:768] = o.bf16_round(rng.standard_normal((256, 256)).astype(np.float32))
    cubic = o.cubic_blocked_matmul(a, b, bm=32, bn=128, bk=256, output_dtype="float32")
    exact = o.strassen_matmul(a, b, bm=32, bn=128, bk=256, classical_panels=(2,), output_dtype="float32")
    np.testing.assert_array_equal(exact, cubic)
    other = o.strassen_matmul(a, b, bm=32, bn=128, bk=256, classical_panels=(1,), output_dtype="float32")
    plain = o.strassen_matmul(a, b, bm=32, bn=128, bk=256, output_dtype="float32")
    np.testing.assert_array_equal(other, plain)
    assert not np.array_equal(plain, cubic)


def test_panel_schedule_is_the_prefetched_form_of_classical_panels():
    a, b = (o.bf16_round(np.random.default_rng(14).standard_normal(s).astype(np.float32))
            for s in ((64, 1024), (1024, 256)))
    static = o.strassen_matmul(a, b, bm=32, bn=128, bk=256, classical_panels=(0, 3))
    prefetched = o.strassen_matmul(a, b, bm=32, bn=128, bk=256, panel_schedule=np.array([1, 0, 0, 7], np.int32))
    np.testing.assert_array_equal(static, prefetched)


# FP32 inputs (compute dtype float32): operand sums in float32, every operand
# rounded once to bf16 by the DEFAULT-precision product. The exact rounding
# of XLA's f32 dot at DEFAULT precision on the TPU is not reproducible here
# (parity unpinned); these checks pin what the semantics fix.

@pytest.mark.parametrize("formula", ["classical", "dual"])
def test_fp32_path_equals_bf16_path_on_bf16_values(formula):
    """Two bf16 values sum to the same bf16 whether the sum is rounded from
    float32 or from bf16 arithmetic, so bf16-valued inputs give identical
    results on both paths (and through the packed operands)."""
    rng = np.random.default_rng(15)
    a = o.bf16_round(rng.standard_normal((64, 1024)).astype(np.float32))
    b = o.bf16_round(rng.standard_normal((1024, 256)).astype(np.float32))
    kw = dict(bm=32, bn=128, bk=256, formula_variant=formula, block_permutation=3, output_dtype="float32")
    np.testing.assert_array_equal(o.strassen_matmul(a, b, input_dtype="float32", **kw),
                                  o.strassen_matmul(a, b, **kw))
    for side, x in (("lhs", np.zeros((256, 512), np.float32) + a[:1, :512].T[:256, :1]), ("rhs", b[:512, :256])):
        np.testing.assert_array_equal(o.packed_operand(x, 7, side, 256, 256, formula, 3, input_dtype="float32"),
                                      o.packed_operand(x, 7, side, 256, 256, formula, 3))


def test_fp32_inputs_are_a_one_pass_bf16_product():
    """Random float32 inputs: the result differs from the bf16-rounded-input
    path (sums see the unrounded float32 values) and its error against the
    float64 product sits at the one-pass bf16 level, like the bf16 path's."""
    rng = np.random.default_rng(16)
    a = rng.standard_normal((64, 1024)).astype(np.float32)
    b = rng.standard_normal((1024, 256)).astype(np.float32)
    kw = dict(bm=32, bn=128, bk=256, output_dtype="float32")
    f32 = o.strassen_matmul(a, b, input_dtype="float32", **kw)
    pre = o.strassen_matmul(o.bf16_round(a), o.bf16_round(b), **kw)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    err = np.linalg.norm(f32 - ref) / np.linalg.norm(ref)
    err_pre = np.linalg.norm(pre - ref) / np.linalg.norm(ref)
    assert not np.array_equal(f32, pre)
    assert 1e-3 < err < 1e-2 and abs(err - err_pre) < 0.25 * err_pre
    # the cubic control on FP32 inputs is the bf16-rounded-input cubic
    np.testing.assert_array_equal(o.cubic_blocked_matmul(a, b, **kw),
                                  o.cubic_blocked_matmul(o.bf16_round(a), o.bf16_round(b), **kw))


# ---------------------------------------------------------------------------
# Multi-pass FP32 products (dot_precision HIGH / HIGHEST)
# ---------------------------------------------------------------------------
# XLA's multi-pass bf16 products are not observable here (no TPU, no JAX);
# the pass pairs are those of the published bf16_3x / bf16_6x algorithms
# (parity unpinned against a TPU run). These checks pin the expansion, the
# pairs and the accuracy each precision must reach.

def test_bf16_parts_reconstruct_float32_exactly():
    """p0 + p1 + p2 == x for normal float32 x (24 bits in three 8-bit parts
    with signed remainders), and each part is a bf16 value below half an
    ulp of the previous one."""
    rng = np.random.default_rng(17)
    x = (rng.standard_normal(20000) * np.exp2(rng.integers(-60, 60, 20000))).astype(np.float32)
    p0, p1, p2 = (o.bf16_part(x, i) for i in range(3))
    for p in (p0, p1, p2):
        np.testing.assert_array_equal(p, o.bf16_round(p))
    np.testing.assert_array_equal(p0.astype(np.float64) + p1 + p2, x.astype(np.float64))
    assert np.all(np.abs(p1) <= np.abs(p0) * 2.0 ** -8) and np.all(np.abs(p2) <= np.abs(p1) * 2.0 ** -8)
    # two parts do not suffice: the third carries information
    assert np.mean(p0.astype(np.float64) + p1 != x) > 0.5
    np.testing.assert_array_equal(o.bf16_part(x, 0), o.bf16_round(x))


def test_pass_product_known_answers():
    """s = 1 + 2^-10 + 2^-20 (parts 1, 2^-10, 2^-20), t = 3 + 2^-9 (parts 3,
    2^-9, 0): each precision keeps exactly its pass pairs, so a wrong or
    missing pair changes the sum. Every partial sum is exact in float32."""
    s = np.array([[1 + 2.0 ** -10 + 2.0 ** -20]], np.float32)
    t = np.array([[3 + 2.0 ** -9]], np.float32)
    s_parts, t_parts = (1.0, 2.0 ** -10, 2.0 ** -20), (3.0, 2.0 ** -9, 0.0)
    for i, (ps, pt) in enumerate(zip(s_parts, t_parts)):
        assert o.bf16_part(s, i)[0, 0] == ps and o.bf16_part(t, i)[0, 0] == pt
    want = {1: 3.0,
            3: 3.0 + 2.0 ** -9 + 3 * 2.0 ** -10,
            6: 3.0 + 2.0 ** -9 + 3 * 2.0 ** -10 + 2.0 ** -19 + 3 * 2.0 ** -20}
    for passes, value in want.items():
        assert o.pass_product(s, t, passes)[0, 0] == np.float32(value), passes
    # the pairs are not symmetric in the parts: swapping the operands keeps the
    # value only because each pass set is closed under swapping A and B
    for passes in (1, 3, 6):
        assert o.pass_product(t.T, s.T, passes)[0, 0] == o.pass_product(s, t, passes)[0, 0]
    assert [o.precision_passes(p) for p in (None, "default", "bfloat16", "high", "tensorfloat32", "highest",
                                            "float32")] == [1, 1, 1, 3, 3, 6, 6]
    assert o.precision_passes("highest", "bfloat16") == 1
    with pytest.raises(ValueError, match="unknown dot_precision"):
        o.precision_passes("fp64")


@pytest.mark.parametrize("formula", ["classical", "dual", "powers"])
def test_multi_pass_accuracy_ladder(formula):
    """Against the float64 product: DEFAULT is at the bf16 level, HIGH drops
    only second-order parts (about 2^-16), HIGHEST only third-order ones, so
    it reaches the FP32 accumulation level. The cubic control climbs the
    same ladder."""
    rng = np.random.default_rng(18)
    a = rng.standard_normal((64, 1024)).astype(np.float32)
    b = rng.standard_normal((1024, 256)).astype(np.float32)
    ref64 = a.astype(np.float64) @ b.astype(np.float64)
    kw = dict(bm=32, bn=128, bk=256, output_dtype="float32", input_dtype="float32", formula_variant=formula)
    err = {}
    for precision in ("default", "high", "highest"):
        got = o.strassen_matmul(a, b, dot_precision=precision, **kw)
        err[precision] = np.linalg.norm(got - ref64) / np.linalg.norm(ref64)
        cubic = o.cubic_blocked_matmul(a, b, bm=32, bn=128, bk=256, output_dtype="float32", dot_precision=precision)
        err["cubic_" + precision] = np.linalg.norm(cubic - ref64) / np.linalg.norm(ref64)
    # measured: DEFAULT ~4.7e-3, HIGH ~8.7e-6, HIGHEST ~2.1e-7 (the cubic half of each)
    assert 1e-3 < err["default"] < 1e-2
    assert 2e-6 < err["high"] < 3e-5
    assert err["highest"] < 1e-6 and err["highest"] < err["high"] / 10
    assert err["cubic_highest"] < 1e-6 < err["cubic_high"] < 1e-4 < err["cubic_default"]
    # bf16 inputs take one pass whatever dot_precision says
    a16, b16 = o.bf16_round(a), o.bf16_round(b)
    kw16 = dict(kw, input_dtype="bfloat16")
    np.testing.assert_array_equal(o.strassen_matmul(a16, b16, dot_precision="highest", **kw16),
                                  o.strassen_matmul(a16, b16, **kw16))


def test_multi_pass_packed_planes():
    """Packed depth runs (pass, K panel, local k): pass i of every panel
    holds the operand's bf16 part PASS_PARTS[passes][side][i], HIGH's passes
    are HIGHEST's last three, and the three distinct parts of a HIGHEST
    operand sum to the float32 operand sums recomputed from the quadrants."""
    rng = np.random.default_rng(19)
    hk, npanels = 256, 2
    for side, x in (("lhs", rng.standard_normal((256, 1024)).astype(np.float32)),
                    ("rhs", rng.standard_normal((1024, 256)).astype(np.float32))):
        one = o.operand_planes(x, 7, side, 256, 512, input_dtype="float32")
        three = o.operand_planes(x, 7, side, 256, 512, input_dtype="float32", dot_precision="high")
        six = o.operand_planes(x, 7, side, 256, 512, input_dtype="float32", dot_precision="highest")
        width = npanels * hk
        assert three.shape[2] == 3 * width and six.shape[2] == 6 * width
        np.testing.assert_array_equal(three, six[:, :, 3 * width:])
        np.testing.assert_array_equal(six[:, :, 5 * width:], one)  # the leading pass comes last
        if side == "lhs":
            q = [np.concatenate(c, axis=1) for c in zip(*(ref._split_a(x, 256, 512, s) for s in range(npanels)))]
            ops = np.stack(o.strassen_a_operands(q, ref._identity))
        else:
            q = [np.concatenate(c, axis=0).T for c in zip(*(ref._split_b(x, 256, 512, s) for s in range(npanels)))]
            ops = np.stack(o.strassen_b_operands(q, ref._identity))
        parts = o.PASS_PARTS[6][0 if side == "lhs" else 1]
        for i, part in enumerate(parts):
            np.testing.assert_array_equal(six[:, :, i * width:(i + 1) * width], o.bf16_part(ops, part))
        first = {part: i for i, part in reversed(list(enumerate(parts)))}
        total = sum(six[:, :, first[p] * width:(first[p] + 1) * width].astype(np.float64) for p in range(3))
        np.testing.assert_array_equal(total, ops.astype(np.float64))


def test_torch_cpu_restatement_integer_known_answer():
    """The torch-CPU restatement (the bench's CPU baseline) reproduces A @ B
    bit for bit on small-integer operands, where every bf16 operand sum and
    FP32 product is exact (the technique of the reference's
    Strassen_MM_Focus/tests/test_kernels_v001.py:59-80)."""
    import torch

    from oracle import strassen_torch_cpu as tc

    rng = np.random.default_rng(187)
    for (m, k, n), (bm, bn, bk) in (((256, 512, 256), (256, 256, 512)), ((512, 1024, 256), (256, 128, 256))):
        a = rng.integers(-3, 4, (m, k)).astype(np.float32)
        b = rng.integers(-3, 4, (k, n)).astype(np.float32)
        got = tc.strassen_matmul(torch.from_numpy(a), torch.from_numpy(b), bm=bm, bn=bn, bk=bk)
        assert np.array_equal(got.float().numpy(), o.bf16_round(a @ b))
        # a planted sign error in one update fails the known answer
        saved = tc.PRODUCT_UPDATES[5]
        try:
            tc.PRODUCT_UPDATES[5] = ((0, +1), (1, +1))
            bad = tc.strassen_matmul(torch.from_numpy(a), torch.from_numpy(b), bm=bm, bn=bn, bk=bk)
            assert not np.array_equal(bad.float().numpy(), o.bf16_round(a @ b))
        finally:
            tc.PRODUCT_UPDATES[5] = saved


def test_torch_cpu_restatement_matches_numpy_oracle():
    """Random bf16 inputs at the 1024^3 seed-0 configuration: the torch-CPU
    restatement and the numpy oracle round the same operand sums and add the
    same products in the same order; only the BLAS libraries' FP32 summation
    inside each product differs, so results agree to one bf16 ulp on all but
    a few elements and the accuracy against FP32 is the same."""
    import torch

    from oracle import strassen_torch_cpu as tc

    rng = np.random.default_rng(0)
    a = o.bf16_round(rng.standard_normal((1024, 1024)).astype(np.float32))
    b = o.bf16_round((rng.standard_normal((1024, 1024)) / 32).astype(np.float32))
    want = o.strassen_matmul(a, b, bm=1024, bn=1024, bk=512, interleave_products=True)
    got = tc.strassen_matmul(torch.from_numpy(a), torch.from_numpy(b), bm=1024, bn=1024, bk=512).float().numpy()
    ulp = np.abs(want) * 2.0 ** -7 + 1e-6
    assert np.all(np.abs(got - want) <= ulp)
    assert np.mean(got != want) < 0.02
    ref = a.astype(np.float64) @ b.astype(np.float64)
    e_got = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    e_want = np.linalg.norm(want - ref) / np.linalg.norm(ref)
    assert abs(e_got - e_want) < 0.02 * e_want


# ---------------------------------------------------------------------------
# Closed-form pins of the unfused RMSNorm / RoPE helpers
# (benchmark_qwen3_32b_layer.py:258-284), independent of the block's copies.
# ---------------------------------------------------------------------------

def test_rope_values_closed_form():
    """cos / sin [p, i] = cos / sin(p theta^(-2 (i mod D/2) / D)), both halves
    equal, position 0 the identity; the float32 angle computation and the one
    bf16 rounding stay within one bf16 ulp of the float64 value."""
    seq, hd, theta = 64, 128, 1e6
    cos, sin = o.rope_values(seq, hd, theta)
    i = np.arange(hd) % (hd // 2)
    angles = np.arange(seq, dtype=np.float64)[:, None] * theta ** (-2.0 * i[None, :] / hd)
    for got, want in ((cos, np.cos(angles)), (sin, np.sin(angles))):
        assert got.shape == (seq, hd)
        assert np.array_equal(got[:, : hd // 2], got[:, hd // 2:])
        assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.maximum(np.abs(want), 2.0 ** -8) + 1e-7)
    assert np.array_equal(cos[0], np.ones(hd)) and np.array_equal(sin[0], np.zeros(hd))
    # a planted mistake (the inverse frequency over D/2 instead of D) fails it
    wrong = np.cos(np.arange(seq, dtype=np.float64)[:, None] * theta ** (-2.0 * i[None, :] / (hd // 2)))
    assert np.max(np.abs(cos - wrong)) > 0.5


def test_apply_rope_closed_forms():
    """Position 0 is the identity; a basis vector e_i (i < D/2) maps to
    cos e_i + sin e_{i+D/2} and e_{i+D/2} to -sin e_i + cos e_{i+D/2} (the
    reference's x cos + concat(-x2, x1) sin); each (i, i + D/2) pair keeps
    its norm; rotating by p then by q is rotating by p + q (float64 tables,
    so only the bf16 output rounding remains)."""
    rng = np.random.default_rng(41)
    hd, seq = 128, 8
    x = o.bf16_round(rng.standard_normal((1, seq, 2, hd)).astype(np.float32))
    cos, sin = o.rope_values(seq, hd, 1e6)
    assert np.array_equal(o.apply_rope(x[:, :1], cos[:1], sin[:1]), x[:, :1])
    angle = 0.75
    c = np.full((1, hd), np.cos(angle), np.float32)
    s = np.full((1, hd), np.sin(angle), np.float32)
    for i in (0, 5, hd // 2 - 1):
        e = np.zeros((1, 1, 1, hd), np.float32)
        e[..., i] = 1.0
        out = o.apply_rope(e, c, s)[0, 0, 0]
        want = np.zeros(hd, np.float32)
        want[i], want[i + hd // 2] = np.cos(angle), np.sin(angle)
        assert np.allclose(out, o.bf16_round(want), atol=0), i
        e2 = np.zeros((1, 1, 1, hd), np.float32)
        e2[..., i + hd // 2] = 1.0
        out2 = o.apply_rope(e2, c, s)[0, 0, 0]
        want2 = np.zeros(hd, np.float32)
        want2[i], want2[i + hd // 2] = -np.sin(angle), np.cos(angle)
        assert np.allclose(out2, o.bf16_round(want2), atol=0), i
    # norm of each pair, and composition, with exact (float64-derived) tables
    p, q = 3.0, 11.0
    freq = 1e6 ** (-2.0 * (np.arange(hd) % (hd // 2)) / hd)
    tables = {a: (np.cos(a * freq)[None].astype(np.float32), np.sin(a * freq)[None].astype(np.float32))
              for a in (p, q, p + q)}
    y = x[:, :1]
    once = o.apply_rope(y, *tables[p])
    pair = lambda v: v[..., : hd // 2] ** 2 + v[..., hd // 2:] ** 2  # noqa: E731
    assert np.allclose(pair(once), pair(y), rtol=2 ** -6, atol=1e-3)
    twice = o.apply_rope(once, *tables[q])
    direct = o.apply_rope(y, *tables[p + q])
    assert np.allclose(twice, direct, rtol=2 ** -6, atol=2 ** -6)


def test_rms_norm_closed_forms():
    """Under unit gamma a normalised row has unit RMS (to bf16 rounding);
    gamma scales the output elementwise; with eps = 0 the map is invariant
    to scaling a row by a power of two (every step scales exactly); a
    constant row maps to +-1."""
    rng = np.random.default_rng(42)
    x = o.bf16_round(rng.standard_normal((16, 512)).astype(np.float32) * 3.0)
    y = o.rms_norm(x, np.ones(512, np.float32), 1e-6)
    rms = np.sqrt(np.mean(y.astype(np.float64) ** 2, axis=-1))
    assert np.all(np.abs(rms - 1.0) < 2 ** -8)
    g = o.bf16_round((1 + 0.1 * rng.standard_normal(512)).astype(np.float32))
    unscaled = o.rms_norm(x, np.ones(512, np.float32), 0.0)
    assert np.allclose(o.rms_norm(x, g, 0.0), o.bf16_round(unscaled * g), rtol=2 ** -7, atol=0)
    assert np.array_equal(o.rms_norm(4.0 * x, g, 0.0), o.rms_norm(x, g, 0.0))
    const = np.full((2, 64), -2.5, np.float32)
    assert np.array_equal(o.rms_norm(const, np.ones(64, np.float32), 0.0), -np.ones((2, 64), np.float32))


# SHA-256 of the reference's real-weight test tensors, from its manifest
# (Strassen_MM_Focus/data/qwen3-0.6b-real-v001/manifest.json, "tensors" list).
REAL_WEIGHT_SHA256 = {
    "q_proj": "7592f6e783c400f502653f77d9b483cb03e96c3061af16f538da0d695d21bc53",
    "down_proj": "01cc5c354c8ac9cf4917157d74beceb0b3ce3f38d9bdec271ae691bded0b2e3b",
}


@pytest.mark.parametrize("name,shape", [("q_proj", (256, 512)), ("down_proj", (256, 1024))])
def test_real_weight_slices(name, shape):
    """The committed slices come from the manifest-checked reference tensors
    (tests/golden/make_golden.py) and hold finite, weight-sized bf16 values;
    the oracle's Strassen product on them lands in the reference's published
    error band against FP32 (a few 1e-3, strassen_v5e_classical_comparison.jsonl:3)."""
    data = np.load(os.path.join(GOLDEN, f"qwen3_0p6b_{name}_slice.npz"))
    assert str(data["source_sha256"]) == REAL_WEIGHT_SHA256[name]
    assert str(data["source"]).endswith(f"layer0_{name}.bf16[:{shape[0]}, :{shape[1]}]")
    bits = data["weight_bits"]
    assert bits.shape == shape and bits.dtype == np.uint16
    w = o.bits_to_f32(bits)
    assert np.isfinite(w).all() and 1e-3 < float(np.std(w)) < 0.2
    b = np.ascontiguousarray(w.T)  # [K, N]
    rng = np.random.default_rng(77)
    a = o.bf16_round(rng.standard_normal((256, b.shape[0])).astype(np.float32))
    ref = o.high_precision_reference(a, b).astype(np.float64)
    got = o.strassen_matmul(a, b, bm=256, bn=256, bk=256)
    err = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    assert 1e-3 < err < 1e-2
