"""GPU parity of the gfx950 Strassen / cubic kernels against the CPU oracle.

Bars:
* exact-integer operands: bit-exact equality with A @ B (rounded once to bf16);
* random bf16 operands: the same bf16 operand sums as the oracle, so outputs
  agree to within one bf16 ulp everywhere (FP32 summation order differs), with
  at most a small fraction of elements not bit-identical;
* against the FP32 product: relative Frobenius error <= 1e-2 and <= 1.5x the
  oracle Strassen's own error on the same inputs;
* full Qwen3-32B shapes: sampled (bm, bn) output tiles recomputed by the
  oracle (a Strassen tile depends only on its own A rows and B columns), plus
  the whole-output error bound against an FP32 product.
"""

import ctypes
import json
import os

import numpy as np
import pytest
import torch

import oracle as o
import strassen_tpu_amd as smx

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DEV = torch.device("cuda:0")


def say(*args):
    print(*args, flush=True)


def dev(x):
    """float32 numpy (bf16 values) -> bf16 device tensor."""
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(DEV).to(torch.bfloat16)


def dev_weight(b):
    """[K, N] numpy -> K-contiguous [K, N] bf16 device view of [N, K] storage."""
    return dev(np.ascontiguousarray(np.asarray(b, np.float32).T)).t()


def host(t):
    return t.float().cpu().numpy()


def bf16_ulp(v):
    bits = np.abs(np.asarray(v, np.float32)).view(np.uint32)
    exponent = ((bits >> 23) & 0xFF).astype(np.int32)
    exponent = np.maximum(exponent, 1)
    return np.ldexp(np.float32(1.0), exponent - 127 - 7).astype(np.float32)


def fp32_floor(want, k):
    """Absolute FP32 summation-error allowance for outputs near zero.

    The kernel and the oracle sum the same bf16 products in different FP32
    orders; the kernel keeps seven product accumulators over K/2 terms and
    combines them at the end, so its absolute error grows like
    eps_f32 * sqrt(K) * |output scale|. Elements much smaller than that scale
    can then differ by several of their own (tiny) bf16 ulps. The allowance
    8 * 2^-24 * sqrt(K) * rms(want) stays far below one bf16 ulp at typical
    magnitudes, so algebra or rounding mistakes still fail.
    """
    rms = float(np.sqrt(np.mean(np.asarray(want, np.float64) ** 2)))
    return 8.0 * 2.0 ** -24 * np.sqrt(k) * rms


def assert_ulp_close(got, want, *, k, max_mismatch_frac=0.02):
    """|got - want| <= 1 bf16 ulp of want (or the FP32 summation allowance
    near zero), and most elements bit-identical."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape
    assert np.isfinite(got).all()
    floor = fp32_floor(want, k)
    diff = np.abs(got - want)
    bad = diff > np.maximum(bf16_ulp(want), floor)
    assert not bad.any(), (
        f"{int(bad.sum())} elements beyond 1 ulp; worst {float(diff.max())} at "
        f"{np.unravel_index(int(np.argmax(diff)), diff.shape)}")
    frac = float(np.mean(diff > 0))
    assert frac <= max_mismatch_frac, f"{frac:.4f} of elements differ"


def rel_l2(got, ref):
    return float(np.linalg.norm(np.asarray(got, np.float64) - ref) / np.linalg.norm(ref))


# The four kernels behind the surface: Strassen and the cubic control with a
# plain weight on the compact kernel (operand sums / quadrants read from
# row-major A and B^T), and both with packed operands (the packed kernel:
# weight packed offline, activation packed per call). A plain weight whose
# tile suits the packed kernel is otherwise packed per call; the plain arms
# select the compact kernel explicitly.
ARMS = ("strassen_plain", "strassen_packed", "cubic_plain", "cubic_packed")


def run_arm(arm, a, b, *, bm, bn, bk, **kw):
    """a: [M, K] numpy or device tensor; b: [K, N] numpy or K-contiguous
    device tensor. Returns the device result."""
    say(f"  arm {arm} tile=({bm},{bn},{bk}) epilogue={kw.get('epilogue')}")
    a_dev = a if torch.is_tensor(a) else dev(a)
    b_dev = b if torch.is_tensor(b) else dev_weight(b)
    if arm.endswith("plain"):
        with smx.plain_weight_kernel("compact"):
            return _run_arm(arm, a_dev, b_dev, bm=bm, bn=bn, bk=bk, **kw)
    return _run_arm(arm, a_dev, b_dev, bm=bm, bn=bn, bk=bk, **kw)


def _run_arm(arm, a_dev, b_dev, *, bm, bn, bk, **kw):
    if arm == "strassen_plain":
        return smx.strassen_matmul(a_dev, b_dev, bm=bm, bn=bn, bk=bk, **kw)
    if arm == "strassen_packed":
        w = smx.strassen_weight_layout(b_dev, bn, bk, dot_precision=kw.get("dot_precision"))
        return smx.strassen_matmul(a_dev, w, bm=bm, bn=bn, bk=bk, **kw)
    kw.pop("interleave_products", None)
    kw.pop("product_aware_swiglu", None)
    kw.pop("product_aware_residual", None)
    if arm == "cubic_packed":
        b_dev = smx.cubic_weight_layout(b_dev, bn, bk, dot_precision=kw.get("dot_precision"))
    return smx.cubic_matmul(a_dev, b_dev, bm=bm, bn=bn, bk=bk, **kw)


def oracle_arm(arm, a, b, **kw):
    if arm.startswith("strassen"):
        return o.strassen_matmul(a, b, **kw)
    for key in ("interleave_products", "product_aware_swiglu", "product_aware_residual"):
        kw.pop(key, None)
    return o.cubic_blocked_matmul(a, b, **kw)


@pytest.fixture(autouse=True)
def _announce(request):
    say(f"\n[gpu] {request.node.nodeid}")
    yield
    torch.cuda.synchronize()


# ---------------------------------------------------------------------------
# Exact-integer known answers
# ---------------------------------------------------------------------------

INT_CASES = [
    ((256, 512, 256), (256, 256, 512)),
    ((512, 1024, 512), (256, 256, 256)),
    ((1024, 2048, 768), (512, 256, 512)),
    # the fewest K stages the surface allows (bk % 256): 8 stages of 32
    ((512, 256, 512), (256, 256, 256)),
]


@pytest.mark.parametrize("k", [64, 128, 192])
@pytest.mark.parametrize("algo", [7, 8])
def test_short_k_ring_through_c_abi(k, algo):
    """2, 4 and 6 K stages (bk = 64, which the C ABI accepts and the surface's
    TPU rule does not): the stage ring's prologue and the prefetches past the
    last stage, which re-load it and are never read. Integer operands, so the
    bf16 output equals the exact product rounded once."""
    from strassen_tpu_amd import _lib

    m, n, bm, bn, bk = 512, 512, 256, 256, 64
    rng = np.random.default_rng(511 + k)
    a = rng.integers(-2, 3, (m, k)).astype(np.float32)
    b = rng.integers(-2, 3, (k, n)).astype(np.float32)
    say(f"  algo={algo} shape={(m, k, n)} tile={(bm, bn, bk)}")
    pa = smx.pack_activation(dev(a), algo, bm, bk)
    pb = (smx.strassen_weight_layout if algo == 7 else smx.cubic_weight_layout)(dev_weight(b), bn, bk)
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    d = _lib.SmxGemmDesc()
    d.m, d.n, d.k = m, n, k
    d.lda, d.ldb, d.ldc, d.ldr = k, k, n, 0
    d.bm, d.bn, d.bk = bm, bn, bk
    d.algo, d.epilogue = algo, _lib.SMX_EPI[None]
    d.a_layout, d.b_layout = _lib.SMX_A_PACKED, _lib.SMX_B_PACKED
    d.rope_head_dim, d.rope_eps = 128, 1e-6
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(_lib.load().smx_gemm(d, _lib.ptr(pa.data), _lib.ptr(pb.data), _lib.ptr(out), None, None, None, None,
                                    None, ctypes.c_void_p(stream)))
    want = o.bf16_round((a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32))
    np.testing.assert_array_equal(host(out), want)


@pytest.mark.parametrize("shape,tile", INT_CASES)
@pytest.mark.parametrize("arm", ARMS)
def test_integer_kat_bit_exact(shape, tile, arm):
    m, k, n = shape
    bm, bn, bk = tile
    rng = np.random.default_rng(187)
    a = rng.integers(-2, 3, (m, k)).astype(np.float32)
    b = rng.integers(-2, 3, (k, n)).astype(np.float32)
    say(f"  {arm} shape={shape} tile={tile}")
    got = host(run_arm(arm, a, b, bm=bm, bn=bn, bk=bk))
    assert np.array_equal(got, o.bf16_round(a @ b))


@pytest.mark.parametrize("algo", [7, 8])
def test_pack_kernel_matches_oracle(algo):
    rng = np.random.default_rng(5)
    # (rows x K of the operand, tile_rows, bk): several tiles and K panels,
    # and a K panel wider than one pack wave's four stages.
    for (rows, k), (tile, bk) in (((1024, 1024), (512, 512)), ((512, 768), (256, 256)),
                                  ((768, 4160), (256, 320))):
        say(f"  algo={algo} rows={rows} k={k} tile={tile} bk={bk}")
        a = o.bf16_round(rng.standard_normal((rows, k)).astype(np.float32))
        got = smx.pack_activation(dev(a), algo, tile, bk)
        assert np.array_equal(host(got.data), o.packed_operand(a, algo, "lhs", tile, bk))
        b = o.bf16_round(rng.standard_normal((k, rows)).astype(np.float32))
        w = smx.pack_operand(dev_weight(b), algo=algo, side="rhs", tile_rows=tile, bk=bk)
        assert np.array_equal(host(w.data), o.packed_operand(b, algo, "rhs", tile, bk))
        # a row-major weight gives the same packing
        w2 = smx.pack_operand(dev(b), algo=algo, side="rhs", tile_rows=tile, bk=bk)
        assert torch.equal(w.data, w2.data)
    with pytest.raises(ValueError, match="does not tile"):
        smx.strassen_weight_layout(dev(np.zeros((500, 256), np.float32)), 256, 512)


def test_integer_kat_row_major_weight():
    """A row-major [K, N] weight is transposed by the surface and gives the
    same exact answer."""
    rng = np.random.default_rng(190)
    a = rng.integers(-2, 3, (256, 512)).astype(np.float32)
    b = rng.integers(-2, 3, (512, 256)).astype(np.float32)
    got = host(smx.strassen_matmul(dev(a), dev(b), bm=256, bn=256, bk=512))
    assert np.array_equal(got, o.bf16_round(a @ b))


# ---------------------------------------------------------------------------
# Random bf16 operands vs the oracle
# ---------------------------------------------------------------------------

def _gaussian(seed, m, k, n, a_std=1.0, b_std=0.02):
    rng = np.random.default_rng(seed)
    a = o.bf16_round(rng.standard_normal((m, k)).astype(np.float32) * np.float32(a_std))
    b = o.bf16_round(rng.standard_normal((k, n)).astype(np.float32) * np.float32(b_std))
    return rng, a, b


def test_config1_1024_cube_seed0():
    """A[1024,1024] ~ N(0,1), B ~ N(0, 1/32), seed 0, reference default tile
    (1024, 1024, 512), bf16 out, vs FP32 cubic."""
    gen = torch.Generator().manual_seed(0)
    a = o.bf16_round(torch.randn(1024, 1024, generator=gen).numpy())
    b = o.bf16_round((torch.randn(1024, 1024, generator=gen) / 32).numpy())
    ref = o.high_precision_reference(a, b).astype(np.float64)
    for arm in ARMS:
        kw = dict(bm=1024, bn=1024, bk=512, interleave_products=True)
        want = oracle_arm(arm, a, b, **kw)
        got = host(run_arm(arm, a, b, **kw))
        assert_ulp_close(got, want, k=1024)
        e_got, e_want = rel_l2(got, ref), rel_l2(want, ref)
        say(f"  {arm} rel err gpu={e_got:.4e} oracle={e_want:.4e}")
        assert e_got <= 1e-2 and e_got <= 1.5 * e_want


@pytest.mark.parametrize("shape,tile", [
    ((512, 2048, 1024), (256, 256, 512)),
    ((768, 1536, 512), (256, 512, 256)),
])
def test_random_matches_oracle(shape, tile):
    m, k, n = shape
    _, a, b = _gaussian(42, m, k, n)
    bm, bn, bk = tile
    for arm in ARMS:
        got = host(run_arm(arm, a, b, bm=bm, bn=bn, bk=bk))
        assert_ulp_close(got, oracle_arm(arm, a, b, bm=bm, bn=bn, bk=bk), k=k)


def test_repeated_calls_reset_accumulators():
    _, a, b = _gaussian(3, 256, 1024, 256)
    for arm in ARMS:
        first = host(run_arm(arm, a, b, bm=256, bn=256, bk=512))
        second = host(run_arm(arm, -a, b, bm=256, bn=256, bk=512))
        assert_ulp_close(first, oracle_arm(arm, a, b, bm=256, bn=256, bk=512), k=1024)
        assert_ulp_close(second, oracle_arm(arm, -a, b, bm=256, bn=256, bk=512), k=1024)


def test_real_qwen3_weight_slice():
    """Real Qwen3-0.6B layer-0 q_proj weights (reference test data) as B."""
    data = np.load(os.path.join(GOLDEN, "qwen3_0p6b_q_proj_slice.npz"))
    w_bits = data["weight_bits"]  # [out=256, in=512] bf16 bits
    w = o.bits_to_f32(w_bits)     # [N, K]
    b = np.ascontiguousarray(w.T)  # [K, N]
    rng = np.random.default_rng(2026)
    a = o.bf16_round(rng.standard_normal((256, 512)).astype(np.float32))
    b_dev = torch.from_numpy(w_bits.view(np.int16)).view(torch.bfloat16).to(DEV).t()
    ref = o.high_precision_reference(a, b).astype(np.float64)
    for arm in ARMS:
        got = host(run_arm(arm, a, b_dev, bm=256, bn=256, bk=256))
        want = oracle_arm(arm, a, b, bm=256, bn=256, bk=256)
        assert_ulp_close(got, want, k=512)
        assert rel_l2(got, ref) <= 1.5 * max(rel_l2(want, ref), 1e-4)


def test_real_qwen3_down_proj_slice_residual_add():
    """Real Qwen3-0.6B layer-0 down_proj weights (a [256 out, 1024 in] slice
    of the reference's test data, SHA-checked when the fixture was written)
    as B of the residual_add site: H [512, 1024] SwiGLU-sized activations
    (silu(g) u of unit normals) and a unit-normal residual, every arm within
    one bf16 ulp of the oracle and within 1.5x the oracle's error against
    FP32."""
    data = np.load(os.path.join(GOLDEN, "qwen3_0p6b_down_proj_slice.npz"))
    w_bits = data["weight_bits"]  # [out=256, in=1024]
    w = o.bits_to_f32(w_bits)
    b = np.ascontiguousarray(w.T)  # [K=1024, N=256]
    rng = np.random.default_rng(2027)
    g, u = rng.standard_normal((2, 512, 1024)).astype(np.float32)
    h = o.bf16_round(g / (1.0 + np.exp(-g)) * u)
    r = o.bf16_round(rng.standard_normal((512, 256)).astype(np.float32))
    b_dev = torch.from_numpy(w_bits.view(np.int16)).view(torch.bfloat16).to(DEV).t()
    ref = (o.high_precision_reference(h, b) + r).astype(np.float64)
    kw = dict(bm=256, bn=256, bk=512, epilogue="residual_add")
    for arm in ARMS:
        got = host(run_arm(arm, h, b_dev, residual=dev(r), **kw))
        want = oracle_arm(arm, h, b, residual=r, **kw)
        assert_ulp_close(got, want, k=1024)
        assert rel_l2(got, ref) <= 1.5 * max(rel_l2(want, ref), 1e-4), arm


@pytest.mark.slow
def test_published_accuracy_gate_on_gpu():
    """The reference's accuracy gate, regenerated: Strassen error vs FP32 on
    the GPU matches the published TPU value (4.6988e-3) and the oracle."""
    spec = json.load(open(os.path.join(GOLDEN, "accuracy_gate_reference.json")))
    a, b = o.host_uniform_inputs(tuple(spec["shape_mkn"]), spec["seed"])
    bm, bn, bk = spec["tile_bm_bn_bk"]
    ref_t = torch.matmul(dev(a).float(), dev(b).float())  # FP32 product on the GPU
    published = spec["errors_vs_reference"]
    for arm in ARMS:
        got = run_arm(arm, dev(a), dev_weight(b), bm=bm, bn=bn, bk=bk).float()
        err = float(torch.linalg.norm(got - ref_t) / torch.linalg.norm(ref_t))
        want = published["strassen" if arm.startswith("strassen") else "cubic_blocked"]["l2_relative"]
        say(f"  {arm} {err:.6e} (published {want:.6e})")
        assert err == pytest.approx(want, rel=5e-3)
        assert err <= 1.5 * want


# ---------------------------------------------------------------------------
# Epilogues
# ---------------------------------------------------------------------------

def test_swiglu_epilogue():
    _, a, b = _gaussian(318, 512, 1024, 2048)
    bm, bn, bk = 256, 512, 512
    laid = o.swiglu_weight_layout(b, bn)
    laid_dev = smx.swiglu_weight_layout(dev_weight(b), bn)
    assert np.array_equal(host(laid_dev), laid)
    for arm in ARMS:
        got = host(run_arm(arm, a, laid_dev, bm=bm, bn=bn, bk=bk, epilogue="swiglu"))
        assert got.shape == (512, 1024)
        assert_ulp_close(got, oracle_arm(arm, a, laid, bm=bm, bn=bn, bk=bk, epilogue="swiglu"), k=1024)
    # product-aware flag is accepted and selects the same kernel
    got = host(smx.strassen_matmul(dev(a), laid_dev, bm=bm, bn=bn, bk=bk, epilogue="swiglu",
                                   interleave_products=True, product_aware_swiglu=True))
    assert_ulp_close(got, o.strassen_matmul(a, laid, bm=bm, bn=bn, bk=bk, epilogue="swiglu",
                                            interleave_products=True, product_aware_swiglu=True), k=1024)


def test_geglu_epilogue():
    _, a, b = _gaussian(330, 512, 1024, 2048)
    bm, bn, bk = 256, 512, 512
    laid = o.swiglu_weight_layout(b, bn)
    laid_dev = smx.swiglu_weight_layout(dev_weight(b), bn)
    for arm in ARMS:
        got = host(run_arm(arm, a, laid_dev, bm=bm, bn=bn, bk=bk, epilogue="geglu"))
        assert got.shape == (512, 1024)
        assert_ulp_close(got, oracle_arm(arm, a, laid, bm=bm, bn=bn, bk=bk, epilogue="geglu"), k=1024)


def test_fp32_output():
    """output_dtype=float32: the unrounded FP32 quadrant values (the
    reference's output-as-accumulator path, strassen_pallas.py:1048-1057; the
    reference allows it only without a fused epilogue)."""
    _, a, b = _gaussian(331, 512, 1024, 1024)
    kw = dict(bm=256, bn=512, bk=512)
    for arm in ARMS:
        got_t = run_arm(arm, a, b, output_dtype=torch.float32, **kw)
        assert got_t.dtype == torch.float32
        got = host(got_t)
        want = oracle_arm(arm, a, b, output_dtype="float32", **kw)
        # FP32 summation order differs: a few FP32 ulps plus the near-zero floor.
        tol = 4 * np.abs(want) * 2.0 ** -23 + fp32_floor(want, 1024)
        assert np.all(np.abs(got - want) <= tol), arm
        # rounding it gives the kernel's bf16 result (same FP32 values)
        bf = host(run_arm(arm, a, b, **kw))
        assert np.array_equal(bf, o.bf16_round(got)), arm
    with pytest.raises(ValueError, match="BF16 output tile"):
        smx.strassen_matmul(dev(a), dev_weight(b), epilogue="residual_add", residual=dev(a[:, :1024]),
                            output_dtype=torch.float32, **kw)


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_lhs_transposed(out_dtype):
    """a stored [K, M]: the transposed pack reads it in place; the product
    equals the oracle's Strassen of a.T (strassen_pallas.py:1224-1312)."""
    rng = np.random.default_rng(332)
    k, m, n = 1024, 512, 768
    a_t = o.bf16_round(rng.standard_normal((k, m)).astype(np.float32))
    b = o.bf16_round(rng.standard_normal((k, n)).astype(np.float32) * np.float32(0.02))
    packed = smx.pack_operand(dev(a_t), algo=7, side="lhs_t", tile_rows=256, bk=512)
    assert np.array_equal(host(packed.data), o.packed_operand(a_t.T, 7, "lhs", 256, 512))
    got = smx.strassen_matmul_lhs_transposed(dev(a_t), dev(b), bm=256, bn=256, bk=512, output_dtype=out_dtype)
    assert got.dtype == out_dtype and tuple(got.shape) == (m, n)
    want = o.strassen_matmul_lhs_transposed(a_t, b, bm=256, bn=256, bk=512,
                                            output_dtype="float32" if out_dtype == torch.float32 else "bfloat16")
    if out_dtype == torch.bfloat16:
        assert_ulp_close(host(got), want, k=k)
    else:
        tol = 4 * np.abs(want) * 2.0 ** -23 + fp32_floor(want, k)
        assert np.all(np.abs(host(got) - want) <= tol)
    # integer data: exactly a.T @ b
    ai = rng.integers(-2, 3, (k, m)).astype(np.float32)
    bi = rng.integers(-2, 3, (k, n)).astype(np.float32)
    got = host(smx.strassen_matmul_lhs_transposed(dev(ai), dev(bi), bm=256, bn=256, bk=512))
    assert np.array_equal(got, o.bf16_round(ai.T @ bi))


VARIANTS = [("classical", 5), ("dual", 0), ("dual", 3), ("powers", 0), ("powers", 6)]


@pytest.mark.parametrize("formula,perm", VARIANTS)
def test_formula_variant_pack_matches_oracle(formula, perm):
    rng = np.random.default_rng(410)
    a = o.bf16_round(rng.standard_normal((512, 1024)).astype(np.float32))
    b = o.bf16_round(rng.standard_normal((1024, 512)).astype(np.float32))
    pa = smx.pack_operand(dev(a), algo=7, side="lhs", tile_rows=256, bk=512, formula=formula, block_permutation=perm)
    assert np.array_equal(host(pa.data), o.packed_operand(a, 7, "lhs", 256, 512, formula, perm))
    pb = smx.pack_operand(dev_weight(b), algo=7, side="rhs", tile_rows=256, bk=512, formula=formula,
                          block_permutation=perm)
    assert np.array_equal(host(pb.data), o.packed_operand(b, 7, "rhs", 256, 512, formula, perm))


@pytest.mark.parametrize("formula", ["classical", "dual", "powers"])
def test_formula_variant_integer_kat(formula):
    rng = np.random.default_rng(411)
    a = rng.integers(-2, 3, (512, 1024)).astype(np.float32)
    b = rng.integers(-2, 3, (1024, 512)).astype(np.float32)
    for perm in range(8):
        say(f"  {formula} perm={perm}")
        got = host(smx.strassen_matmul(dev(a), dev_weight(b), bm=256, bn=256, bk=512, formula_variant=formula,
                                       block_permutation=perm))
        assert np.array_equal(got, o.bf16_round(a @ b)), perm


@pytest.mark.parametrize("formula,perm", VARIANTS)
def test_formula_variant_random_matches_oracle(formula, perm):
    _, a, b = _gaussian(412, 512, 2048, 512)
    kw = dict(bm=256, bn=256, bk=512, formula_variant=formula, block_permutation=perm)
    w = smx.strassen_weight_layout(dev_weight(b), 256, 512, formula_variant=formula, block_permutation=perm)
    got = host(smx.strassen_matmul(dev(a), w, **kw))
    want = o.strassen_matmul(a, b, **kw)
    assert_ulp_close(got, want, k=2048)
    ref = o.high_precision_reference(a, b).astype(np.float64)
    assert rel_l2(got, ref) <= 1e-2 and rel_l2(got, ref) <= 1.5 * rel_l2(want, ref)


def test_dual_permuted_with_fused_epilogues():
    rng, a, b = _gaussian(413, 512, 1024, 2048)
    laid = o.swiglu_weight_layout(b, 512)
    kw = dict(bm=256, bn=512, bk=512, formula_variant="dual", block_permutation=6)
    got = host(smx.strassen_matmul(dev(a), dev_weight(laid), epilogue="swiglu", **kw))
    assert_ulp_close(got, o.strassen_matmul(a, laid, epilogue="swiglu", **kw), k=1024)
    r = o.bf16_round(rng.standard_normal((512, 2048)).astype(np.float32))
    got = host(smx.strassen_matmul(dev(a), dev_weight(b), epilogue="residual_add", residual=dev(r), **kw))
    assert_ulp_close(got, o.strassen_matmul(a, b, epilogue="residual_add", residual=r, **kw), k=1024)


# ---------------------------------------------------------------------------
# Exact panels (classical_panels / panel_schedule): Strassen over the ordinary
# K panels into an FP32 partial, the cubic over the exact panels adding it.
# ---------------------------------------------------------------------------

EXACT_CASES = [((1,), "classical", 0), ((0, 3), "dual", 5), ((0, 1, 2, 3), "classical", 7),
               ((3,), "classical", 2)]


def _gather_panels(x, panels, bk, axis):
    cols = np.concatenate([np.arange(p * bk, (p + 1) * bk) for p in panels])
    return np.take(x, cols, axis=axis)


def test_pack_panel_map_matches_oracle():
    """A split operand's two parts are the oracle's packing of the gathered
    ordinary panels (Strassen sums) and exact panels (cubic quadrants)."""
    rng = np.random.default_rng(430)
    a = o.bf16_round(rng.standard_normal((512, 2048)).astype(np.float32))
    b = o.bf16_round(rng.standard_normal((2048, 512)).astype(np.float32))
    for formula, perm in (("classical", 0), ("dual", 3)):
        pa = smx.pack_activation(dev(a), 7, 256, 512, formula_variant=formula, block_permutation=perm,
                                 classical_panels=(2, 0))
        assert pa.schedule.exact == (0, 2) and pa.schedule.ordinary == (1, 3)
        assert np.array_equal(host(pa.ordinary.data), o.packed_operand(_gather_panels(a, (1, 3), 512, 1), 7,
                                                                       "lhs", 256, 512, formula, perm))
        assert np.array_equal(host(pa.exact.data), o.packed_operand(_gather_panels(a, (0, 2), 512, 1), 8,
                                                                    "lhs", 256, 512))
        pb = smx.strassen_weight_layout(dev_weight(b), 256, 512, formula_variant=formula, block_permutation=perm,
                                        panel_schedule=torch.tensor([1, 0, 1, 0], device=DEV))
        assert np.array_equal(host(pb.ordinary.data), o.packed_operand(_gather_panels(b, (1, 3), 512, 0), 7,
                                                                       "rhs", 256, 512, formula, perm))
        assert np.array_equal(host(pb.exact.data), o.packed_operand(_gather_panels(b, (0, 2), 512, 0), 8,
                                                                    "rhs", 256, 512))
    every = smx.pack_activation(dev(a), 7, 256, 512, classical_panels=range(4))
    assert every.ordinary is None
    assert np.array_equal(host(every.exact.data), o.packed_operand(a, 8, "lhs", 256, 512))


@pytest.mark.parametrize("panels,formula,perm", EXACT_CASES)
def test_exact_panels_integer_kat(panels, formula, perm):
    rng = np.random.default_rng(431)
    a = rng.integers(-2, 3, (512, 2048)).astype(np.float32)
    b = rng.integers(-2, 3, (2048, 512)).astype(np.float32)
    want = o.bf16_round(a @ b)
    kw = dict(bm=256, bn=256, bk=512, formula_variant=formula, block_permutation=perm)
    got = smx.strassen_matmul(dev(a), dev_weight(b), classical_panels=panels, **kw)
    assert np.array_equal(host(got), want)
    flags = torch.zeros(4, dtype=torch.int32, device=DEV)
    flags[list(panels)] = 1
    got = smx.strassen_matmul(dev(a), dev_weight(b), panel_schedule=flags, **kw)
    assert np.array_equal(host(got), want)
    w = smx.strassen_weight_layout(dev_weight(b), 256, 512, formula_variant=formula, block_permutation=perm,
                                   classical_panels=panels)
    got = smx.strassen_matmul(dev(a), w, classical_panels=panels, **kw)
    assert np.array_equal(host(got), want)


@pytest.mark.parametrize("panels,formula,perm", EXACT_CASES)
def test_exact_panels_random_matches_oracle(panels, formula, perm):
    _, a, b = _gaussian(432, 512, 2048, 512)
    kw = dict(bm=256, bn=256, bk=512, formula_variant=formula, block_permutation=perm, classical_panels=panels)
    got = host(smx.strassen_matmul(dev(a), dev_weight(b), **kw))
    want = o.strassen_matmul(a, b, **kw)
    assert_ulp_close(got, want, k=2048)
    ref = o.high_precision_reference(a, b).astype(np.float64)
    assert rel_l2(got, ref) <= 1e-2 and rel_l2(got, ref) <= 1.5 * rel_l2(want, ref)
    # FP32 output: the unrounded sum, to FP32 summation order
    got32 = host(smx.strassen_matmul(dev(a), dev_weight(b), output_dtype=torch.float32, **kw))
    want32 = o.strassen_matmul(a, b, output_dtype="float32", **kw)
    assert np.all(np.abs(got32 - want32) <= 4 * np.abs(want32) * 2.0 ** -23 + fp32_floor(want32, 2048))


def test_exact_panels_with_fused_epilogues():
    rng, a, b = _gaussian(433, 512, 2048, 1024)
    panels = (1, 2)
    laid = o.swiglu_weight_layout(b, 512)
    kw = dict(bm=256, bn=512, bk=512, classical_panels=panels)
    got = host(smx.strassen_matmul(dev(a), dev_weight(laid), epilogue="swiglu", **kw))
    assert_ulp_close(got, o.strassen_matmul(a, laid, epilogue="swiglu", **kw), k=2048)
    got = host(smx.strassen_matmul(dev(a), dev_weight(laid), epilogue="geglu", **kw))
    assert_ulp_close(got, o.strassen_matmul(a, laid, epilogue="geglu", **kw), k=2048)
    r = o.bf16_round(rng.standard_normal((512, 1024)).astype(np.float32))
    got = host(smx.strassen_matmul(dev(a), dev_weight(b), epilogue="residual_add", residual=dev(r), **kw))
    assert_ulp_close(got, o.strassen_matmul(a, b, epilogue="residual_add", residual=r, **kw), k=2048)
    bias = o.bf16_round(rng.standard_normal(1024).astype(np.float32))
    got = host(smx.strassen_matmul(dev(a), dev_weight(b), epilogue="bias_add", bias=dev(bias), **kw))
    assert_ulp_close(got, o.strassen_matmul(a, b, epilogue="bias_add", bias=bias, **kw), k=2048)
    g = o.bf16_round((1 + 0.1 * rng.standard_normal(1024)).astype(np.float32))
    kw_norm = dict(kw, bn=1024, epilogue="norm_residual_add")
    got = host(smx.strassen_matmul(dev(a), dev_weight(b), residual=dev(r), norm_scale=dev(g), **kw_norm))
    assert_ulp_close(got, o.strassen_matmul(a, b, residual=r, norm_scale=g, **kw_norm), k=2048)


def test_split_weight_reuse_and_mismatch():
    """A weight split once serves repeated calls with its schedule and is
    refused for another schedule or none."""
    _, a, b = _gaussian(434, 256, 2048, 512)
    w = smx.strassen_weight_layout(dev_weight(b), 256, 512, classical_panels=(0,))
    kw = dict(bm=256, bn=256, bk=512)
    first = smx.strassen_matmul(dev(a), w, classical_panels=(0,), **kw)
    second = smx.strassen_matmul(dev(a), w, panel_schedule=[1, 0, 0, 0], **kw)
    assert torch.equal(first, second)
    assert_ulp_close(host(first), o.strassen_matmul(a, b, classical_panels=(0,), **kw), k=2048)
    with pytest.raises(ValueError, match="packed for the exact panels"):
        smx.strassen_matmul(dev(a), w, classical_panels=(1,), **kw)
    with pytest.raises(ValueError, match="called without exact panels"):
        smx.strassen_matmul(dev(a), w, **kw)


@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float32])
def test_norm_residual_add_epilogue(scale_dtype):
    """Row RMSNorm over the whole output row, scale, residual (two passes on
    gfx950: FP32 GEMM result, then the row kernel)."""
    rng, a, b = _gaussian(421, 512, 2048, 1024)
    r = o.bf16_round(rng.standard_normal((512, 1024)).astype(np.float32))
    g = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)
    if scale_dtype == torch.bfloat16:
        g = o.bf16_round(g)
    g_dev = torch.from_numpy(g).to(DEV).to(scale_dtype)
    kw = dict(bm=256, bn=1024, bk=512, epilogue="norm_residual_add")
    for arm in ARMS:
        got = host(run_arm(arm, a, b, residual=dev(r), norm_scale=g_dev, **kw))
        want = oracle_arm(arm, a, b, residual=r, norm_scale=g, **kw)
        assert_ulp_close(got, want, k=2048)


def test_residual_add_epilogue():
    rng, a, b = _gaussian(319, 512, 2048, 1024)
    r = o.bf16_round(rng.standard_normal((512, 1024)).astype(np.float32))
    for arm in ARMS:
        got = host(run_arm(arm, a, b, bm=256, bn=512, bk=512, epilogue="residual_add", residual=dev(r)))
        assert_ulp_close(got, oracle_arm(arm, a, b, bm=256, bn=512, bk=512, epilogue="residual_add", residual=r),
                         k=2048)


@pytest.mark.parametrize("bias_dtype", [torch.bfloat16, torch.float32])
def test_bias_add_epilogue(bias_dtype):
    rng, a, b = _gaussian(321, 256, 1024, 1024)
    bias = rng.standard_normal(1024).astype(np.float32)
    if bias_dtype == torch.bfloat16:
        bias = o.bf16_round(bias)
    bias_dev = torch.from_numpy(bias).to(DEV).to(bias_dtype)
    for arm in ARMS:
        got = host(run_arm(arm, a, b, bm=256, bn=256, bk=512, epilogue="bias_add", bias=bias_dev))
        assert_ulp_close(got, oracle_arm(arm, a, b, bm=256, bn=256, bk=512, epilogue="bias_add", bias=bias), k=1024)


def _qk_problem(seed, batch, seq, heads, k, bn, hd=128):
    rng = np.random.default_rng(seed)
    tokens, n = batch * seq, heads * hd
    x = o.bf16_round(rng.standard_normal((tokens, k)).astype(np.float32))
    w = o.bf16_round(rng.standard_normal((k, n)).astype(np.float32) * np.float32(0.02))
    gamma = o.bf16_round((1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32))
    cos, sin = o.rope_values(seq, hd, 1e6)
    laid = o.rope_weight_layout(w, bn, hd)
    tcos, tsin = o.rope_layout_tables(np.tile(cos, (batch, 1)), np.tile(sin, (batch, 1)), bn // 2, hd)
    scale = o.rope_scale_layout(gamma, bn, hd)
    return x, w, laid, tcos, tsin, scale


@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float32])
def test_qk_norm_rope_epilogue(scale_dtype):
    batch, seq, heads, k, bn = 2, 256, 8, 1024, 512
    x, w, laid, tcos, tsin, scale = _qk_problem(11, batch, seq, heads, k, bn)
    kw = dict(bm=256, bn=bn, bk=512, epilogue="qk_norm_rope", rope_head_dim=128, rope_eps=1e-6)
    laid_dev = smx.rope_weight_layout(dev_weight(w), bn)
    assert np.array_equal(host(laid_dev), laid)
    for arm in ARMS:
        got = host(run_arm(arm, x, laid_dev, rope_cos=dev(tcos), rope_sin=dev(tsin),
                           rope_scale=torch.from_numpy(scale).to(DEV).to(scale_dtype), **kw))
        want = oracle_arm(arm, x, laid, rope_cos=tcos, rope_sin=tsin, rope_scale=scale, **kw)
        assert_ulp_close(got, want, k=k)


# ---------------------------------------------------------------------------
# FP32 inputs: the one-pass DEFAULT product (operand sums in float, each
# operand rounded once to bf16, FP32 accumulation)
# ---------------------------------------------------------------------------

def dev32(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(DEV)


def dev32_weight(b):
    """[K, N] float32 as a K-contiguous view of [N, K] device storage."""
    return dev32(np.asarray(b, np.float32).T).t()


def _gaussian32(seed, m, k, n, b_std=0.02):
    """Float32 inputs whose values are (almost all) not bf16 values."""
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32) * np.float32(b_std)
    assert not np.array_equal(a, o.bf16_round(a))
    return rng, a, b


def assert_f32_close(got, want, k):
    """FP32 results summed in another order: a few FP32 ulps plus the
    near-zero floor."""
    got = np.asarray(got, np.float32)
    assert got.dtype == np.float32 and np.isfinite(got).all()
    tol = 4 * np.abs(want) * 2.0 ** -23 + fp32_floor(want, k)
    bad = np.abs(got - want) > tol
    assert not bad.any(), f"{int(bad.sum())} elements beyond the FP32 tolerance"


FP32_PACK_CASES = [(7, "classical", 0), (7, "classical", 5), (7, "dual", 3), (7, "powers", 6), (8, "classical", 0)]


@pytest.mark.parametrize("algo,formula,perm", FP32_PACK_CASES)
def test_fp32_pack_matches_oracle(algo, formula, perm):
    """The packing pass on float32 sources: sums in float, one bf16
    rounding per operand, bit for bit (lhs, transposed lhs and rhs)."""
    _, a, b = _gaussian32(501, 512, 1024, 512)
    kw = dict(formula=formula, block_permutation=perm)
    pa = smx.pack_operand(dev32(a), algo=algo, side="lhs", tile_rows=256, bk=512, **kw)
    want_a = o.packed_operand(a, algo, "lhs", 256, 512, formula, perm, input_dtype="float32")
    assert pa.source_dtype == torch.float32
    assert np.array_equal(host(pa.data), want_a)
    pt = smx.pack_operand(dev32(a.T), algo=algo, side="lhs_t", tile_rows=256, bk=512, **kw)
    assert np.array_equal(host(pt.data), want_a)
    pb = smx.pack_operand(dev32_weight(b), algo=algo, side="rhs", tile_rows=256, bk=512, **kw)
    assert np.array_equal(host(pb.data), o.packed_operand(b, algo, "rhs", 256, 512, formula, perm,
                                                          input_dtype="float32"))
    # a row-major [K, N] weight is transposed by the wrapper, same bits
    pr = smx.pack_operand(dev32(b), algo=algo, side="rhs", tile_rows=256, bk=512, **kw)
    assert torch.equal(pr.data, pb.data)


def test_fp32_integer_kat():
    """Integer float32 data is exact under any summation order."""
    rng = np.random.default_rng(502)
    a = rng.integers(-2, 3, (512, 1024)).astype(np.float32)
    b = rng.integers(-2, 3, (1024, 512)).astype(np.float32)
    kw = dict(bm=256, bn=256, bk=512)
    for fn in (smx.strassen_matmul, smx.cubic_matmul):
        got = fn(dev32(a), dev32_weight(b), **kw)
        assert got.dtype == torch.float32
        assert np.array_equal(host(got), a @ b)


@pytest.mark.parametrize("arm", ARMS)
def test_fp32_inputs_match_oracle(arm):
    """FP32 inputs on every arm (the plain arms are packed for the call: FP32
    reaches the kernels through the packing pass). Default output FP32, and
    BF16 when asked; error against the float64 product within the gate."""
    _, a, b = _gaussian32(503, 512, 2048, 768)
    kw = dict(bm=256, bn=256, bk=512)
    okw = dict(kw, input_dtype="float32") if arm.startswith("strassen") else dict(kw)
    got = run_arm(arm, dev32(a), dev32_weight(b), **kw)
    assert got.dtype == torch.float32
    want = oracle_arm(arm, a, b, output_dtype="float32", **okw)
    assert_f32_close(host(got), want, 2048)
    got16 = run_arm(arm, dev32(a), dev32_weight(b), output_dtype=torch.bfloat16, **kw)
    assert got16.dtype == torch.bfloat16
    assert np.array_equal(host(got16), o.bf16_round(host(got)))
    # the gate: <= 1e-2 and <= 1.5x the reference algorithm's own error. With
    # FP32 inputs the one-pass product rounds Strassen's operand sums, which
    # costs about 2x the cubic's error (the cubic rounds single quadrants).
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert rel_l2(host(got), ref) <= 1e-2
    assert rel_l2(host(got), ref) <= 1.5 * rel_l2(want, ref)


@pytest.mark.parametrize("formula,perm", VARIANTS)
def test_fp32_formula_variants(formula, perm):
    _, a, b = _gaussian32(504, 512, 1024, 512)
    kw = dict(bm=256, bn=256, bk=512, formula_variant=formula, block_permutation=perm)
    got = host(smx.strassen_matmul(dev32(a), dev32_weight(b), **kw))
    assert_f32_close(got, o.strassen_matmul(a, b, output_dtype="float32", input_dtype="float32", **kw), 1024)
    w = smx.strassen_weight_layout(dev32_weight(b), 256, 512, formula_variant=formula, block_permutation=perm)
    assert torch.equal(torch.from_numpy(got), smx.strassen_matmul(dev32(a), w, **kw).cpu())


def test_fp32_epilogues():
    """Fused epilogues on FP32 inputs: a BF16 tile when asked (one rounding of
    the same FP32 values), else an FP32 tile; FP32 residual and bias."""
    rng, a, b = _gaussian32(505, 512, 1024, 1024)
    kw = dict(bm=256, bn=512, bk=512)
    okw = dict(kw, input_dtype="float32")
    laid = o.swiglu_weight_layout(b, 512)
    laid_dev = smx.swiglu_weight_layout(dev32_weight(b), 512)
    r = rng.standard_normal((512, 1024)).astype(np.float32)
    bias = rng.standard_normal(1024).astype(np.float32)
    cases = [
        (dict(epilogue="swiglu"), dict(epilogue="swiglu"), laid_dev, laid),
        (dict(epilogue="geglu"), dict(epilogue="geglu"), laid_dev, laid),
        (dict(epilogue="residual_add", residual=dev32(r)), dict(epilogue="residual_add", residual=r),
         dev32_weight(b), b),
        (dict(epilogue="bias_add", bias=dev32(bias)), dict(epilogue="bias_add", bias=bias), dev32_weight(b), b),
    ]
    for dkw, hkw, w_dev, w in cases:
        say(f"  {dkw['epilogue']}")
        got16 = host(smx.strassen_matmul(dev32(a), w_dev, output_dtype=torch.bfloat16, **dkw, **kw))
        assert_ulp_close(got16, o.strassen_matmul(a, w, **hkw, **okw), k=1024)
        got = smx.strassen_matmul(dev32(a), w_dev, **dkw, **kw)
        assert got.dtype == torch.float32
        want = o.strassen_matmul(a, w, output_dtype="float32", **hkw, **okw)
        assert rel_l2(host(got), want) <= 1e-6
    g = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)
    nkw = dict(kw, bn=1024, epilogue="norm_residual_add")
    got = host(smx.strassen_matmul(dev32(a), dev32_weight(b), residual=dev32(r), norm_scale=dev32(g),
                                   output_dtype=torch.bfloat16, **nkw))
    assert_ulp_close(got, o.strassen_matmul(a, b, residual=r, norm_scale=g, input_dtype="float32", **nkw), k=1024)


def test_fp32_lhs_transposed():
    rng = np.random.default_rng(506)
    k, m, n = 1024, 512, 768
    a_t = rng.standard_normal((k, m)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32) * np.float32(0.02)
    got = smx.strassen_matmul_lhs_transposed(dev32(a_t), dev32(b), bm=256, bn=256, bk=512)
    assert got.dtype == torch.float32 and tuple(got.shape) == (m, n)
    want = o.strassen_matmul_lhs_transposed(a_t, b, bm=256, bn=256, bk=512, output_dtype="float32",
                                            input_dtype="float32")
    assert_f32_close(host(got), want, k)


@pytest.mark.parametrize("panels,formula,perm", [((1,), "classical", 0), ((0, 3), "dual", 2)])
def test_fp32_exact_panels(panels, formula, perm):
    _, a, b = _gaussian32(507, 512, 2048, 512)
    kw = dict(bm=256, bn=256, bk=512, formula_variant=formula, block_permutation=perm, classical_panels=panels)
    got = host(smx.strassen_matmul(dev32(a), dev32_weight(b), **kw))
    assert_f32_close(got, o.strassen_matmul(a, b, output_dtype="float32", input_dtype="float32", **kw), 2048)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert rel_l2(got, ref) <= 1e-2


# ---------------------------------------------------------------------------
# FP32 inputs at dot_precision HIGH / HIGHEST (3 / 6 bf16 passes per product)
# ---------------------------------------------------------------------------

PRECISIONS = ("high", "highest")
# float64-product error bounds per precision on N(0,1) x N(0,0.02) data at
# K = 2048 (HIGH drops second-order parts, ~1e-5; HIGHEST reaches the FP32
# accumulation level, ~1e-6)
PRECISION_BOUND = {"high": 3e-5, "highest": 3e-6}


@pytest.mark.parametrize("precision", PRECISIONS)
@pytest.mark.parametrize("algo,formula,perm", [(7, "classical", 0), (7, "dual", 3), (7, "powers", 6),
                                               (8, "classical", 0)])
def test_multi_pass_pack_matches_oracle(precision, algo, formula, perm):
    """Packed bf16 parts, panel by panel with each panel's passes, bit for
    bit (lhs, transposed lhs and rhs)."""
    _, a, b = _gaussian32(511, 512, 1024, 512)
    kw = dict(formula=formula, block_permutation=perm, dot_precision=precision)
    okw = dict(input_dtype="float32", dot_precision=precision)
    pa = smx.pack_operand(dev32(a), algo=algo, side="lhs", tile_rows=256, bk=512, **kw)
    assert pa.passes == {"high": 3, "highest": 6}[precision] and pa.k == 1024
    want_a = o.packed_operand(a, algo, "lhs", 256, 512, formula, perm, **okw)
    assert np.array_equal(host(pa.data), want_a)
    pt = smx.pack_operand(dev32(a.T), algo=algo, side="lhs_t", tile_rows=256, bk=512, **kw)
    assert np.array_equal(host(pt.data), want_a)
    pb = smx.pack_operand(dev32_weight(b), algo=algo, side="rhs", tile_rows=256, bk=512, **kw)
    assert np.array_equal(host(pb.data), o.packed_operand(b, algo, "rhs", 256, 512, formula, perm, **okw))


@pytest.mark.parametrize("precision", PRECISIONS)
@pytest.mark.parametrize("arm", ARMS)
def test_multi_pass_matches_oracle(precision, arm):
    _, a, b = _gaussian32(512, 512, 2048, 512)
    kw = dict(bm=256, bn=256, bk=512, dot_precision=precision)
    okw = dict(kw, input_dtype="float32") if arm.startswith("strassen") else dict(kw)
    got = host(run_arm(arm, dev32(a), dev32_weight(b), **kw))
    want = oracle_arm(arm, a, b, output_dtype="float32", **okw)
    passes = {"high": 3, "highest": 6}[precision]
    assert_f32_close(got, want, passes * 2048)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert rel_l2(got, ref) <= PRECISION_BOUND[precision]
    assert rel_l2(got, ref) <= 1.5 * rel_l2(want, ref) + 1e-7


def test_multi_pass_variants_and_epilogues():
    """Formula variants, an offline-packed weight, exact panels, the
    transposed LHS and a fused epilogue at HIGHEST; a weight packed for
    another precision is refused."""
    rng, a, b = _gaussian32(513, 512, 2048, 512)
    kw = dict(bm=256, bn=256, bk=512, dot_precision="highest")
    okw = dict(kw, input_dtype="float32", output_dtype="float32")
    for formula, perm in (("dual", 5), ("powers", 2)):
        vkw = dict(formula_variant=formula, block_permutation=perm)
        got = host(smx.strassen_matmul(dev32(a), dev32_weight(b), **vkw, **kw))
        assert_f32_close(got, o.strassen_matmul(a, b, **vkw, **okw), 6 * 2048)
    w = smx.strassen_weight_layout(dev32_weight(b), 256, 512, dot_precision="highest")
    got = host(smx.strassen_matmul(dev32(a), w, **kw))
    assert_f32_close(got, o.strassen_matmul(a, b, **okw), 6 * 2048)
    with pytest.raises(ValueError, match="bf16 pass"):
        smx.strassen_matmul(dev32(a), w, bm=256, bn=256, bk=512, dot_precision="high")
    with pytest.raises(ValueError, match="bf16 pass"):
        smx.strassen_matmul(dev32(a), w, bm=256, bn=256, bk=512)
    got = host(smx.strassen_matmul(dev32(a), dev32_weight(b), classical_panels=(1, 2), **kw))
    assert_f32_close(got, o.strassen_matmul(a, b, classical_panels=(1, 2), **okw), 6 * 2048)
    got = host(smx.strassen_matmul_lhs_transposed(dev32(a.T), dev32(b), bm=256, bn=256, bk=512,
                                                  dot_precision="high"))
    assert_f32_close(got, o.strassen_matmul(a, b, **dict(okw, dot_precision="high")), 3 * 2048)
    r = rng.standard_normal((512, 512)).astype(np.float32)
    got = host(smx.strassen_matmul(dev32(a), dev32_weight(b), epilogue="residual_add", residual=dev32(r), **kw))
    want = o.strassen_matmul(a, b, epilogue="residual_add", residual=r, **okw)
    assert rel_l2(got, want) <= 1e-6
    ref = a.astype(np.float64) @ b.astype(np.float64) + r
    assert rel_l2(got, ref) <= PRECISION_BOUND["highest"]


# ---------------------------------------------------------------------------
# Block permutations with every fused epilogue: the permutation moves where a
# quadrant is stored, and swaps the gate/up and a/b roles of a column swap
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("formula", ["classical", "dual"])
@pytest.mark.parametrize("perm", range(8))
def test_permutation_with_every_epilogue(formula, perm):
    rng, a, b = _gaussian(450 + perm, 512, 1024, 1024)
    kw = dict(bm=256, bn=512, bk=512, formula_variant=formula, block_permutation=perm)
    laid = o.swiglu_weight_layout(b, 512)
    for epi in ("swiglu", "geglu"):
        got = host(smx.strassen_matmul(dev(a), dev_weight(laid), epilogue=epi, **kw))
        assert_ulp_close(got, o.strassen_matmul(a, laid, epilogue=epi, **kw), k=1024)
    got = host(smx.strassen_matmul(dev(a), dev_weight(b), **kw))
    assert_ulp_close(got, o.strassen_matmul(a, b, **kw), k=1024)
    r = o.bf16_round(rng.standard_normal((512, 1024)).astype(np.float32))
    got = host(smx.strassen_matmul(dev(a), dev_weight(b), epilogue="residual_add", residual=dev(r), **kw))
    assert_ulp_close(got, o.strassen_matmul(a, b, epilogue="residual_add", residual=r, **kw), k=1024)
    bias = o.bf16_round(rng.standard_normal(1024).astype(np.float32))
    got = host(smx.strassen_matmul(dev(a), dev_weight(b), epilogue="bias_add", bias=dev(bias), **kw))
    assert_ulp_close(got, o.strassen_matmul(a, b, epilogue="bias_add", bias=bias, **kw), k=1024)
    x, w, lq, tcos, tsin, scale = _qk_problem(460 + perm, 2, 256, 8, 1024, 512)
    qkw = dict(kw, epilogue="qk_norm_rope", rope_head_dim=128, rope_eps=1e-6)
    got = host(smx.strassen_matmul(dev(x), dev_weight(lq), rope_cos=dev(tcos), rope_sin=dev(tsin),
                                   rope_scale=dev(scale), **qkw))
    assert_ulp_close(got, o.strassen_matmul(x, lq, rope_cos=tcos, rope_sin=tsin, rope_scale=scale, **qkw), k=1024)


# ---------------------------------------------------------------------------
# Full Qwen3-32B shapes (8 x 1024 tokens)
# ---------------------------------------------------------------------------

QWEN_SHAPES = {
    "gate_up": (8192, 5120, 25600),
    "down": (8192, 25600, 5120),
    "o": (8192, 8192, 5120),
}


@pytest.mark.parametrize("site", sorted(QWEN_SHAPES))
def test_qwen3_32b_shapes_sampled_tiles(site):
    m, k, n = QWEN_SHAPES[site]
    bm, bn, bk = 1024, 1024, 512
    gen = torch.Generator(device=DEV).manual_seed(7)
    a = torch.randn(m, k, device=DEV, generator=gen).to(torch.bfloat16)
    w = (torch.randn(n, k, device=DEV, generator=gen) * 0.02).to(torch.bfloat16)
    b = w.t()  # [K, N], K-contiguous
    say(f"  {site} m={m} k={k} n={n}")
    got = smx.strassen_matmul(a, b, bm=bm, bn=bn, bk=bk, interleave_products=True)
    pre = smx.strassen_matmul(a, smx.strassen_weight_layout(b, bn, bk), bm=bm, bn=bn, bk=bk)
    cub = smx.cubic_matmul(a, smx.cubic_weight_layout(b, bn, bk), bm=bm, bn=bn, bk=bk)
    cub_plain = smx.cubic_matmul(a, b, bm=bm, bn=bn, bk=bk)
    torch.cuda.synchronize()
    # The compact and packed kernels compute the same bf16 operand sums.
    e_pre = float(torch.linalg.norm(pre.float() - got.float()) / torch.linalg.norm(got.float()))
    e_cub = float(torch.linalg.norm(cub.float() - cub_plain.float()) / torch.linalg.norm(cub.float()))
    say(f"  compact vs packed rel diff strassen {e_pre:.3e} cubic {e_cub:.3e}")
    assert e_pre < 1e-3 and e_cub < 1e-3
    # Whole-output bound against an FP32 product computed on the GPU.
    ref = torch.matmul(a.float(), b.float())
    e_s = float(torch.linalg.norm(got.float() - ref) / torch.linalg.norm(ref))
    e_c = float(torch.linalg.norm(cub.float() - ref) / torch.linalg.norm(ref))
    say(f"  whole-output rel err strassen={e_s:.4e} cubic={e_c:.4e}")
    assert e_s <= 1e-2 and e_c <= 1e-2 and e_c < e_s
    # Sampled tiles recomputed by the oracle from their own rows / columns.
    rng = np.random.default_rng(1)
    a_h, b_h = host(a), host(b)
    for _ in range(2):
        i = int(rng.integers(m // bm))
        j = int(rng.integers(n // bn))
        rows, cols = slice(i * bm, (i + 1) * bm), slice(j * bn, (j + 1) * bn)
        want = o.strassen_matmul(a_h[rows], b_h[:, cols], bm=bm, bn=bn, bk=bk, interleave_products=True)
        assert_ulp_close(host(got[rows, cols]), want, k=k)
        assert_ulp_close(host(pre[rows, cols]), want, k=k)
        ref_tile = o.high_precision_reference(a_h[rows], b_h[:, cols]).astype(np.float64)
        assert rel_l2(host(got[rows, cols]), ref_tile) <= 1.5 * rel_l2(want, ref_tile)
        want_c = o.cubic_blocked_matmul(a_h[rows], b_h[:, cols], bm=bm, bn=bn, bk=bk)
        assert_ulp_close(host(cub[rows, cols]), want_c, k=k)


def test_output_beyond_2gib():
    """M = 65536 tokens on the gate|up shape: the 3.4 GB output (and the
    residual of residual_add) lie past 2^31 bytes, so every store and load
    offset needs 64 bits. Tiles at the far end are recomputed by the oracle."""
    m, k, n = 65536, 5120, 25600
    bm, bn, bk = 1024, 1024, 512
    gen = torch.Generator(device=DEV).manual_seed(11)
    a = torch.randn(m, k, device=DEV, generator=gen).to(torch.bfloat16)
    b = (torch.randn(n, k, device=DEV, generator=gen) * 0.02).to(torch.bfloat16).t()
    r = torch.randn(m, n, device=DEV, generator=gen).to(torch.bfloat16)
    assert r.numel() * 2 > 2 ** 31
    say(f"  m={m} k={k} n={n}")
    w = smx.strassen_weight_layout(b, bn, bk)
    got = smx.strassen_matmul(a, w, bm=bm, bn=bn, bk=bk)
    res = smx.strassen_matmul(a, w, bm=bm, bn=bn, bk=bk, epilogue="residual_add", residual=r)
    cub = smx.cubic_matmul(a, smx.cubic_weight_layout(b, bn, bk), bm=bm, bn=bn, bk=bk)
    torch.cuda.synchronize()
    for i, j in ((m // bm - 1, n // bn - 1), (m // bm - 2, 3), (45, n // bn - 2)):
        rows, cols = slice(i * bm, (i + 1) * bm), slice(j * bn, (j + 1) * bn)
        assert (i * bm) * n * 2 >= 2 ** 31
        a_h, b_h, r_h = host(a[rows]), host(b[:, cols]), host(r[rows, cols])
        want = o.strassen_matmul(a_h, b_h, bm=bm, bn=bn, bk=bk)
        assert_ulp_close(host(got[rows, cols]), want, k=k)
        want_r = o.strassen_matmul(a_h, b_h, bm=bm, bn=bn, bk=bk, epilogue="residual_add", residual=r_h)
        assert_ulp_close(host(res[rows, cols]), want_r, k=k)
        assert_ulp_close(host(cub[rows, cols]), o.cubic_blocked_matmul(a_h, b_h, bm=bm, bn=bn, bk=bk), k=k)
