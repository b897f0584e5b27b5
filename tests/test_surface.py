"""Host-side behaviour of the drop-in surface: the reference's argument
checks (strassen_pallas.py:927-1047) raise the same exception types and
messages, and unsupported research options fail loudly. No GPU is used: every
case is rejected before a launch."""

import pytest
import torch

import strassen_tpu_amd as smx
from strassen_tpu_amd import strassen as surface


def t(*shape, dtype=torch.bfloat16):
    return torch.zeros(*shape, dtype=dtype)


@pytest.mark.parametrize("kwargs,args,exc,match", [
    ({}, (t(4), t(4, 4)), ValueError, "two rank-2 matrices"),
    ({}, (t(256, 512), t(256, 256)), ValueError, "inner dimensions disagree: 512 vs 256"),
    ({}, (t(256, 512), t(512, 256, dtype=torch.float32)), ValueError, "input dtypes disagree"),
    ({}, (t(256, 512, dtype=torch.float16), t(512, 256, dtype=torch.float16)), ValueError, "BF16 or FP32"),
    ({"block_permutation": 9}, None, ValueError, "block_permutation must be"),
    ({"formula_variant": "fancy"}, None, ValueError, "formula_variant must be"),
    ({"epilogue": "gelu"}, None, ValueError, "unknown epilogue"),
    ({"epilogue": "swiglu", "formula_variant": "powers"}, None, ValueError, "quadrant-basis formula"),
    ({"epilogue": "swiglu", "output_dtype": torch.float32}, None, ValueError, "BF16 output tile"),
    ({"epilogue": "residual_add"}, None, ValueError, "requires residual="),
    ({"epilogue": "bias_add"}, None, ValueError, "requires bias="),
    ({"residual": t(256, 256)}, None, ValueError, "residual= is only used"),
    ({"bias": t(256)}, None, ValueError, "bias= is only used"),
    ({"epilogue": "qk_norm_rope"}, None, ValueError, "requires rope_cos="),
    ({"epilogue": "qk_norm_rope", "bn": 128, "rope_cos": t(256, 64), "rope_sin": t(256, 64),
      "rope_scale": t(128)}, None, ValueError, "multiple of 2\\*head_dim"),
    ({"epilogue": "qk_norm_rope", "rope_cos": t(256, 64), "rope_sin": t(256, 64),
      "rope_scale": t(256)}, None, ValueError, "rope tables must be"),
    ({"epilogue": "qk_norm_rope", "rope_cos": t(256, 128), "rope_sin": t(256, 128),
      "rope_scale": t(128)}, None, ValueError, "rope_scale must be laid out"),
    ({"rope_cos": t(256, 128)}, None, ValueError, "rope_\\* are only used"),
    ({"product_aware_swiglu": True}, None, ValueError, "product_aware_swiglu is only valid"),
    ({"product_aware_residual": True}, None, ValueError, "product_aware_residual is only valid"),
    ({"epilogue": "bias_add", "bias": t(128)}, None, ValueError, "bias shape"),
    ({"allow_input_fusion": (True,)}, None, ValueError, "one boolean per operand"),
    ({"allow_input_fusion": (1, 0)}, None, TypeError, "must be bool"),
    ({"classical_panels": (0,), "panel_schedule": [0]}, None, ValueError, "not both"),
    ({"classical_panels": (5,)}, None, ValueError, "outside 0..0"),
    ({"bm": 96}, None, ValueError, "M=256 is not divisible by 96"),
    ({"bm": 8, "bn": 128, "bk": 128}, (t(256, 512), t(512, 256)), ValueError, "TPU v5e alignment"),
    ({"output_dtype": torch.float16}, None, ValueError, "output_dtype must be"),
])
def test_reference_argument_errors(kwargs, args, exc, match):
    a, b = args if args is not None else (t(256, 512), t(512, 256))
    base = {"bm": 256, "bn": 256, "bk": 512}
    base.update(kwargs)
    with pytest.raises(exc, match=match):
        smx.strassen_matmul(a, b, **base)


@pytest.mark.parametrize("kwargs,match", [
    # strassen_pallas.py:1079-1090
    ({"panel_schedule": [1], "epilogue": "bias_add", "bias": t(256)}, "does not support fused epilogues"),
    ({"panel_schedule": [1, 0]}, "must have shape \\(1,\\), got \\(2,\\)"),
    ({"panel_schedule": torch.zeros(1, 1, dtype=torch.int32)}, "must have shape \\(1,\\), got \\(1, 1\\)"),
    ({"panel_schedule": [1], "formula_variant": "powers"}, "quadrant-basis formula"),
    ({"classical_panels": (0,), "formula_variant": "powers"}, "quadrant-basis formula"),
    # the kernel's product-aware checks (:299-322): not on the final K panel
    ({"classical_panels": (0,), "epilogue": "swiglu", "product_aware_swiglu": True}, "product-aware SwiGLU"),
    ({"epilogue": "swiglu", "product_aware_swiglu": True, "block_permutation": 1}, "product-aware SwiGLU"),
    ({"classical_panels": (0,), "epilogue": "residual_add", "residual": t(256, 256),
      "product_aware_residual": True}, "product-aware residual"),
])
def test_exact_panel_argument_errors(kwargs, match):
    a, b = t(256, 512), t(512, 256)
    with pytest.raises(ValueError, match=match):
        smx.strassen_matmul(a, b, bm=256, bn=256, bk=512, **kwargs)


def test_exact_schedule_resolution():
    from strassen_tpu_amd.packing import exact_schedule

    assert exact_schedule(4) is None
    assert exact_schedule(4, panel_schedule=[0, 0, 0, 0]) is None
    s = exact_schedule(4, classical_panels=(3, 1, 1))
    assert (s.exact, s.ordinary, s.nk) == ((1, 3), (0, 2), 4)
    assert exact_schedule(4, panel_schedule=[0, 2, 0, -1]) == s
    # int32 conversion truncates toward zero, like jnp.asarray(..., int32)
    assert exact_schedule(4, panel_schedule=[0.5, 1.0, 0.0, 0.9]).exact == (1,)
    with pytest.raises(ValueError, match="outside 0..3"):
        exact_schedule(4, classical_panels=(4,))


def test_split_operand_checks():
    from strassen_tpu_amd.packing import SplitOperand, exact_schedule

    def part(algo, k):
        return smx.PackedOperand(t(1), algo=algo, side="rhs", rows=512, k=k, tile_rows=512, bk=512)

    sched = exact_schedule(2, classical_panels=(1,))
    w = SplitOperand(part(7, 512), part(8, 512), side="rhs", rows=512, k=1024, tile_rows=512, bk=512,
                     formula="classical", block_permutation=0, schedule=sched)
    assert w.shape == (1024, 512) and "exact_panels=(1,)" in repr(w)
    a = t(256, 1024)
    with pytest.raises(ValueError, match="packed for the exact panels \\(1,\\); called without"):
        smx.strassen_matmul(a, w, bm=256, bn=512, bk=512)
    with pytest.raises(ValueError, match="packed for the exact panels \\(1,\\); called with \\(0,\\)"):
        smx.strassen_matmul(a, w, bm=256, bn=512, bk=512, classical_panels=(0,))
    with pytest.raises(ValueError, match="packed for formula_variant"):
        smx.strassen_matmul(a, w, bm=256, bn=512, bk=512, classical_panels=(1,), formula_variant="dual")
    plain = smx.PackedOperand(t(1), algo=7, side="rhs", rows=512, k=1024, tile_rows=512, bk=512)
    with pytest.raises(ValueError, match="packed without exact panels"):
        smx.strassen_matmul(a, plain, bm=256, bn=512, bk=512, classical_panels=(1,))
    with pytest.raises(ValueError, match="HIP device"):
        smx.strassen_matmul(a, w, bm=256, bn=512, bk=512, classical_panels=(1,))


@pytest.mark.parametrize("kwargs", [
    {"interpret": True},
])
def test_unported_options_raise_not_implemented(kwargs):
    a, b = t(256, 512), t(512, 256)
    with pytest.raises(NotImplementedError):
        smx.strassen_matmul(a, b, bm=256, bn=256, bk=512, **kwargs)


def test_fp32_inputs_and_dot_precision():
    """FP32 inputs run the product of dot_precision: one bf16 pass at
    DEFAULT, 3 at HIGH, 6 at HIGHEST (names and aliases as jax.lax.Precision
    takes them, the same mapping as the oracle's); bf16 inputs always take
    one pass. CPU tensors stop at the device check."""
    import enum

    import oracle as o
    a, b = t(256, 512, dtype=torch.float32), t(512, 256, dtype=torch.float32)

    class Precision(enum.Enum):  # the shape of jax.lax.Precision members
        DEFAULT = 0
        HIGH = 1
        HIGHEST = 2

    names = [None, "DEFAULT", "default", "fastest", "bfloat16", "high", "HIGH", "bfloat16_3x", "tensorfloat32",
             "highest", "float32", "Precision.HIGHEST", Precision.DEFAULT, Precision.HIGH, Precision.HIGHEST]
    for precision in names:
        passes = smx.precision_passes(precision, torch.float32)
        assert passes == o.precision_passes(precision, "float32")
        assert smx.precision_passes(precision, torch.bfloat16) == 1
        with pytest.raises(ValueError, match="HIP device"):
            smx.strassen_matmul(a, b, bm=256, bn=256, bk=512, dot_precision=precision)
        with pytest.raises(ValueError, match="HIP device"):
            smx.cubic_matmul(a, b, bm=256, bn=256, bk=512, dot_precision=precision)
        with pytest.raises(ValueError, match="HIP device"):
            smx.strassen_matmul_lhs_transposed(t(512, 256, dtype=torch.float32), b, bm=256, bn=256, bk=512,
                                               dot_precision=precision)
    assert [smx.precision_passes(p, torch.float32) for p in (Precision.DEFAULT, Precision.HIGH,
                                                             Precision.HIGHEST)] == [1, 3, 6]
    assert smx.precision_passes(("high", Precision.HIGH), torch.float32) == 3
    with pytest.raises(NotImplementedError, match="two different precisions"):
        smx.precision_passes(("high", "highest"), torch.float32)
    with pytest.raises(ValueError, match="unknown dot_precision"):
        smx.strassen_matmul(a, b, bm=256, bn=256, bk=512, dot_precision="fp64")
    with pytest.raises(ValueError, match="input dtypes disagree"):
        smx.cubic_matmul(a, t(512, 256), bm=256, bn=256, bk=512)


def test_gfx950_tile_rule_and_device_check():
    a, b = t(256, 512), t(512, 256)
    # every tile the reference's check_tiling accepts passes the gfx950 rule
    # (bm=16 runs the thin-tiling kernels) and fails here only on CPU tensors
    for bm in (16, 32, 128):
        with pytest.raises(ValueError, match="HIP device"):
            smx.strassen_matmul(a, b, bm=bm, bn=256, bk=256)
    with pytest.raises(ValueError, match="HIP device"):
        smx.strassen_matmul(a, b, bm=256, bn=256, bk=512)
    with pytest.raises(ValueError, match="HIP device"):
        smx.cubic_matmul(a, b, bm=256, bn=256, bk=512)


def test_cubic_surface_checks():
    a, b = t(256, 512), t(512, 256)
    with pytest.raises(ValueError, match="unknown cubic variant"):
        smx.cubic_matmul(a, b, variant="sparse")
    with pytest.raises(ValueError, match="not divisible"):
        smx.cubic_matmul(a, b, bm=96, bn=256, bk=512)
    w = smx.PackedOperand(t(1, 1), algo=7, side="rhs", rows=256, k=512, tile_rows=256, bk=512)
    with pytest.raises(ValueError, match="packed as"):
        smx.cubic_matmul(a, w, bm=256, bn=256, bk=512)


@pytest.mark.parametrize("kwargs,match", [
    ({"epilogue": "gelu"}, "unknown epilogue"),
    ({"epilogue": "swiglu", "output_dtype": torch.float32}, "BF16 output tile"),
    ({"epilogue": "residual_add"}, "requires residual="),
    ({"epilogue": "residual_add", "residual": t(256, 128)}, "residual shape"),
    ({"epilogue": "residual_add", "residual": t(128, 256)}, "residual shape"),
    ({"epilogue": "bias_add"}, "requires bias="),
    ({"epilogue": "bias_add", "bias": t(128)}, "bias shape"),
    ({"bias": t(256)}, "bias= is only used"),
    ({"residual": t(256, 256)}, "residual= is only used"),
    ({"epilogue": "qk_norm_rope"}, "requires rope_cos="),
    ({"epilogue": "qk_norm_rope", "rope_cos": t(64, 128), "rope_sin": t(64, 128), "rope_scale": t(256)},
     "rope tables must be"),
    ({"epilogue": "qk_norm_rope", "rope_cos": t(256, 128), "rope_sin": t(256, 128), "rope_scale": t(128)},
     "rope_scale must be laid out"),
    ({"rope_cos": t(256, 128)}, "rope_\\* are only used"),
    ({"epilogue": "norm_residual_add", "residual": t(256, 256)}, "requires residual= and norm_scale="),
    ({"epilogue": "norm_residual_add", "residual": t(256, 128), "norm_scale": t(256)}, "residual shape"),
    ({"epilogue": "norm_residual_add", "residual": t(256, 256), "norm_scale": t(128)}, "norm_scale shape"),
])
def test_cubic_epilogue_operand_checks(kwargs, match):
    """The cubic control checks its epilogue operands like strassen_matmul:
    the kernels read them by address only, so a short bias, residual or
    table would otherwise be read out of bounds on the device."""
    base = {"bm": 256, "bn": 256, "bk": 512}
    base.update(kwargs)
    with pytest.raises(ValueError, match=match):
        smx.cubic_matmul(t(256, 512), t(512, 256), **base)


def packed_weight(algo=7, n=512, k=512, bn=512, bk=512):
    return smx.PackedOperand(t(n // 2 * k // 2 * (7 if algo == 7 else 4)), algo=algo, side="rhs",
                             rows=n, k=k, tile_rows=bn, bk=bk)


def test_packed_weight_surface():
    a = t(256, 512)
    w = packed_weight()
    assert w.shape == (512, 512) and w.dim() == 2 and w.dtype == torch.bfloat16
    with pytest.raises(ValueError, match="packed for the tile"):
        smx.strassen_matmul(a, w, bm=256, bn=256, bk=512)
    with pytest.raises(ValueError, match="HIP device"):
        smx.strassen_matmul(a, w, bm=256, bn=512, bk=512)
    with pytest.raises(ValueError, match="packed as"):
        smx.strassen_matmul(a, packed_weight(algo=8), bm=256, bn=512, bk=512)
    pa = smx.PackedOperand(t(1), algo=7, side="lhs", rows=256, k=512, tile_rows=256, bk=512)
    with pytest.raises(ValueError, match="needs a packed weight"), smx.plain_weight_kernel("compact"):
        smx.strassen_matmul(pa, t(512, 512), bm=256, bn=512, bk=512)
    # by default a plain weight with a packed-kernel tile is packed for the call
    with pytest.raises(ValueError, match="HIP device"):
        smx.strassen_matmul(pa, t(512, 512), bm=256, bn=512, bk=512)
    with pytest.raises(ValueError, match="must be 'pack' or 'compact'"), smx.plain_weight_kernel("fast"):
        pass
    with pytest.raises(ValueError, match="HIP device"):
        smx.strassen_weight_layout(t(512, 256), 256, 512)
    with pytest.raises(ValueError, match="bf16 or float32"):
        smx.strassen_weight_layout(t(512, 256, dtype=torch.float16), 256, 512)


@pytest.mark.parametrize("algo", [7, 8])
@pytest.mark.parametrize("side", ["lhs", "rhs"])
def test_oracle_packed_layout_brute_force(algo, side):
    """Walk every packed position with explicit index arithmetic."""
    import numpy as np

    import oracle as o

    rng = np.random.default_rng(1)
    tile, bk = 512, 64
    rows, k = 1024, 128  # 2 row tiles, 2 K panels; R = 512, depth 64
    x = o.bf16_round(rng.standard_normal((rows, k) if side == "lhs" else (k, rows)).astype(np.float32))
    flat = o.packed_operand(x, algo, side, tile, bk)
    nops = 7 if algo == 7 else 4
    assert flat.size == rows // 2 * k // 2 * nops
    ht, hk = tile // 2, bk // 2
    r = lambda v: o.bf16_round(np.float32(v)).item()
    at = lambda row, col: x[row, col] if side == "lhs" else x[col, row]
    pos = 0
    for ptile in range(rows // 2 // 128):
        for stage in range(k // 2 // 16):
            for op in range(nops):
                for block in range(4):
                    for lane in range(64):
                        prow = ptile * 128 + block * 32 + lane % 32
                        i, rr = divmod(prow, ht)
                        first, second = i * tile + rr, i * tile + rr + ht
                        got = flat[pos:pos + 8]
                        pos += 8
                        want = []
                        for e in range(8):
                            kp = stage * 16 + (lane // 32) * 8 + e
                            s_, kk = divmod(kp, hk)
                            lo, hi = s_ * bk + kk, s_ * bk + kk + hk
                            if side == "lhs":  # A0 A1 A2 A3 = (top,lo) (top,hi) (bot,lo) (bot,hi)
                                q0, q1, q2, q3 = at(first, lo), at(first, hi), at(second, lo), at(second, hi)
                                ops = [r(q0 + q3), r(q2 + q3), q0, q3, r(q0 + q1), r(q2 - q0), r(q1 - q3)]
                            else:  # B0 B1 B2 B3 = (lo,left) (lo,right) (hi,left) (hi,right)
                                q0, q1, q2, q3 = at(first, lo), at(second, lo), at(first, hi), at(second, hi)
                                ops = [r(q0 + q3), q0, r(q1 - q3), r(q2 - q0), q3, r(q0 + q1), r(q2 + q3)]
                            want.append(ops[op] if algo == 7 else (q0, q1, q2, q3)[op])
                        assert list(got) == want, (ptile, stage, op, block, lane)
    assert pos == flat.size


def test_oracle_packed_cubic_round_trip():
    import numpy as np

    import oracle as o

    rng = np.random.default_rng(2)
    a = o.bf16_round(rng.standard_normal((512, 256)).astype(np.float32))
    planes = o.unpack_operand(o.packed_operand(a, 8, "lhs", 256, 64), 4, 256, 128)
    # Reassemble A from its quadrant planes: plane q = (row half q//2, K half q%2).
    back = np.empty_like(a)
    for q in range(4):
        rh, kh = divmod(q, 2)
        v = planes[q].reshape(2, 128, 4, 32)  # (row tile, row, panel, k)
        for i in range(2):
            for s in range(4):
                back[i * 256 + rh * 128:i * 256 + rh * 128 + 128, s * 64 + kh * 32:s * 64 + kh * 32 + 32] = v[i, :, s, :]
    assert np.array_equal(back, a)


def test_torch_relayouts_match_oracle():
    import numpy as np

    import oracle as o

    w = torch.arange(64 * 1024, dtype=torch.float32).reshape(64, 1024)
    assert np.array_equal(smx.swiglu_weight_layout(w, 256).numpy(), o.swiglu_weight_layout(w.numpy(), 256))
    assert np.array_equal(smx.rope_weight_layout(w, 256).numpy(), o.rope_weight_layout(w.numpy(), 256))
    # K-contiguous weights keep their layout through the permutation.
    wk = w.t().contiguous().t()
    laid = smx.swiglu_weight_layout(wk, 256)
    assert smx.is_k_contiguous(laid)
    assert torch.equal(laid, smx.swiglu_weight_layout(w, 256))
    cos = torch.randn(32, 128)
    sin = torch.randn(32, 128)
    tc, ts = smx.rope_layout_tables(cos, sin, 128)
    oc, os_ = o.rope_layout_tables(cos.numpy(), sin.numpy(), 128)
    assert np.array_equal(tc.numpy(), oc) and np.array_equal(ts.numpy(), os_)
    g = torch.randn(128)
    assert np.array_equal(smx.rope_scale_layout(g, 256).numpy(), o.rope_scale_layout(g.numpy(), 256))
    flat = torch.randn(2 * 4 * 1024).reshape(8, 1024)
    assert np.array_equal(smx.rope_layout_to_heads(flat, 8, 256, 2, 4).numpy(),
                          o.rope_layout_to_heads(flat.numpy(), 8, 256, 2, 4))


@pytest.mark.parametrize("args,kwargs,exc,match", [
    ((t(4), t(4, 4)), {}, ValueError, "expects rank-2 inputs"),
    ((t(512, 256), t(256, 256)), {}, ValueError, "contracting dimensions disagree: 512 vs 256"),
    ((t(512, 256), t(512, 256, dtype=torch.float32)), {}, ValueError, "input dtypes disagree"),
    ((t(512, 256, dtype=torch.float16), t(512, 256, dtype=torch.float16)), {}, ValueError, "BF16 or FP32"),
    ((t(512, 256), t(512, 256)), {"bm": 96}, ValueError, "M=256 is not divisible by 96"),
    ((t(512, 256), t(512, 256)), {"allow_input_fusion": (True,)}, ValueError, "two booleans"),
    ((t(512, 256), t(512, 256)), {"output_dtype": torch.float16}, ValueError, "BF16 or FP32"),
    ((t(512, 256, dtype=torch.float32), t(512, 256, dtype=torch.float32)), {"dot_precision": "HIGHEST"},
     ValueError, "HIP device"),
    ((t(512, 256, dtype=torch.float32), t(512, 256, dtype=torch.float32)), {"dot_precision": "fp64"},
     ValueError, "unknown dot_precision"),
    ((t(512, 256, dtype=torch.float32), t(512, 256, dtype=torch.float32)), {}, ValueError, "HIP device"),
    ((t(512, 256), t(512, 256)), {"interpret": True}, NotImplementedError, "interpret"),
    ((t(512, 256), t(512, 256)), {}, ValueError, "HIP device"),
])
def test_lhs_transposed_surface(args, kwargs, exc, match):
    """strassen_matmul_lhs_transposed's checks (strassen_pallas.py:1250-1267)."""
    kw = dict(bm=256, bn=256, bk=512)
    kw.update(kwargs)
    with pytest.raises(exc, match=match):
        smx.strassen_matmul_lhs_transposed(*args, **kw)


def test_packed_weight_variant_must_match_the_call():
    w = smx.PackedOperand(t(1), algo=7, side="rhs", rows=512, k=512, tile_rows=512, bk=512, formula="dual")
    with pytest.raises(ValueError, match="formula_variant='dual'"):
        smx.strassen_matmul(t(256, 512), w, bm=256, bn=512, bk=512)
    w = smx.PackedOperand(t(1), algo=7, side="rhs", rows=512, k=512, tile_rows=512, bk=512, block_permutation=5)
    with pytest.raises(ValueError, match="block_permutation=5"):
        smx.strassen_matmul(t(256, 512), w, bm=256, bn=512, bk=512, block_permutation=4)
    with pytest.raises(ValueError, match="formula_variant must be"):
        smx.pack_operand(t(512, 512), algo=7, side="rhs", tile_rows=512, bk=512, formula="winograd")


def test_norm_residual_add_surface_checks():
    """strassen_pallas.py:972-985."""
    a, b = t(256, 512), t(512, 256)
    kw = dict(bm=256, bn=256, bk=512, epilogue="norm_residual_add")
    with pytest.raises(ValueError, match="requires residual= and norm_scale="):
        smx.strassen_matmul(a, b, residual=t(256, 256), **kw)
    with pytest.raises(ValueError, match="residual shape"):
        smx.strassen_matmul(a, b, residual=t(128, 256), norm_scale=t(256), **kw)
    with pytest.raises(ValueError, match="norm_scale shape"):
        smx.strassen_matmul(a, b, residual=t(256, 256), norm_scale=t(128), **kw)
    with pytest.raises(ValueError, match="HIP device"):
        smx.strassen_matmul(a, b, residual=t(256, 256), norm_scale=t(256), **kw)


def test_packed_weight_cache_logic():
    """The packed-weight cache (CPU tensors stand in for device weights;
    ``make`` counts packings): disabled by default, hits on a fresh view of
    the same weight, repacks after an in-place update, least-recently used
    eviction by packed bytes, and no entry for an operand above capacity."""
    from strassen_tpu_amd.packing import PackedOperand, _WeightCache

    made = []

    def maker(nbytes):
        def make():
            made.append(nbytes)
            return PackedOperand(torch.empty(nbytes // 2, dtype=torch.bfloat16), algo=7, side="rhs", rows=256,
                                 k=256, tile_rows=256, bk=256)
        return make

    w = torch.zeros(256, 256, dtype=torch.bfloat16)
    off = _WeightCache(0)
    off.lookup(w.t(), ("p",), maker(1000))
    off.lookup(w.t(), ("p",), maker(1000))
    assert len(made) == 2 and not off.entries

    cache = _WeightCache(3000)
    first = cache.lookup(w.t(), ("p",), maker(1000))
    again = cache.lookup(w.t(), ("p",), maker(1000))  # a new view of the same storage
    assert again is first and len(made) == 3 and cache.hits == 1
    cache.lookup(w.t(), ("other tile",), maker(1000))  # another packing of the same weight
    assert len(made) == 4 and cache.bytes == 2000
    w.add_(1)  # in-place update: the version counter moves
    repacked = cache.lookup(w.t(), ("p",), maker(1000))
    assert repacked is not first and cache.stale == 1 and len(made) == 5
    v = torch.ones(256, 256, dtype=torch.bfloat16)
    cache.lookup(v, ("p",), maker(1500))  # 3500 bytes > 3000: the least recently used entry goes
    assert cache.bytes <= 3000 and len(cache.entries) == 2
    cache.lookup(v, ("big",), maker(4000))  # above capacity: packed, not kept
    assert all(key[-1] != ("big",) for key in cache.entries)
    cache.resize(0)
    assert not cache.entries and cache.bytes == 0


def test_cache_packed_weights_api():
    previous = smx.cache_packed_weights(1 << 20)
    try:
        info = smx.packed_weight_cache_info()
        assert info["capacity"] == 1 << 20
        assert set(info) == {"hits", "misses", "stale", "entries", "bytes", "capacity"}
    finally:
        smx.cache_packed_weights(previous)
    assert smx.packed_weight_cache_info()["capacity"] == previous


def test_strassen_kernel_choice():
    """The packed Strassen kernel is chosen per process: the product-major
    kernel on whole rounds by default, or one of the two kernels alone."""
    assert surface.STRASSEN_KERNEL == "product_major_rounds"
    for kind in surface.STRASSEN_KERNELS:
        with smx.strassen_kernel(kind):
            assert surface.STRASSEN_KERNEL == kind
        assert surface.STRASSEN_KERNEL == "product_major_rounds"
    with pytest.raises(ValueError, match="Strassen kernel must be one of"):
        with smx.strassen_kernel("fastest"):
            pass


def test_bench_head_columns():
    """bench.py's head_columns restates the library's pm_round_columns: the
    most 256-column product tiles per tile row that fill whole rounds of the
    CUs and end on a bn tile boundary, none below K = 4096."""
    import bench

    # gate|up at 8 x 1024 tokens on 256 CUs: 32 tile rows, 8 columns a round.
    assert bench.head_columns(8192, 5120, 51200, 1024, 256) == 49152
    assert bench.head_columns(8192, 8192, 5120, 1024, 256) == 4096   # o: one round
    assert bench.head_columns(8192, 25600, 5120, 1024, 256) == 4096  # down
    assert bench.head_columns(8192, 5120, 1024, 1024, 256) == 0      # v: under one round
    assert bench.head_columns(8192, 2048, 51200, 1024, 256) == 0     # K below 4096
    assert bench.head_columns(1024, 4096, 34816, 1024, 256) == 32768
    # bn / 2 = 1024: whole bn tiles of 4 columns; 24 tile rows: 32 a round.
    assert bench.head_columns(6144, 4096, 2 * 256 * 72, 2048, 256) == 2 * 256 * 64
    assert bench.head_columns(8192, 5120, 51200, 1024, 304) == 2 * 256 * 76  # 38 columns a round
