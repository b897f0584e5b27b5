"""The C-ABI library loads and exports every function include/*.h declares;
argument errors come back as status codes without touching the GPU."""

import ctypes
import glob
import os
import re

import pytest

from strassen_tpu_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for header in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(header).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(smx_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_header_declares_expected_entry_points():
    assert set(_lib.EXPORTS) == set(declared_functions())


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_version_and_macros_match_header():
    header = open(os.path.join(ROOT, "include", "strassen_mi355x.h")).read()
    version = int(re.search(r"#define SMX_VERSION (\d+)", header).group(1))
    assert _lib.load().smx_version() == version
    for name in ("SMX_OK", "SMX_ERR_INVALID", "SMX_ERR_UNSUPPORTED", "SMX_ERR_LAUNCH",
                 "SMX_ALGO_STRASSEN", "SMX_ALGO_CUBIC", "SMX_A_ROWMAJOR", "SMX_A_PACKED",
                 "SMX_B_KCONTIG", "SMX_B_PACKED", "SMX_SIDE_LHS", "SMX_SIDE_RHS", "SMX_SIDE_LHS_T",
                 "SMX_FLAG_OUT_F32", "SMX_FLAG_PRODUCT_MAJOR", "SMX_FLAG_PRODUCT_MAJOR_ROUNDS",
                 "SMX_AUX_BIAS_F32", "SMX_AUX_SCALE_F32"):
        value = int(re.search(rf"#define {name} (\d+)", header).group(1))
        assert getattr(_lib, name) == value, name
    for name, code in _lib.SMX_FORMULA.items():
        assert int(re.search(rf"#define SMX_FORMULA_{name.upper()} (\d+)", header).group(1)) == code
    for epi, code in _lib.SMX_EPI.items():
        if epi is not None:
            macro = "SMX_EPI_" + epi.upper()
            assert int(re.search(rf"#define {macro} (\d+)", header).group(1)) == code


def test_descriptor_layout_matches_header_order():
    header = open(os.path.join(ROOT, "include", "strassen_mi355x.h")).read()
    body = re.search(r"typedef struct smx_gemm_desc \{(.*?)\} smx_gemm_desc;", header, re.S).group(1)
    body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
    fields = []
    for line in body.splitlines():
        line = line.strip().rstrip(";")
        if not line:
            continue
        if line.startswith("const "):
            line = line[len("const "):]
        ctype, names = line.split(None, 1)
        if ctype.endswith("*") or names.startswith("*"):  # a device pointer
            ctype, names = "pointer", names.lstrip("*")
        fields += [(n.strip(), ctype) for n in names.split(",")]
    kinds = {"int64_t": ctypes.c_int64, "int32_t": ctypes.c_int32, "float": ctypes.c_float,
             "pointer": ctypes.c_void_p}
    assert [(n, kinds[t]) for n, t in fields] == list(_lib.SmxGemmDesc._fields_)


def _desc(**kw):
    d = _lib.SmxGemmDesc()
    d.m, d.n, d.k = 256, 256, 128
    d.lda, d.ldb, d.ldc, d.ldr = 128, 128, 256, 256
    d.bm, d.bn, d.bk = 256, 256, 128
    d.algo = _lib.SMX_ALGO_STRASSEN
    d.epilogue = 0
    d.a_layout = _lib.SMX_A_ROWMAJOR
    d.b_layout = _lib.SMX_B_KCONTIG
    d.rope_head_dim = 128
    d.rope_eps = 1e-6
    for key, value in kw.items():
        setattr(d, key, value)
    return d


@pytest.mark.parametrize("field,value,code", [
    ("algo", 5, _lib.SMX_ERR_INVALID),
    ("m", 0, _lib.SMX_ERR_INVALID),
    ("bm", 100, _lib.SMX_ERR_INVALID),
    ("bm", 128, _lib.SMX_ERR_UNSUPPORTED),
    ("bn", 64, _lib.SMX_ERR_UNSUPPORTED),
    ("bk", 32, _lib.SMX_ERR_UNSUPPORTED),
    ("b_layout", 0, _lib.SMX_ERR_INVALID),
    ("a_layout", 5, _lib.SMX_ERR_INVALID),
    ("a_layout", _lib.SMX_A_PACKED, _lib.SMX_ERR_UNSUPPORTED),  # packed A needs packed B
    ("b_layout", _lib.SMX_B_PACKED, _lib.SMX_ERR_UNSUPPORTED),  # and vice versa
    ("lda", 100, _lib.SMX_ERR_INVALID),
    ("epilogue", 9, _lib.SMX_ERR_INVALID),
    ("flags", 8, _lib.SMX_ERR_INVALID),
    ("flags", _lib.SMX_FLAG_PRODUCT_MAJOR | _lib.SMX_FLAG_PRODUCT_MAJOR_ROUNDS, _lib.SMX_ERR_INVALID),
    ("formula", 3, _lib.SMX_ERR_INVALID),
    ("block_permutation", 8, _lib.SMX_ERR_INVALID),
    ("formula", 1, _lib.SMX_ERR_UNSUPPORTED),            # variants need packed operands
    ("block_permutation", 2, _lib.SMX_ERR_UNSUPPORTED),
])
def test_invalid_descriptors_are_rejected_before_any_launch(field, value, code):
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 16)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    rc = lib.smx_gemm(_desc(**{field: value}), p, p, p, None, None, None, None, None, None)
    assert rc == code
    assert _lib.last_error()


@pytest.mark.parametrize("fields,code,match", [
    (dict(bm=8), _lib.SMX_ERR_UNSUPPORTED, "bm % 16"),       # below the reference's bm % 16
    (dict(bm=24, m=240), _lib.SMX_ERR_UNSUPPORTED, "bm % 16"),
    (dict(bn=128), _lib.SMX_ERR_UNSUPPORTED, "bn % 256"),
    (dict(bk=32), _lib.SMX_ERR_UNSUPPORTED, "bk % 64"),
    (dict(epilogue=_lib.SMX_EPI["qk_norm_rope"], rope_head_dim=64), _lib.SMX_ERR_UNSUPPORTED, "smx_qk_norm_rope"),
])
def test_packed_tile_rule(fields, code, match):
    """Packed operands take bm % 16 (thin tilings included), bn % 256 and
    bk % 64; the fused q/k epilogue takes head_dim 128 and names the
    two-pass route for other widths."""
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 64)()
    base = ctypes.addressof(buf)
    p = ctypes.c_void_p(base + (-base) % 16)
    kw = dict(a_layout=_lib.SMX_A_PACKED, b_layout=_lib.SMX_B_PACKED)
    kw.update(fields)
    rc = lib.smx_gemm(_desc(**kw), p, p, p, None, None, p, p, p, None)
    assert rc == code
    assert match in _lib.last_error()


@pytest.mark.parametrize("args,match", [
    (dict(m=0), "empty"),
    (dict(head_dim=3), "even head_dim"),
    (dict(head_dim=96), "multiple of 2*head_dim"),   # bn 256 % 192
    (dict(n=384), "not divisible"),
    (dict(ldx=100), "row strides"),
    (dict(dtypes=2), "dtype bits"),
    (dict(bn=16384, n=16384, ldx=16384, ldo=16384), "LDS"),
])
def test_qk_norm_rope_rejects_bad_arguments(args, match):
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    a = dict(m=16, n=512, ldx=512, bn=256, head_dim=64, dtypes=0, ldo=512)
    a.update(args)
    rc = lib.smx_qk_norm_rope(a["m"], a["n"], p, a["ldx"], p, p, p, a["dtypes"], a["bn"], a["head_dim"], 1e-6, p,
                              a["ldo"], None)
    assert rc == _lib.SMX_ERR_INVALID or rc == _lib.SMX_ERR_UNSUPPORTED
    assert match in _lib.last_error()
    assert lib.smx_qk_norm_rope(16, 512, None, 512, p, p, p, 0, 256, 64, 1e-6, p, 512, None) == _lib.SMX_ERR_INVALID


def test_null_pointers_and_missing_epilogue_operands():
    lib = _lib.load()
    assert lib.smx_gemm(None, None, None, None, None, None, None, None, None, None) == _lib.SMX_ERR_INVALID
    buf = (ctypes.c_uint8 * 16)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    assert lib.smx_gemm(_desc(), None, p, p, None, None, None, None, None, None) == _lib.SMX_ERR_INVALID
    rc = lib.smx_gemm(_desc(epilogue=_lib.SMX_EPI["residual_add"]), p, p, p, None, None, None, None, None, None)
    assert rc == _lib.SMX_ERR_INVALID and "residual" in _lib.last_error()
    rc = lib.smx_gemm(_desc(epilogue=_lib.SMX_EPI["qk_norm_rope"]), p, p, p, None, None, None, None, None, None)
    assert rc == _lib.SMX_ERR_INVALID and "rope" in _lib.last_error()


def test_tile_requirements():
    plain = _lib.tile_requirements(_lib.SMX_ALGO_STRASSEN, None, _lib.SMX_B_KCONTIG)
    packed = _lib.tile_requirements(_lib.SMX_ALGO_STRASSEN, None, _lib.SMX_B_PACKED)
    # Both algorithms share each kernel's tiling.
    assert plain == _lib.tile_requirements(_lib.SMX_ALGO_CUBIC, None, _lib.SMX_B_KCONTIG)
    assert packed == _lib.tile_requirements(_lib.SMX_ALGO_CUBIC, None, _lib.SMX_B_PACKED)
    # packed: every bm the reference allows (bm % 16), thin tilings included
    assert packed == (8, 128, 32) and plain == (128, 64, 32)
    with pytest.raises(ValueError):
        _lib.tile_requirements(3, None)
    with pytest.raises(ValueError):
        _lib.tile_requirements(_lib.SMX_ALGO_CUBIC, None, 7)


def test_packed_bytes():
    lib = _lib.load()
    out = ctypes.c_int64()
    assert lib.smx_packed_bytes(7, 512, 256, ctypes.byref(out)) == _lib.SMX_OK
    assert out.value == 256 * 128 * 7 * 2
    assert lib.smx_packed_bytes(8, 512, 256, ctypes.byref(out)) == _lib.SMX_OK
    assert out.value == 512 * 256 * 2
    assert lib.smx_packed_bytes(5, 512, 256, ctypes.byref(out)) == _lib.SMX_ERR_INVALID
    assert lib.smx_packed_bytes(7, 511, 256, ctypes.byref(out)) == _lib.SMX_ERR_INVALID
    # a thin tiling's product rows are padded to whole 128-row tiles
    assert lib.smx_packed_bytes(7, 32, 256, ctypes.byref(out)) == _lib.SMX_OK
    assert out.value == 128 * 128 * 7 * 2
    assert lib.smx_packed_bytes(8, 272 * 2, 256, ctypes.byref(out)) == _lib.SMX_OK
    assert out.value == 384 * 128 * 4 * 2


@pytest.mark.parametrize("args,code", [
    ((7, 0, 0, 512, 512, 256, 512), _lib.SMX_ERR_INVALID),        # rows = 0
    ((7, 0, 512, 512, 512, 256, 500), _lib.SMX_ERR_INVALID),      # k % bk
    ((7, 3, 512, 512, 512, 256, 512), _lib.SMX_ERR_INVALID),      # side
    ((7, 2, 512, 512, 256, 256, 512), _lib.SMX_ERR_INVALID),      # transposed A: ld < rows
    ((6, 0, 512, 512, 512, 256, 512), _lib.SMX_ERR_INVALID),      # algo
    ((7, 0, 480, 512, 512, 24, 512), _lib.SMX_ERR_UNSUPPORTED),   # A: tile_rows % 16
    ((7, 1, 512, 512, 512, 128, 512), _lib.SMX_ERR_UNSUPPORTED),  # B: tile_rows % 256
    ((8, 1, 512, 512, 512, 256, 48), _lib.SMX_ERR_INVALID),       # k % bk
    ((8, 1, 512, 480, 480, 256, 48), _lib.SMX_ERR_UNSUPPORTED),   # bk % 64
    ((7, 0, 512, 480, 480, 256, 96), _lib.SMX_ERR_UNSUPPORTED),   # bk % 64
    ((7, 0, 512, 512, 100, 256, 512), _lib.SMX_ERR_INVALID),      # ld < k
])
def test_pack_operand_rejects_bad_arguments(args, code):
    algo, side, rows, k, ld, tile_rows, bk = args
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 16)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    assert lib.smx_pack_operand(algo, 0, 0, side, rows, k, p, _lib.SMX_DTYPE_BF16, 1, ld, tile_rows, bk, None, 0, p,
                                None) == code
    assert _lib.last_error()


@pytest.mark.parametrize("src_k,ld,code", [
    (0, 1024, _lib.SMX_ERR_INVALID),      # empty source
    (1000, 1024, _lib.SMX_ERR_INVALID),   # source K not a multiple of bk
    (1024, 512, _lib.SMX_ERR_INVALID),    # ld below the source K
])
def test_pack_operand_panel_map_arguments(src_k, ld, code):
    """With a panel map, the source is src_k wide and k is the packed K."""
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 16)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    assert lib.smx_pack_operand(7, 0, 0, 0, 512, 512, p, _lib.SMX_DTYPE_BF16, 1, ld, 256, 512, p, src_k, p, None) == code
    assert "source K" in _lib.last_error() or "ld must be" in _lib.last_error()


@pytest.mark.parametrize("algo,formula,perm", [(7, 3, 0), (7, -1, 0), (7, 0, 8), (8, 1, 0), (8, 0, 2)])
def test_pack_operand_rejects_bad_variants(algo, formula, perm):
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 16)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    assert lib.smx_pack_operand(algo, formula, perm, 0, 512, 512, p, _lib.SMX_DTYPE_BF16, 1, 512, 256, 512, None, 0, p,
                                None) == \
        _lib.SMX_ERR_INVALID


@pytest.mark.parametrize("src_dtype,ld,code", [
    (2, 512, _lib.SMX_ERR_INVALID),                  # unknown source dtype
    (-1, 512, _lib.SMX_ERR_INVALID),
    (_lib.SMX_DTYPE_BF16, 516, _lib.SMX_ERR_INVALID),  # bf16 rows need ld % 8 == 0
    (_lib.SMX_DTYPE_F32, 515, _lib.SMX_ERR_INVALID),   # f32 rows need ld % 4 == 0
])
def test_pack_operand_source_dtype(src_dtype, ld, code):
    """The source is bf16 or float32; its row stride keeps rows 16-byte aligned."""
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 16)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    assert lib.smx_pack_operand(7, 0, 0, 0, 512, 512, p, src_dtype, 1, ld, 256, 512, None, 0, p, None) == code
    assert _lib.last_error()


@pytest.mark.parametrize("src_dtype,passes,k,code", [
    (_lib.SMX_DTYPE_F32, 2, 1536, _lib.SMX_ERR_INVALID),   # passes not 1, 3 or 6
    (_lib.SMX_DTYPE_F32, 0, 1536, _lib.SMX_ERR_INVALID),
    (_lib.SMX_DTYPE_BF16, 3, 1536, _lib.SMX_ERR_INVALID),  # multi-pass needs a float32 source
    (_lib.SMX_DTYPE_F32, 3, 1024, _lib.SMX_ERR_INVALID),   # packed K not whole passes of bk panels
    (_lib.SMX_DTYPE_F32, 6, 1536, _lib.SMX_ERR_INVALID),
])
def test_pack_operand_passes(src_dtype, passes, k, code):
    """Multi-pass packing: 3 or 6 passes of a float32 source; the packed K is
    passes x the source K."""
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 16)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    assert lib.smx_pack_operand(7, 0, 0, 0, 512, k, p, src_dtype, passes, 512, 256, 512, None, 0, p, None) == code
    assert "pass" in _lib.last_error()


def test_powers_refuses_fused_epilogues():
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 16)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    d = _desc(a_layout=_lib.SMX_A_PACKED, b_layout=_lib.SMX_B_PACKED, formula=2,
              epilogue=_lib.SMX_EPI["residual_add"])
    assert lib.smx_gemm(d, p, p, p, p, None, None, None, None, None) == _lib.SMX_ERR_INVALID
    assert "quadrant-basis" in _lib.last_error()


@pytest.mark.parametrize("fields,match", [
    ({"algo": _lib.SMX_ALGO_STRASSEN}, "cubic algorithm only"),
    ({"algo": _lib.SMX_ALGO_CUBIC, "ldp": 100}, "ldp >= N"),
])
def test_partial_product_arguments(fields, match):
    """The FP32 partial (the Strassen half of an exact-panel schedule) is
    added by the cubic kernel only, with a full row stride."""
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 16)()
    p = ctypes.cast(buf, ctypes.c_void_p)
    d = _desc(a_layout=_lib.SMX_A_PACKED, b_layout=_lib.SMX_B_PACKED, **fields)
    d.partial = ctypes.cast(buf, ctypes.c_void_p).value
    if "ldp" not in fields:
        d.ldp = d.n
    assert lib.smx_gemm(d, p, p, p, None, None, None, None, None, None) == _lib.SMX_ERR_INVALID
    assert match in _lib.last_error()


@pytest.mark.parametrize("case,match", [
    ("c_offset", "C rows must be 16-byte aligned"),
    ("ldc", "C rows must be 16-byte aligned"),
    ("ldc_f32", "C rows must be 16-byte aligned"),
    ("residual_offset", "residual rows must be 16-byte aligned"),
    ("ldr", "residual rows must be 16-byte aligned"),
    ("partial_offset", "16-byte alignment"),
    ("ldp", "ldp % 4"),
])
def test_epilogue_rows_are_16_byte_aligned(case, match):
    """The epilogue moves output, residual and partial rows in 16-byte
    chunks: their base pointers and row strides must keep rows 16-byte
    aligned (checked before any launch)."""
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 256)()
    base = (ctypes.addressof(buf) + 15) & ~15
    good, odd = ctypes.c_void_p(base), ctypes.c_void_p(base + 4)
    c, residual = good, None
    d = _desc()
    if case == "c_offset":
        c = odd
    elif case == "ldc":
        d.ldc = 260
    elif case == "ldc_f32":
        d.flags, d.ldc = _lib.SMX_FLAG_OUT_F32, 258
    elif case in ("residual_offset", "ldr"):
        d.epilogue = _lib.SMX_EPI["residual_add"]
        residual = odd if case == "residual_offset" else good
        if case == "ldr":
            d.ldr = 260
    else:
        d = _desc(algo=_lib.SMX_ALGO_CUBIC, a_layout=_lib.SMX_A_PACKED, b_layout=_lib.SMX_B_PACKED)
        d.partial = base + 4 if case == "partial_offset" else base
        d.ldp = 256 if case == "partial_offset" else 258
    assert lib.smx_gemm(d, good, good, c, residual, None, None, None, None, None) == _lib.SMX_ERR_INVALID
    assert match in _lib.last_error()


@pytest.mark.parametrize("odd_arg", ["rope_cos", "rope_sin", "rope_scale"])
def test_qk_tables_and_scale_are_16_byte_aligned(odd_arg):
    """The q/k epilogue reads the RoPE tables and the per-column scale eight
    values (16 bytes) at a time: a misaligned pointer to any of them is
    refused before any launch."""
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 256)()
    base = (ctypes.addressof(buf) + 15) & ~15
    good, odd = ctypes.c_void_p(base), ctypes.c_void_p(base + 2)
    rope = {"rope_cos": good, "rope_sin": good, "rope_scale": good}
    rope[odd_arg] = odd
    d = _desc(epilogue=_lib.SMX_EPI["qk_norm_rope"])
    rc = lib.smx_gemm(d, good, good, good, None, None, rope["rope_cos"], rope["rope_sin"], rope["rope_scale"], None)
    assert rc == _lib.SMX_ERR_INVALID
    assert "must be 16-byte aligned" in _lib.last_error() and "rope_scale" in _lib.last_error()


def test_workspace_arguments():
    """The tail-split workspace: a misaligned pointer or a negative size is
    refused before any launch, as is every descriptor smx_gemm refuses; an
    unpacked call never needs one (both answered without a device)."""
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 64)()
    base = ctypes.addressof(buf)
    p = ctypes.c_void_p(base + (-base) % 16)
    for fields in (dict(workspace=p.value + 4, workspace_bytes=1 << 20), dict(workspace=p.value, workspace_bytes=-1)):
        assert lib.smx_gemm(_desc(**fields), p, p, p, None, None, None, None, None, None) == _lib.SMX_ERR_INVALID
        assert "workspace" in _lib.last_error()
    need = ctypes.c_int64(-1)
    assert lib.smx_gemm_workspace_bytes(_desc(k=4096, lda=4096, ldb=4096), ctypes.byref(need)) == _lib.SMX_OK
    assert need.value == 0
    assert lib.smx_gemm_workspace_bytes(_desc(bm=100), ctypes.byref(need)) == _lib.SMX_ERR_INVALID
    assert lib.smx_gemm_workspace_bytes(None, ctypes.byref(need)) == _lib.SMX_ERR_INVALID
    assert lib.smx_gemm_workspace_bytes(_desc(), None) == _lib.SMX_ERR_INVALID


def test_inline_asm_kernel_check():
    """The build refuses device code that touches MFMA accumulators between
    the first inline-asm MFMA and the drain."""
    from strassen_tpu_amd import build

    drain = "\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n"
    ok = ("_ZN3smx2v27gemm_v2ILi7ELi0EEEvNS_6ParamsE: ; @x\n\tscratch_store_dword off, v1, off\n"
          "\t;;#ASMSTART\n\tv_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]\n\t;;#ASMEND\n" + drain +
          "\tv_accvgpr_read_b32 v0, a0\n\ts_endpgm\n")
    builtin = ("_ZN3smx2v27gemm_v2ILi8ELi0EEEvNS_6ParamsE:\n"
               "\tv_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]\n\tv_accvgpr_read_b32 v0, a0\n"
               "\ts_endpgm\n")
    assert build.verify_inline_asm_kernels(ok) == 1
    assert build.verify_inline_asm_kernels(ok + builtin) == 1  # builtin MFMAs are the compiler's business
    no_drain = ok.replace(drain, "")
    with pytest.raises(RuntimeError, match="without the drain"):
        build.verify_inline_asm_kernels(no_drain)
    for bad in ("\tv_accvgpr_read_b32 v0, a0\n", "\tscratch_store_dwordx4 off, v[0:3], off\n",
                "\tv_accvgpr_mov_b32 a1, a0\n"):
        text = ok.replace(drain, bad + drain)
        with pytest.raises(RuntimeError, match="before the MFMA drain"):
            build.verify_inline_asm_kernels(text)
    with pytest.raises(RuntimeError):
        build.verify_inline_asm_kernels("no kernels here")
    # a wave that ends early does not hide another wave's MFMA loop
    early = ok.replace("; @x\n", "; @x\n\ts_cbranch_scc1 .LBB0_2\n\ts_endpgm\n.LBB0_2:\n")
    assert build.verify_inline_asm_kernels(early) == 1
    with pytest.raises(RuntimeError, match="before the MFMA drain"):
        build.verify_inline_asm_kernels(early.replace(drain, "\tv_accvgpr_read_b32 v0, a0\n" + drain))


def test_kernel_scratch_check():
    """The build refuses GEMM kernels whose registers spill to scratch."""
    from strassen_tpu_amd import build

    def desc(name, size):
        return (f"\t.amdhsa_kernel {name}\n\t\t.amdhsa_group_segment_fixed_size 0\n"
                f"\t\t.amdhsa_private_segment_fixed_size {size}\n\t.end_amdhsa_kernel\n")

    split_swiglu = "_ZN3smx5split10gemm_splitILi1ELi2ELb0EEEvNS_6ParamsE"
    split_qk = "_ZN3smx5split10gemm_splitILi4ELi2ELb0EEEvNS_6ParamsE"
    thin_swiglu = "_ZN3smx5split10gemm_splitILi1ELi2ELb1EEEvNS_6ParamsE"
    thin_qk = "_ZN3smx5split10gemm_splitILi4ELi2ELb1EEEvNS_6ParamsE"
    cubic = "_ZN3smx6packed11gemm_packedILi8ELi2ELi0ELi3ELb0EEEvNS_6ParamsE"
    cubic_partial = "_ZN3smx6packed11gemm_packedILi8ELi2ELi1ELi3ELb0EEEvNS_6ParamsE"
    thin_cubic = "_ZN3smx6packed11gemm_packedILi8ELi2ELi0ELi3ELb1EEEvNS_6ParamsE"
    other = "_ZN3smx6packed9pack_rowsILi7ELi0EEEvPKtlliiiiPKiiPh"
    assert build.scratch_limit(split_swiglu) == 0
    assert build.scratch_limit(split_qk) == 0
    assert build.scratch_limit(thin_swiglu) == 0
    assert build.scratch_limit(thin_qk) == 0
    assert build.scratch_limit(cubic) == 0
    assert build.scratch_limit(cubic_partial) == build.PARTIAL_SCRATCH_CAP
    assert build.scratch_limit(thin_cubic) == 0
    assert build.scratch_limit(other) is None
    clean = (desc(split_swiglu, 0) + desc(split_qk, 0) + desc(thin_qk, 0) + desc(cubic, 0)
             + desc(cubic_partial, 792) + desc(other, 64))
    assert build.verify_kernel_scratch(clean) == 5
    for name, size in ((split_swiglu, 8), (split_qk, 4), (thin_swiglu, 4),
                       (thin_qk, 4), (cubic, 4), (thin_cubic, 4),
                       (cubic_partial, build.PARTIAL_SCRATCH_CAP + 4)):
        with pytest.raises(RuntimeError, match="scratch per lane"):
            build.verify_kernel_scratch(clean + desc(name, size))
    assert build.verify_kernel_scratch(desc(other, 0), require=False) == 0
    with pytest.raises(RuntimeError, match="no GEMM kernel"):
        build.verify_kernel_scratch(desc(other, 0))


def test_noalloc_entry_point_rejects_before_any_launch():
    """smx_gemm_noalloc checks its descriptor (the smx_gemm checks, on the
    packed call it will make) and the scratch limit before touching the
    device: every case here fails without a GPU."""
    lib = _lib.load()
    buf = (ctypes.c_uint8 * 4096)()
    base = ctypes.addressof(buf)
    p = ctypes.c_void_p(base + (-base) % 256)
    ok = dict(m=512, n=512, k=512, lda=512, ldc=512, bm=512, bn=512, bk=512, a_layout=_lib.SMX_A_ROWMAJOR,
              b_layout=_lib.SMX_B_PACKED)

    def call(**kw):
        fields = dict(ok)
        fields.update(kw)
        return lib.smx_gemm_noalloc(_desc(**fields), p, p, p, None, None, None, None, None, None)

    assert call(b_layout=_lib.SMX_B_KCONTIG) == _lib.SMX_ERR_INVALID
    assert "row-major bf16 A" in _lib.last_error()
    assert call(a_layout=_lib.SMX_A_PACKED) == _lib.SMX_ERR_INVALID
    d = _desc(**ok)
    d.partial, d.ldp = p.value, 512
    assert lib.smx_gemm_noalloc(d, p, p, p, None, None, None, None, None, None) == _lib.SMX_ERR_UNSUPPORTED
    assert "partial" in _lib.last_error()
    assert call(bn=128) == _lib.SMX_ERR_UNSUPPORTED            # the packed kernel's tile rule
    assert call(bm=8) == _lib.SMX_ERR_UNSUPPORTED
    assert call(epilogue=_lib.SMX_EPI["residual_add"]) == _lib.SMX_ERR_INVALID
    assert call(lda=500) == _lib.SMX_ERR_INVALID
    assert "lda" in _lib.last_error()
    assert lib.smx_gemm_noalloc(_desc(**ok), None, p, p, None, None, None, None, None, None) == _lib.SMX_ERR_INVALID
    # the scratch limit: M*K beyond 256 MiB of packed Strassen operand sums
    limit = _lib.NOALLOC_SCRATCH_BYTES
    m, k = 16384, 5120  # 16384 * 5120 * 3.5 bytes > 256 MiB
    assert m * k * 7 // 2 > limit
    assert call(m=m, k=k, lda=k, bm=1024, bn=512, bk=512) == _lib.SMX_ERR_UNSUPPORTED
    assert "scratch" in _lib.last_error() and str(limit) in _lib.last_error()
    # the cubic's four quadrants fit where Strassen's seven operand sums do not
    assert m * k * 2 <= limit
