"""ctypes binding of ``libstrassen_mi355x.so`` (the C ABI in
``include/strassen_mi355x.h``).

The library links the HIP runtime by SONAME ``libamdhip64.so.7``; importing
torch first makes it bind to the runtime torch already loaded, so both share
one HIP context and torch's streams are valid handles here.
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (load torch's HIP runtime before the library)

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libstrassen_mi355x.so")

SMX_OK = 0
SMX_ERR_INVALID = 1
SMX_ERR_UNSUPPORTED = 2
SMX_ERR_LAUNCH = 3

SMX_ALGO_STRASSEN = 7
SMX_ALGO_CUBIC = 8

SMX_EPI = {
    None: 0,
    "swiglu": 1,
    "residual_add": 2,
    "bias_add": 3,
    "qk_norm_rope": 4,
    "geglu": 5,
}

SMX_A_ROWMAJOR = 0
SMX_A_PACKED = 1
SMX_B_KCONTIG = 1
SMX_B_PACKED = 2
SMX_SIDE_LHS = 0
SMX_SIDE_RHS = 1
SMX_SIDE_LHS_T = 2
SMX_FLAG_OUT_F32 = 1
SMX_FLAG_PRODUCT_MAJOR = 2
SMX_FLAG_PRODUCT_MAJOR_ROUNDS = 4
SMX_FORMULA = {"classical": 0, "dual": 1, "powers": 2}
SMX_AUX_BIAS_F32 = 1
SMX_AUX_SCALE_F32 = 2
SMX_AUX_RESIDUAL_F32 = 4
# Largest packed activation smx_gemm_noalloc stages in its device scratch.
NOALLOC_SCRATCH_BYTES = 256 << 20

SMX_DTYPE_BF16 = 0
SMX_DTYPE_F32 = 1
SMX_NRA_SCALE_F32 = 1
SMX_NRA_RESIDUAL_F32 = 2
SMX_NRA_OUT_F32 = 4
SMX_QK_SCALE_F32 = 1
SMX_QK_OUT_F32 = 4

EXPORTS = ("smx_gemm", "smx_gemm_noalloc", "smx_gemm_workspace_bytes", "smx_tile_requirements", "smx_packed_bytes", "smx_pack_operand",
           "smx_norm_residual_add", "smx_qk_norm_rope", "smx_last_error", "smx_version")


class SmxGemmDesc(ctypes.Structure):
    _fields_ = [
        ("m", ctypes.c_int64), ("n", ctypes.c_int64), ("k", ctypes.c_int64),
        ("lda", ctypes.c_int64), ("ldb", ctypes.c_int64), ("ldc", ctypes.c_int64),
        ("ldr", ctypes.c_int64),
        ("bm", ctypes.c_int32), ("bn", ctypes.c_int32), ("bk", ctypes.c_int32),
        ("algo", ctypes.c_int32), ("epilogue", ctypes.c_int32),
        ("a_layout", ctypes.c_int32), ("b_layout", ctypes.c_int32),
        ("rope_head_dim", ctypes.c_int32),
        ("rope_eps", ctypes.c_float), ("aux_f32", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("formula", ctypes.c_int32), ("block_permutation", ctypes.c_int32),
        ("partial", ctypes.c_void_p), ("ldp", ctypes.c_int64),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
    ]


_lib = None


def load():
    """Load the built library, or raise: there is no fallback path."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY):
        raise RuntimeError(
            f"{LIBRARY} is missing: build it with `python -m strassen_tpu_amd.build` "
            "(the Strassen GEMM has no CPU or fallback implementation)")
    lib = ctypes.CDLL(LIBRARY)
    vp = ctypes.c_void_p
    lib.smx_gemm.argtypes = [ctypes.POINTER(SmxGemmDesc), vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.smx_gemm.restype = ctypes.c_int
    lib.smx_gemm_noalloc.argtypes = [ctypes.POINTER(SmxGemmDesc), vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.smx_gemm_noalloc.restype = ctypes.c_int
    lib.smx_gemm_workspace_bytes.argtypes = [ctypes.POINTER(SmxGemmDesc), ctypes.POINTER(ctypes.c_int64)]
    lib.smx_gemm_workspace_bytes.restype = ctypes.c_int
    lib.smx_tile_requirements.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                          ctypes.POINTER(ctypes.c_int32),
                                          ctypes.POINTER(ctypes.c_int32),
                                          ctypes.POINTER(ctypes.c_int32)]
    lib.smx_tile_requirements.restype = ctypes.c_int
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    lib.smx_packed_bytes.argtypes = [i32, i64, i64, ctypes.POINTER(i64)]
    lib.smx_packed_bytes.restype = ctypes.c_int
    lib.smx_pack_operand.argtypes = [i32, i32, i32, i32, i64, i64, vp, i32, i32, i64, i32, i32, vp, i64, vp, vp]
    lib.smx_pack_operand.restype = ctypes.c_int
    f32 = ctypes.c_float
    lib.smx_norm_residual_add.argtypes = [i64, i64, vp, i64, vp, i64, vp, i32, f32, vp, i64, vp]
    lib.smx_norm_residual_add.restype = ctypes.c_int
    lib.smx_qk_norm_rope.argtypes = [i64, i64, vp, i64, vp, vp, vp, i32, i32, i32, f32, vp, i64, vp]
    lib.smx_qk_norm_rope.restype = ctypes.c_int
    lib.smx_last_error.argtypes = []
    lib.smx_last_error.restype = ctypes.c_char_p
    lib.smx_version.argtypes = []
    lib.smx_version.restype = ctypes.c_int
    _lib = lib
    return lib


def last_error():
    return load().smx_last_error().decode("utf-8", "replace")


def tile_requirements(algo, epilogue, b_layout=SMX_B_KCONTIG):
    lib = load()
    tm, tn, tk = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    rc = lib.smx_tile_requirements(algo, SMX_EPI[epilogue], b_layout, 0,
                                   ctypes.byref(tm), ctypes.byref(tn), ctypes.byref(tk))
    if rc != SMX_OK:
        raise ValueError(last_error())
    return tm.value, tn.value, tk.value


def check(rc):
    if rc == SMX_OK:
        return
    message = last_error()
    if rc in (SMX_ERR_INVALID, SMX_ERR_UNSUPPORTED):
        raise ValueError(message)
    raise RuntimeError(message)


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def k_shares(m, k, n, tile, algo=SMX_ALGO_STRASSEN):
    """K shares smx_gemm gives the split tiles of a packed (m, k, n) launch
    on the current device (1: no split), from smx_gemm_workspace_bytes."""
    lib = load()
    d = SmxGemmDesc()
    d.m, d.n, d.k = m, n, k
    d.lda, d.ldb, d.ldc = k, k, n
    d.bm, d.bn, d.bk = tile
    d.algo = algo
    d.a_layout, d.b_layout = SMX_A_PACKED, SMX_B_PACKED
    d.rope_head_dim, d.rope_eps = 128, 1e-6
    need = ctypes.c_int64()
    check(lib.smx_gemm_workspace_bytes(d, ctypes.byref(need)))
    if not need.value:
        return 1
    # The workspace holds one 256 x 256 FP32 block per share and split tile;
    # the split tiles are the last round's (128 x 128 product tiles, one per CU
    # and round).
    cus = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    tiles = -(-(m // 2) // 128) * ((n // 2) // 128)
    split = tiles % cus or cus
    return need.value // (split * 256 * 256 * 4)
