"""The allocation-free entry point smx_gemm_noalloc on the GPU, through the
C ABI: its result equals that of the existing path it replaces for callers
that cannot allocate (smx_pack_operand of A into a caller buffer, then
smx_gemm), bit for bit, for the Strassen and the cubic algorithm, on calls in
a row that each get smaller (the device scratch keeps the previous call's
contents), the last on a thin tiling. Named to be collected after every other
test."""

import ctypes

import pytest
import torch

from strassen_tpu_amd import _lib

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def say(*args):
    print(*args, flush=True)


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)


def pack(lib, algo, side, x, tile_rows, bk):
    """x: row-major bf16 [rows, k] on the device -> its packed form."""
    rows, k = x.shape
    nbytes = ctypes.c_int64()
    _lib.check(lib.smx_packed_bytes(algo, rows, k, ctypes.byref(nbytes)))
    out = torch.empty(nbytes.value // 2, dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.smx_pack_operand(algo, 0, 0, side, rows, k, _lib.ptr(x), _lib.SMX_DTYPE_BF16, 1, k, tile_rows, bk,
                                    None, 0, _lib.ptr(out), stream()))
    return out


def desc(m, n, k, tile, algo, epilogue, a_layout):
    d = _lib.SmxGemmDesc()
    d.m, d.n, d.k = m, n, k
    d.bm, d.bn, d.bk = tile
    d.lda = k
    d.ldc = n // 2 if epilogue in ("swiglu", "geglu") else n
    d.ldr = n
    d.algo, d.epilogue = algo, _lib.SMX_EPI[epilogue]
    d.a_layout, d.b_layout = a_layout, _lib.SMX_B_PACKED
    d.rope_head_dim, d.rope_eps = 128, 1e-6
    return d


def compare(lib, algo, m, n, k, tile, epilogue, seed):
    say(f"  smx_gemm_noalloc algo={algo} m={m} n={n} k={k} tile={tile} epilogue={epilogue}")
    g = torch.Generator(device=DEV).manual_seed(seed)
    a = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    bt = (torch.randn(n, k, device=DEV, generator=g) * 0.02).to(torch.bfloat16)  # B^T, row-major
    residual = torch.randn(m, n, device=DEV, generator=g).to(torch.bfloat16) if epilogue == "residual_add" else None
    bm, bn, bk = tile
    b_packed = pack(lib, algo, _lib.SMX_SIDE_RHS, bt, bn, bk)
    d = desc(m, n, k, tile, algo, epilogue, _lib.SMX_A_ROWMAJOR)
    got = torch.full((m, d.ldc), float("nan"), dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.smx_gemm_noalloc(d, _lib.ptr(a), _lib.ptr(b_packed), _lib.ptr(got), _lib.ptr(residual), None, None,
                                    None, None, stream()))
    a_packed = pack(lib, algo, _lib.SMX_SIDE_LHS, a, bm, bk)
    want = torch.full_like(got, float("nan"))
    _lib.check(lib.smx_gemm(desc(m, n, k, tile, algo, epilogue, _lib.SMX_A_PACKED), _lib.ptr(a_packed),
                            _lib.ptr(b_packed), _lib.ptr(want), _lib.ptr(residual), None, None, None, None, stream()))
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, want)
    # a sanity bound against FP32: the entry point computes the GEMM asked for
    ref = torch.matmul(a.float(), bt.float().t())
    if epilogue == "swiglu":
        # gate and up are the left and right halves of every bn-wide tile
        pairs = ref.view(m, n // bn, 2, bn // 2)
        ref = (torch.nn.functional.silu(pairs[:, :, 0]) * pairs[:, :, 1]).reshape(m, n // 2)
    elif epilogue == "residual_add":
        ref = ref + residual.float()
    err = float(torch.linalg.norm(got.float() - ref) / torch.linalg.norm(ref))
    say(f"    bit-identical to smx_gemm; rel err vs FP32 {err:.3e}")
    assert err <= 1e-2


@pytest.mark.parametrize("algo", [_lib.SMX_ALGO_STRASSEN, _lib.SMX_ALGO_CUBIC])
def test_noalloc_matches_existing_entry_point(algo):
    lib = _lib.load()
    compare(lib, algo, 2048, 2048, 2048, (1024, 1024, 512), "swiglu", seed=1)
    compare(lib, algo, 512, 1024, 1024, (512, 512, 512), "residual_add", seed=2)
    compare(lib, algo, 256, 512, 512, (256, 256, 512), None, seed=3)
    # a thin tiling (bm = 16): the packed A is zero-padded to a whole
    # 128-row product tile inside the scratch, and only real rows are stored
    compare(lib, algo, 48, 512, 512, (16, 256, 512), "residual_add", seed=4)


def test_noalloc_refuses_calls_beyond_its_scratch():
    lib = _lib.load()
    m, k, n = 16384, 5120, 512
    d = desc(m, n, k, (1024, 512, 512), _lib.SMX_ALGO_STRASSEN, None, _lib.SMX_A_ROWMAJOR)
    a = torch.empty(16, device=DEV, dtype=torch.bfloat16)  # never read: the call is refused first
    rc = lib.smx_gemm_noalloc(d, _lib.ptr(a), _lib.ptr(a), _lib.ptr(a), None, None, None, None, None, stream())
    assert rc == _lib.SMX_ERR_UNSUPPORTED
    assert "scratch" in _lib.last_error()


def workspace_bytes(lib, d):
    need = ctypes.c_int64()
    _lib.check(lib.smx_gemm_workspace_bytes(d, ctypes.byref(need)))
    return need.value


@pytest.mark.parametrize("flags,shape,tile", [
    (0, (2048, 4096, 2048), (256, 512, 512)),
    (_lib.SMX_FLAG_PRODUCT_MAJOR, (2048, 4096, 2048), (256, 512, 512)),
    # a head of one round of product-major tiles (4 rows x 64 columns on 256
    # CUs), then the split kernel's 32 tiles split over K
    (_lib.SMX_FLAG_PRODUCT_MAJOR_ROUNDS, (1024, 34816, 4096), (1024, 1024, 512)),
])
def test_noalloc_with_the_workspace_it_asks_for(flags, shape, tile):
    """smx_gemm_workspace_bytes sizes the noalloc descriptor (row-major A,
    packed B) as the packed call it becomes: a launch of 128 product tiles
    split over K (flags 0), the product-major kernel's parked sets, or both
    (a product-major head and a split rest). With that workspace the result
    is bit-identical to smx_gemm with the same workspace; with 16 bytes less
    the call is refused before anything is launched (the output keeps its
    NaNs)."""
    lib = _lib.load()
    algo, (m, n, k) = _lib.SMX_ALGO_STRASSEN, shape
    g = torch.Generator(device=DEV).manual_seed(11)
    a = torch.randn(m, k, device=DEV, generator=g).to(torch.bfloat16)
    bt = (torch.randn(n, k, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
    b_packed = pack(lib, algo, _lib.SMX_SIDE_RHS, bt, tile[1], tile[2])
    d = desc(m, n, k, tile, algo, None, _lib.SMX_A_ROWMAJOR)
    d.flags = flags
    need = workspace_bytes(lib, d)
    dp = desc(m, n, k, tile, algo, None, _lib.SMX_A_PACKED)
    dp.flags = flags
    assert need > 0 and need == workspace_bytes(lib, dp)
    say(f"  smx_gemm_noalloc flags={flags} workspace={need}")
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    got = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    d.workspace, d.workspace_bytes = ws.data_ptr(), need - 16
    rc = lib.smx_gemm_noalloc(d, _lib.ptr(a), _lib.ptr(b_packed), _lib.ptr(got), None, None, None, None, None,
                              stream())
    torch.cuda.synchronize()
    assert rc == _lib.SMX_ERR_INVALID and "workspace" in _lib.last_error()
    assert torch.isnan(got.float()).all()
    d.workspace_bytes = need
    _lib.check(lib.smx_gemm_noalloc(d, _lib.ptr(a), _lib.ptr(b_packed), _lib.ptr(got), None, None, None, None, None,
                                    stream()))
    a_packed = pack(lib, algo, _lib.SMX_SIDE_LHS, a, tile[0], tile[2])
    ws2 = torch.empty(need, dtype=torch.uint8, device=DEV)
    dp.workspace, dp.workspace_bytes = ws2.data_ptr(), need
    want = torch.full_like(got, float("nan"))
    _lib.check(lib.smx_gemm(dp, _lib.ptr(a_packed), _lib.ptr(b_packed), _lib.ptr(want), None, None, None, None, None,
                            stream()))
    torch.cuda.synchronize()
    assert torch.isfinite(got.float()).all()
    assert torch.equal(got, want)
