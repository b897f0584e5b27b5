"""GPU parity of the K splits of packed launches.

A packed launch runs one 128 x 128 product tile per CU per round: T tiles on
C CUs make T / C whole rounds and a last round of r = T mod C tiles. Given a
workspace (and K >= 2048), smx_gemm runs those r tiles (every tile of a
launch under one round) as s K shares, s chosen so that the s r workgroups
finish soonest, after the whole rounds with the fused epilogue. The shares
go into the FP32 workspace and a pass sums them and applies the epilogue
(strassen_pallas.py:739-879), thin tilings included. strassen_matmul /
cubic_matmul pass a workspace whenever the library asks for one. Checked
against the oracle and against the same call without a workspace (every tile
over full K): the two differ only in the order of FP32 additions, so they
agree within one bf16 ulp and are almost all bit-identical.

Shapes: with bm = bn = 256 a launch has (M / 256) (N / 256) tiles; on the
256 CUs of an MI355X, 2048 x 4096 is 128 tiles (every tile in two shares) and
3072 x 8192 is 384 (one whole round, then 128 tiles in two shares).
"""

import ctypes
import os

import numpy as np
import pytest
import torch

import oracle as o
import strassen_tpu_amd as smx
from strassen_tpu_amd import _lib
from test_gpu_parity import DEV, _qk_problem, assert_ulp_close, dev, dev32, dev_weight, host, say

pytestmark = pytest.mark.gpu

TILE = (256, 256, 512)
HALF_ROUND = (2048, 2048, 4096)      # m, k, n: 128 tiles
ROUND_AND_HALF = (3072, 2048, 8192)  # 384 tiles


@pytest.fixture(autouse=True)
def _announce(request):
    say(f"\n[gpu] {request.node.nodeid}")
    yield
    torch.cuda.synchronize()


# Workspace of one K share of one split tile: its 256 x 256 FP32 outputs.
SPLIT_TILE_BYTES = 256 * 256 * 4


def _workspace_bytes(m, n, k, bm=256):
    """The workspace the library asks for: s shares of the r split tiles."""
    _, split, s = _plan(m, n, k, bm)
    return s * split * SPLIT_TILE_BYTES if split else 0


def _plan(m, n, k, bm=256):
    """(whole tiles, split tiles, shares) of the library's rule, restated:
    the last round's r tiles (all T of a launch under one round) split into
    the s <= min(16, K / 512, 2^30 / (r 256 KB)) shares that minimise
    ceil(s r / C) (1/s + f) + s r g (f = 400 / K, g = (5/3) / K), when that
    is under 0.95 of the unsplit 1 + f. SMX_TAIL_SPLIT starting with 0 in
    the environment turns the split off."""
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    tiles = -(-(m // 2) // 128) * (n // 256)
    r = tiles % cus
    if os.environ.get("SMX_TAIL_SPLIT", "").startswith("0") or k < 2048 or r == 0:
        return tiles, 0, 1
    s_max = min(16, (k // 32) // 16, (1 << 30) // (r * SPLIT_TILE_BYTES))

    def cost(s):
        f, g = 400.0 / k, (5.0 / 3.0) / k
        return ((s * r + cus - 1) // cus) * (1.0 / s + f) + (s * r) * g

    best_s, best = 1, 0.95 * cost(1)
    for s in range(2, s_max + 1):
        if cost(s) < best:
            best_s, best = s, cost(s)
    return (tiles - r, r, best_s) if best_s > 1 else (tiles, 0, 1)


def _split_tiles(m, n, k, bm=256):
    return _plan(m, n, k, bm)[1]


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream(DEV).cuda_stream)


def _problem(seed, m, k, n):
    rng = np.random.default_rng(seed)
    a = o.bf16_round(rng.standard_normal((m, k)).astype(np.float32))
    b = o.bf16_round((rng.standard_normal((k, n)) * 0.05).astype(np.float32))
    return rng, a, b


def _pack(algo, a, b, tile, formula="classical", block_permutation=0):
    bm, bn, bk = tile
    variant = dict(formula=formula, block_permutation=block_permutation)
    pa = smx.packing.pack_operand(dev(a), algo=algo, side="lhs", tile_rows=bm, bk=bk, **variant)
    pb = smx.packing.pack_operand(dev_weight(b), algo=algo, side="rhs", tile_rows=bn, bk=bk, **variant)
    return pa, pb


def abi_gemm(algo, pa, pb, m, n, k, tile, epilogue=None, *, workspace, out_f32=False, residual=None, bias=None,
             rope=None, formula=0, block_permutation=0, workspace_bytes=None, keep_workspace=False):
    """smx_gemm on packed operands, with the workspace the library asks for
    (workspace=True) or none. Returns (output, bytes asked for), and with
    keep_workspace the workspace too, filled with 0xff bytes before the call
    (a NaN in every float)."""
    lib = _lib.load()
    d = _lib.SmxGemmDesc()
    d.m, d.n, d.k = m, n, k
    d.lda, d.ldb = k, k
    d.ldc = n // 2 if epilogue in ("swiglu", "geglu") else n
    d.bm, d.bn, d.bk = tile
    d.algo, d.epilogue = algo, _lib.SMX_EPI[epilogue]
    d.a_layout, d.b_layout = _lib.SMX_A_PACKED, _lib.SMX_B_PACKED
    d.flags = _lib.SMX_FLAG_OUT_F32 if out_f32 else 0
    d.formula, d.block_permutation = formula, block_permutation
    d.rope_head_dim, d.rope_eps = 128, 1e-6
    aux = 0
    cos = sin = scale = None
    if residual is not None:
        d.ldr = residual.stride(0)
        aux |= _lib.SMX_AUX_RESIDUAL_F32 if residual.dtype == torch.float32 else 0
    if bias is not None:
        aux |= _lib.SMX_AUX_BIAS_F32 if bias.dtype == torch.float32 else 0
    if rope is not None:
        cos, sin, scale = rope
        aux |= _lib.SMX_AUX_SCALE_F32 if scale.dtype == torch.float32 else 0
    d.aux_f32 = aux
    need = ctypes.c_int64()
    _lib.check(lib.smx_gemm_workspace_bytes(d, ctypes.byref(need)))
    ws = None
    if workspace and need.value:
        nbytes = need.value if workspace_bytes is None else workspace_bytes
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=DEV)
        if keep_workspace:
            ws.fill_(0xFF)
        d.workspace, d.workspace_bytes = ws.data_ptr(), nbytes
    out = torch.full((m, d.ldc), float("nan"), dtype=torch.float32 if out_f32 else torch.bfloat16, device=DEV)
    say(f"  smx_gemm algo={algo} m={m} n={n} k={k} tile={tile} epilogue={epilogue} workspace={need.value if ws is not None else 0}")
    _lib.check(lib.smx_gemm(d, _lib.ptr(pa.data), _lib.ptr(pb.data), _lib.ptr(out), _lib.ptr(residual), _lib.ptr(bias),
                            _lib.ptr(cos), _lib.ptr(sin), _lib.ptr(scale), _stream()))
    torch.cuda.synchronize()
    return (out, need.value, ws) if keep_workspace else (out, need.value)


def _aux(rng, epilogue, m, n):
    if epilogue == "residual_add":
        return dict(residual=o.bf16_round(rng.standard_normal((m, n)).astype(np.float32)))
    if epilogue == "bias_add":
        return dict(bias=o.bf16_round(rng.standard_normal(n).astype(np.float32)))
    return {}


def _oracle(algo, a, b, tile, **kw):
    bm, bn, bk = tile
    fn = o.strassen_matmul if algo == 7 else o.cubic_blocked_matmul
    return fn(a, b, bm=bm, bn=bn, bk=bk, **kw)


@pytest.mark.parametrize("epilogue", [None, "swiglu", "geglu", "residual_add", "bias_add"])
@pytest.mark.parametrize("algo", [7, 8])
def test_half_round_split_matches_whole_and_oracle(algo, epilogue):
    m, k, n = HALF_ROUND
    if not _split_tiles(m, n, k):
        pytest.skip("no split at this shape: this device's CU count leaves no half-empty round, or SMX_TAIL_SPLIT=0")
    rng, a, b = _problem(61 + algo, m, k, n)
    aux = _aux(rng, epilogue, m, n)
    aux_dev = {key: dev(v) for key, v in aux.items()}
    pa, pb = _pack(algo, a, b, TILE)
    split, need = abi_gemm(algo, pa, pb, m, n, k, TILE, epilogue, workspace=True, **aux_dev)
    whole, _ = abi_gemm(algo, pa, pb, m, n, k, TILE, epilogue, workspace=False, **aux_dev)
    assert need == _workspace_bytes(m, n, k)
    got, ref = host(split), host(whole)
    assert_ulp_close(got, ref, k=k)
    assert_ulp_close(got, _oracle(algo, a, b, TILE, epilogue=epilogue, **aux), k=k)
    # the surface passes the workspace: its result is the split call's
    fn = smx.strassen_matmul if algo == 7 else smx.cubic_matmul
    via_surface = fn(pa, pb, bm=TILE[0], bn=TILE[1], bk=TILE[2], epilogue=epilogue, **aux_dev)
    assert np.array_equal(host(via_surface), got)


@pytest.mark.parametrize("algo", [7, 8])
def test_whole_rounds_then_split_tail(algo):
    """384 tiles: 256 over full K with the fused epilogue, 128 split."""
    m, k, n = ROUND_AND_HALF
    if not _split_tiles(m, n, k):
        pytest.skip("no split at this shape: this device's CU count leaves no half-empty last round, or SMX_TAIL_SPLIT=0")
    rng, a, b = _problem(71 + algo, m, k, n)
    aux = _aux(rng, "residual_add", m, n)
    pa, pb = _pack(algo, a, b, TILE)
    split, _ = abi_gemm(algo, pa, pb, m, n, k, TILE, "residual_add", workspace=True, residual=dev(aux["residual"]))
    whole, _ = abi_gemm(algo, pa, pb, m, n, k, TILE, "residual_add", workspace=False, residual=dev(aux["residual"]))
    got = host(split)
    assert_ulp_close(got, host(whole), k=k)
    assert_ulp_close(got, _oracle(algo, a, b, TILE, epilogue="residual_add", **aux), k=k)


@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("scale_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("algo", [7, 8])
def test_split_qk_norm_rope(algo, scale_dtype, out_f32):
    """The q/k epilogue on a split tail: heads of 128 (64 columns of each
    tile half), norm over both halves, RoPE with the tables' output rows."""
    batch, seq, heads, k, bn = 2, 1024, 32, 2048, 512
    m, n, tile = batch * seq, heads * 128, (256, bn, 512)
    if not _split_tiles(m, n, k):
        pytest.skip("no split at this shape: this device's CU count leaves no half-empty round, or SMX_TAIL_SPLIT=0")
    x, w, laid, tcos, tsin, scale = _qk_problem(13, batch, seq, heads, k, bn)
    pa, pb = _pack(algo, x, laid, tile)
    rope = (dev(tcos), dev(tsin), torch.from_numpy(scale).to(DEV).to(scale_dtype))
    split, _ = abi_gemm(algo, pa, pb, m, n, k, tile, "qk_norm_rope", workspace=True, out_f32=out_f32, rope=rope)
    whole, _ = abi_gemm(algo, pa, pb, m, n, k, tile, "qk_norm_rope", workspace=False, out_f32=out_f32, rope=rope)
    got = host(split)
    if out_f32:
        np.testing.assert_allclose(got, host(whole), rtol=2e-5, atol=2e-5)
    else:
        assert_ulp_close(got, host(whole), k=k)
        want = _oracle(algo, x, laid, tile, epilogue="qk_norm_rope", rope_cos=tcos, rope_sin=tsin, rope_scale=scale,
                       rope_head_dim=128, rope_eps=1e-6)
        assert_ulp_close(got, want, k=k)


@pytest.mark.parametrize("formula,perm,epilogue", [("dual", 7, "residual_add"), ("powers", 5, None)])
def test_split_formula_variants(formula, perm, epilogue):
    m, k, n = HALF_ROUND
    if not _split_tiles(m, n, k):
        pytest.skip("no split at this shape: this device's CU count leaves no half-empty round, or SMX_TAIL_SPLIT=0")
    rng, a, b = _problem(81, m, k, n)
    aux = _aux(rng, epilogue, m, n)
    aux_dev = {key: dev(v) for key, v in aux.items()}
    pa, pb = _pack(7, a, b, TILE, formula=formula, block_permutation=perm)
    code = _lib.SMX_FORMULA[formula]
    split, _ = abi_gemm(7, pa, pb, m, n, k, TILE, epilogue, workspace=True, formula=code, block_permutation=perm,
                        **aux_dev)
    whole, _ = abi_gemm(7, pa, pb, m, n, k, TILE, epilogue, workspace=False, formula=code, block_permutation=perm,
                        **aux_dev)
    got = host(split)
    assert_ulp_close(got, host(whole), k=k)
    want = o.strassen_matmul(a, b, bm=TILE[0], bn=TILE[1], bk=TILE[2], epilogue=epilogue, formula_variant=formula,
                             block_permutation=perm, **aux)
    assert_ulp_close(got, want, k=k)


# tile counts that are not multiples of 8 (the tile map does not gather
# tiles by XCD then): 100 tiles (all split), 356 = one whole round + 100
RAGGED = [(2560, 2048, 2560), (1024, 2048, 22784)]


@pytest.mark.parametrize("shape", RAGGED)
@pytest.mark.parametrize("algo", [7, 8])
def test_ragged_tail_with_float32_operands(algo, shape):
    """Ragged tile counts, and float32 residual and bias operands read by
    the summing pass."""
    m, k, n = shape
    if not _split_tiles(m, n, k):
        pytest.skip("no split at this shape: this device's CU count leaves no half-empty last round, or SMX_TAIL_SPLIT=0")
    rng, a, b = _problem(101 + algo, m, k, n)
    pa, pb = _pack(algo, a, b, TILE)
    cases = (("residual_add", dict(residual=rng.standard_normal((m, n)).astype(np.float32))),
             ("bias_add", dict(bias=rng.standard_normal(n).astype(np.float32))))
    for epilogue, aux in cases:
        aux_dev = {key: dev32(v) for key, v in aux.items()}
        split, need = abi_gemm(algo, pa, pb, m, n, k, TILE, epilogue, workspace=True, **aux_dev)
        whole, _ = abi_gemm(algo, pa, pb, m, n, k, TILE, epilogue, workspace=False, **aux_dev)
        assert need == _workspace_bytes(m, n, k)
        got = host(split)
        assert_ulp_close(got, host(whole), k=k)
        assert_ulp_close(got, _oracle(algo, a, b, TILE, epilogue=epilogue, **aux), k=k)


def test_split_exact_panels_through_surface():
    """An exact-panel schedule: the Strassen pass over the ordinary panels
    (6 of 8, K = 3072: FP32 result, split) and the cubic pass with that
    partial (not split)."""
    m, _, n = HALF_ROUND
    k = 4096
    rng, a, b = _problem(91, m, k, n)
    kw = dict(bm=TILE[0], bn=TILE[1], bk=TILE[2], classical_panels=(0, 2))
    got = host(smx.strassen_matmul(dev(a), dev_weight(b), **kw))
    assert_ulp_close(got, o.strassen_matmul(a, b, **kw), k=k)


def test_workspace_below_the_size_asked_for_is_refused():
    m, k, n = HALF_ROUND
    if not _split_tiles(m, n, k):
        pytest.skip("no split at this shape: this device's CU count leaves no half-empty round, or SMX_TAIL_SPLIT=0")
    _, a, b = _problem(5, m, k, n)
    pa, pb = _pack(7, a, b, TILE)
    with pytest.raises(ValueError, match="workspace_bytes"):
        abi_gemm(7, pa, pb, m, n, k, TILE, workspace=True, workspace_bytes=_workspace_bytes(m, n, k) - 16)


@pytest.mark.parametrize("case", ["full_round", "short_k", "full_last_round", "partial"])
def test_no_workspace_asked_for(case):
    """Whole rounds, K below 2048, a last round more than half full and FP32
    partials keep every tile over full K: the library asks for no
    workspace."""
    lib = _lib.load()
    d = _lib.SmxGemmDesc()
    m, k, n, tile = 2048, 2048, 4096, TILE
    if case == "full_round":
        m, n = 4096, 4096  # 256 tiles
    elif case == "short_k":
        k = 1024
    elif case == "full_last_round":
        m, n = 6144, 5120  # 480 tiles: one round and 224
    if _plan(m, n, k)[1] and case != "partial":
        pytest.skip("this device's CU count splits this shape")
    d.m, d.n, d.k = m, n, k
    d.lda = d.ldb = k
    d.ldc = n
    d.bm, d.bn, d.bk = tile
    d.algo = 8 if case == "partial" else 7
    d.a_layout, d.b_layout = _lib.SMX_A_PACKED, _lib.SMX_B_PACKED
    d.rope_head_dim, d.rope_eps = 128, 1e-6
    partial = None
    if case == "partial":
        partial = torch.zeros(m, n, dtype=torch.float32, device=DEV)
        d.partial, d.ldp = partial.data_ptr(), n
    need = ctypes.c_int64(-1)
    _lib.check(lib.smx_gemm_workspace_bytes(d, ctypes.byref(need)))
    assert need.value == 0


# Small launches: (m, k, n), tile. 20 tiles in 8 shares (one row tile; a
# thin tiling with decode-sized M); 12 thin tiles over three product-row
# tiles, the last partly padding, in 4 shares.
SMALL = [
    ((256, 4096, 5120), (256, 256, 512)),
    ((16, 4096, 5120), (16, 256, 512)),
    ((544, 2048, 1024), (272, 256, 256)),
]


@pytest.mark.parametrize("epilogue", [None, "swiglu", "residual_add"])
@pytest.mark.parametrize("shape,tile", SMALL)
@pytest.mark.parametrize("algo", [7, 8])
def test_small_launch_split_every_tile(algo, shape, tile, epilogue):
    (m, k, n), bm = shape, tile[0]
    whole_tiles, split, s = _plan(m, n, k, bm)
    if not split:
        pytest.skip("no split at this shape: this device's CU count, or SMX_TAIL_SPLIT=0")
    rng, a, b = _problem(111 + algo, m, k, n)
    aux = _aux(rng, epilogue, m, n)
    aux_dev = {key: dev(v) for key, v in aux.items()}
    pa, pb = _pack(algo, a, b, tile)
    got_split, need = abi_gemm(algo, pa, pb, m, n, k, tile, epilogue, workspace=True, **aux_dev)
    got_whole, _ = abi_gemm(algo, pa, pb, m, n, k, tile, epilogue, workspace=False, **aux_dev)
    assert whole_tiles == 0 and need == s * split * SPLIT_TILE_BYTES
    got = host(got_split)
    assert_ulp_close(got, host(got_whole), k=k)
    assert_ulp_close(got, _oracle(algo, a, b, tile, epilogue=epilogue, **aux), k=k)


@pytest.mark.parametrize("algo", [7, 8])
def test_thin_split_stores_only_real_rows(algo):
    """A thin tiling's K shares store only the tile's real product rows in
    their dense 256 x 256 workspace blocks (rows r and 128 + r for the M/2
    real product rows r): 16 tokens make 8 of the 128, and the padding rows'
    stores would cost 15 times the bytes. The sentinel the workspace is
    filled with survives in every padding row."""
    m, k, n, tile = 16, 25600, 5120, (16, 256, 512)
    _, split, s = _plan(m, n, k, 16)
    if not split:
        pytest.skip("no split at this shape: this device's CU count, or SMX_TAIL_SPLIT=0")
    _, a, b = _problem(131 + algo, m, k, n)
    pa, pb = _pack(algo, a, b, tile)
    out, need, ws = abi_gemm(algo, pa, pb, m, n, k, tile, workspace=True, keep_workspace=True)
    assert need == s * split * SPLIT_TILE_BYTES
    blocks = ws[:need].view(torch.int32).view(s * split, 256, 256).cpu()
    real = torch.zeros(256, dtype=torch.bool)
    real[: m // 2] = True
    real[128: 128 + m // 2] = True
    assert (blocks[:, ~real, :] == -1).all(), "a padding row of a share was stored"
    assert not (blocks[:, real, :] == -1).any(), "a real row of a share was not stored"
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("algo", [7, 8])
def test_small_thin_launch_qk_norm_rope(algo):
    """Decode-sized q/k: 48 tokens (a thin tiling, bm = 16), 8 heads, every
    tile in K shares; the summing pass maps rows as the thin epilogue does
    and reads the tables at the output rows."""
    batch, seq, heads, k, bn = 1, 48, 8, 2048, 256
    m, n, tile = batch * seq, heads * 128, (16, bn, 512)
    if not _split_tiles(m, n, k, 16):
        pytest.skip("no split at this shape: this device's CU count, or SMX_TAIL_SPLIT=0")
    x, w, laid, tcos, tsin, scale = _qk_problem(17, batch, seq, heads, k, bn)
    pa, pb = _pack(algo, x, laid, tile)
    rope = (dev(tcos), dev(tsin), torch.from_numpy(scale).to(DEV).to(torch.bfloat16))
    split, need = abi_gemm(algo, pa, pb, m, n, k, tile, "qk_norm_rope", workspace=True, rope=rope)
    whole, _ = abi_gemm(algo, pa, pb, m, n, k, tile, "qk_norm_rope", workspace=False, rope=rope)
    assert need == _workspace_bytes(m, n, k, 16)
    got = host(split)
    assert_ulp_close(got, host(whole), k=k)
    want = _oracle(algo, x, laid, tile, epilogue="qk_norm_rope", rope_cos=tcos, rope_sin=tsin, rope_scale=scale,
                   rope_head_dim=128, rope_eps=1e-6)
    assert_ulp_close(got, want, k=k)
