"""Packed operands: the layout the packed gfx950 kernel streams into LDS.

A projection weight is static, so the classical B operand sums of
``strassen_pallas.py:324-379`` (B0+B3, B0, B1-B3, B2-B0, B3, B0+B1, B2+B3,
each rounded once to bf16) are formed once, offline, like the reference's
``swiglu_weight_layout`` / ``rope_weight_layout`` relayouts
(``strassen_pallas.py:1315-1411``); the activation's A sums (A0+A3, A2+A3,
A0, A3, A0+A1, A2-A0, A1-A3) are formed once per call by a bandwidth-bound
pass. The cubic control packs the raw quadrants (four operands) the same
way, so both arms stream identical fragment layouts. Results are identical
to forming the sums inside the GEMM.

Storage (``smx_pack_operand``): for ``R`` product rows (``M/2`` of A,
``N/2`` of B) and product depth ``K/2``, ``[R/128][K/32][nops][4][64][8]``
bf16, i.e. 1 KB MFMA operand fragments in lane order; ``nops`` is 7
(Strassen) or 4 (cubic), so a packed operand holds ``nops/4`` times the
elements of the original.

Exact K panels (``classical_panels`` / ``panel_schedule``) split an operand
into a ``SplitOperand``: its ordinary panels packed for Strassen and its
exact panels packed as cubic quadrants. The GEMM runs Strassen over the
ordinary panels into an FP32 partial and the cubic kernel over the exact
panels, which adds the partial before the epilogue.
"""

from __future__ import annotations

import collections
import ctypes
import os
import weakref

import torch

from . import _lib

__all__ = ["PackedOperand", "SplitOperand", "ExactSchedule", "exact_schedule", "pack_operand", "precision_passes",
           "strassen_weight_layout", "cubic_weight_layout", "pack_activation", "cache_packed_weights",
           "packed_weight_cache_info", "pack_weight_for_call", "default_cache_bytes", "weight_cached_or_fits"]

_ALGOS = {_lib.SMX_ALGO_STRASSEN: "strassen", _lib.SMX_ALGO_CUBIC: "cubic"}

# jax.lax.Precision names and their string aliases -> bf16 passes per product
# of FP32 operands (DEFAULT one pass; HIGH the 3-pass and HIGHEST the 6-pass
# bf16 product).
_PRECISION_PASSES = {"DEFAULT": 1, "FASTEST": 1, "BFLOAT16": 1,
                     "HIGH": 3, "BFLOAT16_3X": 3, "TENSORFLOAT32": 3,
                     "HIGHEST": 6, "FLOAT32": 6}


def precision_passes(dot_precision, dtype):
    """bf16 passes per product for ``dot_precision`` on inputs of ``dtype``:
    1 for bf16 inputs (their operands have no low-order part: the reference
    forms bf16 operand sums in bf16, so HIGH / HIGHEST products equal the
    one-pass product), else 1 / 3 / 6 for DEFAULT / HIGH / HIGHEST. A pair
    (lhs, rhs) must name one precision."""
    if isinstance(dot_precision, (tuple, list)):
        if len(dot_precision) != 2:
            raise ValueError(f"dot_precision pair expected, got {dot_precision!r}")
        first, second = (precision_passes(p, torch.float32) for p in dot_precision)
        if first != second:
            raise NotImplementedError("dot_precision pairs with two different precisions are not implemented")
        dot_precision = dot_precision[0]
    if dot_precision is None:
        passes = 1
    else:
        name = str(getattr(dot_precision, "name", dot_precision)).upper()
        name = name.rsplit(".", 1)[-1]
        if name not in _PRECISION_PASSES:
            raise ValueError(f"unknown dot_precision {dot_precision!r}")
        passes = _PRECISION_PASSES[name]
    return passes if dtype == torch.float32 else 1


class ExactSchedule:
    """The exact K panels of a call (``classical_panels`` / ``panel_schedule``):
    ``exact`` and ``ordinary`` are the sorted panel indices of each kind out
    of ``nk``."""

    def __init__(self, nk, exact):
        self.nk = int(nk)
        self.exact = tuple(sorted(int(p) for p in exact))
        exact_set = set(self.exact)
        self.ordinary = tuple(p for p in range(self.nk) if p not in exact_set)

    def panel_map(self, kind, device):
        """int32 device tensor of the ``kind`` ("exact" / "ordinary") panel
        indices, uploaded once per (device, schedule)."""
        key = (str(device), self.nk, self.exact, kind)
        tensor = _PANEL_MAPS.get(key)
        if tensor is None:
            tensor = _PANEL_MAPS[key] = torch.tensor(getattr(self, kind), dtype=torch.int32).to(device)
        return tensor

    def __eq__(self, other):
        return isinstance(other, ExactSchedule) and (self.nk, self.exact) == (other.nk, other.exact)

    def __hash__(self):
        return hash((self.nk, self.exact))

    def __repr__(self):
        return f"ExactSchedule(exact={self.exact}, nk={self.nk})"


_PANEL_MAPS = {}


def exact_schedule(nk, *, classical_panels=(), panel_schedule=None):
    """Resolve the reference's two exact-panel forms (static
    ``classical_panels``, ``strassen_pallas.py:1030-1045``; prefetched
    ``panel_schedule``, ``:1079-1090``) into an ``ExactSchedule``, or None
    when no panel is exact. The split into the two GEMMs is sized on the
    host, so a schedule held on the device is read back (one
    synchronisation)."""
    if panel_schedule is not None:
        if isinstance(panel_schedule, ExactSchedule):
            schedule = panel_schedule
        else:
            flags = torch.as_tensor(panel_schedule)
            if tuple(flags.shape) != (nk,):
                raise ValueError(f"panel_schedule must have shape ({nk},), got {tuple(flags.shape)}")
            # jnp.asarray(..., dtype=int32): fractions truncate toward zero.
            flags = flags.to(torch.int32)
            schedule = ExactSchedule(nk, torch.nonzero(flags).flatten().tolist())
    else:
        panels = tuple(sorted({int(p) for p in classical_panels}))
        if panels and (panels[0] < 0 or panels[-1] >= nk):
            raise ValueError(f"classical_panels {panels} outside 0..{nk - 1}")
        schedule = ExactSchedule(nk, panels)
    return schedule if schedule.exact else None


class PackedOperand:
    """A bf16 operand packed for one algorithm and quadrant tile.

    ``side`` is ``"lhs"`` for an activation ``a [M, K]`` (``tile_rows`` =
    bm) or ``"rhs"`` for a weight ``b [K, N]`` (``tile_rows`` = bn). Pass it
    to ``strassen_matmul`` / ``cubic_matmul`` in place of the tensor, with
    the same tile.
    """

    def __init__(self, data, *, algo, side, rows, k, tile_rows, bk, formula="classical", block_permutation=0,
                 source_dtype=torch.bfloat16, passes=1):
        self.data = data
        self.source_dtype = source_dtype  # the packed fragments are bf16 either way
        # bf16 passes per product (FP32 sources at HIGH / HIGHEST): the packed
        # K is passes * k, pass-major
        self.passes = int(passes)
        self.algo, self.side = int(algo), side
        self.rows, self.k, self.tile_rows, self.bk = int(rows), int(k), int(tile_rows), int(bk)
        self.formula, self.block_permutation = formula, int(block_permutation)

    schedule = None  # packed for every K panel (no exact panels)

    # The parts of the tensor interface the callers' argument checks use.
    @property
    def shape(self):
        return torch.Size((self.rows, self.k) if self.side == "lhs" else (self.k, self.rows))

    @property
    def dtype(self):
        return self.source_dtype

    @property
    def device(self):
        return self.data.device

    def dim(self):
        return 2

    def __repr__(self):
        variant = "" if self.algo != _lib.SMX_ALGO_STRASSEN else \
            f", formula={self.formula}, block_permutation={self.block_permutation}"
        if self.passes > 1:
            variant += f", passes={self.passes}"
        return (f"PackedOperand({_ALGOS[self.algo]}, {self.side}, shape={tuple(self.shape)}, "
                f"tile_rows={self.tile_rows}, bk={self.bk}{variant}, device={self.device})")


class SplitOperand(PackedOperand):
    """A Strassen operand packed for an exact-panel schedule: ``ordinary``
    holds its ordinary K panels packed for Strassen (None if every panel is
    exact), ``exact`` its exact panels packed as cubic quadrants."""

    def __init__(self, ordinary, exact, *, side, rows, k, tile_rows, bk, formula, block_permutation, schedule):
        super().__init__(exact.data, algo=_lib.SMX_ALGO_STRASSEN, side=side, rows=rows, k=k, tile_rows=tile_rows,
                         bk=bk, formula=formula, block_permutation=block_permutation,
                         source_dtype=exact.source_dtype, passes=exact.passes)
        self.ordinary, self.exact, self.schedule = ordinary, exact, schedule

    def __repr__(self):
        return (f"SplitOperand({self.side}, shape={tuple(self.shape)}, tile_rows={self.tile_rows}, bk={self.bk}, "
                f"formula={self.formula}, block_permutation={self.block_permutation}, "
                f"exact_panels={self.schedule.exact}, device={self.device})")


def packed_bytes(algo, rows, k):
    out = ctypes.c_int64()
    _lib.check(_lib.load().smx_packed_bytes(algo, rows, k, ctypes.byref(out)))
    return out.value


def _pack(src, *, algo, side, rows, k, tile_rows, bk, formula, block_permutation, panels=None, passes=1):
    """One smx_pack_operand call over ``src`` (rows x K source, or K x rows
    for lhs_t); ``panels`` (a device int32 map) selects the K panels to
    pack, in order; ``passes`` > 1 packs the bf16 parts of a multi-pass
    product after each panel."""
    packed_k = k if panels is None else panels.numel() * bk
    nbytes = packed_bytes(algo, rows, packed_k * passes)
    data = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=src.device)
    side_id = {"lhs": _lib.SMX_SIDE_LHS, "rhs": _lib.SMX_SIDE_RHS, "lhs_t": _lib.SMX_SIDE_LHS_T}[side]
    stream = torch.cuda.current_stream(src.device).cuda_stream
    src_dtype = _lib.SMX_DTYPE_F32 if src.dtype == torch.float32 else _lib.SMX_DTYPE_BF16
    rc = _lib.load().smx_pack_operand(algo, _lib.SMX_FORMULA[formula], block_permutation, side_id, rows,
                                      packed_k * passes, _lib.ptr(src), src_dtype, passes, src.stride(0), tile_rows,
                                      bk, _lib.ptr(panels), k, _lib.ptr(data), stream)
    _lib.check(rc)
    return PackedOperand(data, algo=algo, side="rhs" if side == "rhs" else "lhs", rows=rows, k=packed_k,
                         tile_rows=tile_rows, bk=bk, formula=formula, block_permutation=block_permutation,
                         source_dtype=src.dtype, passes=passes)


def pack_operand(x, *, algo, side, tile_rows, bk, formula="classical", block_permutation=0, classical_panels=(),
                 panel_schedule=None, dot_precision=None):
    """Pack ``x`` (bf16 on the HIP device): ``a [M, K]`` for ``side="lhs"``,
    the same ``a`` stored transposed as ``[K, M]`` for ``side="lhs_t"``, or a
    weight ``b [K, N]`` for ``side="rhs"`` (any strides; a K-contiguous view
    of ``[N, K]`` storage is read in place). Runs asynchronously on torch's
    current stream. Strassen operands carry the operand sums of
    ``formula`` ("classical", "dual" or "powers") after the quadrant swaps of
    ``block_permutation``; both operands of a GEMM must be packed alike. With
    exact panels (``classical_panels`` or ``panel_schedule``) a Strassen
    operand becomes a ``SplitOperand``. A float32 ``x`` is packed for the
    product of ``dot_precision`` (DEFAULT: each operand rounded once to bf16;
    HIGH / HIGHEST: its bf16 parts for 3 / 6 passes)."""
    if formula not in _lib.SMX_FORMULA:
        raise ValueError("formula_variant must be 'classical', 'dual', or 'powers'")
    if side not in ("lhs", "rhs", "lhs_t"):
        raise ValueError("side must be 'lhs', 'lhs_t' or 'rhs'")
    if algo not in _ALGOS:
        raise ValueError(f"algo must be {_lib.SMX_ALGO_STRASSEN} or {_lib.SMX_ALGO_CUBIC}")
    if x.dim() != 2:
        raise ValueError("pack_operand expects a rank-2 matrix")
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("pack_operand expects bf16 or float32")
    if x.device.type != "cuda":
        raise ValueError("pack_operand runs on the HIP device")
    if side == "lhs_t":
        src = x  # [K, rows], rows contiguous
        k, rows = src.shape
        if src.stride(1) != 1 or src.data_ptr() % 16:
            src = src.contiguous()
    else:
        src = x if side == "lhs" else x.t()  # rows x K, K contiguous
        rows, k = src.shape
        if src.stride(1) != 1 or (src.stride(0) * src.element_size()) % 16 or src.data_ptr() % 16:
            src = src.contiguous()
    if rows % tile_rows or k % bk:
        raise ValueError(f"operand [{rows}, {k}] (rows x K) does not tile by ({tile_rows}, {bk})")
    passes = precision_passes(dot_precision, x.dtype)
    common = dict(side=side, rows=rows, k=k, tile_rows=tile_rows, bk=bk)
    schedule = exact_schedule(k // bk, classical_panels=classical_panels, panel_schedule=panel_schedule)
    if schedule is None:
        return _pack(src, algo=algo, formula=formula, block_permutation=block_permutation, passes=passes, **common)
    if algo != _lib.SMX_ALGO_STRASSEN:
        raise ValueError("exact panels apply to the Strassen algorithm only")
    if formula == "powers":
        raise ValueError("exact panels require a quadrant-basis formula")
    ordinary = None
    if schedule.ordinary:
        ordinary = _pack(src, algo=algo, formula=formula, block_permutation=block_permutation,
                         panels=schedule.panel_map("ordinary", x.device), passes=passes, **common)
    exact = _pack(src, algo=_lib.SMX_ALGO_CUBIC, formula="classical", block_permutation=0,
                  panels=schedule.panel_map("exact", x.device), passes=passes, **common)
    common["side"] = "rhs" if side == "rhs" else "lhs"
    return SplitOperand(ordinary, exact, formula=formula, block_permutation=block_permutation, schedule=schedule,
                        **common)


class _WeightCache:
    """Packed forms of plain weights, reused while a weight is unchanged.

    A call that passes an ordinary ``[K, N]`` weight packs it (the seven
    Strassen operand sums, 7/4 of its bytes, or the cubic's quadrants) before
    the GEMM; the packed form of the same weight is reused on later calls.
    Key: the weight's data address, view geometry, dtype and device, and the
    packing (algorithm, tile, formula, block permutation, exact panels, bf16
    passes). An entry holds a weak reference to the tensor whose storage the
    weight is (the view's base, else the weight itself), never the weight:
    when that tensor is freed the entry goes with it, so neither the plain
    weight nor a stale packed form outlives the caller's weight, and a new
    tensor at the same address cannot match. It also records torch's version
    counter at packing (shared by a tensor and its views): an in-place update
    of the weight through it or any view of it bumps the counter and the next
    call packs again. Writes that bypass the counter (through ``.data``, or
    from outside torch) are not seen. Least-recently used entries are dropped
    beyond the capacity (bytes of packed data, the only device memory the
    cache holds); an operand larger than the capacity is not kept. Not
    thread-safe."""

    def __init__(self, capacity):
        # None: default_cache_bytes(), resolved at first use (it reads the
        # device's memory size, which initialises the GPU runtime)
        self._capacity = None if capacity is None else int(capacity)
        self.entries = collections.OrderedDict()
        self.bytes = 0
        self.hits = self.misses = self.stale = 0

    @property
    def capacity(self):
        if self._capacity is None:
            self._capacity = default_cache_bytes()
        return self._capacity

    @staticmethod
    def _nbytes(packed):
        parts = [packed.ordinary, packed.exact] if isinstance(packed, SplitOperand) else [packed]
        return sum(p.data.numel() * p.data.element_size() for p in parts if p is not None)

    @staticmethod
    def _key(x, packing):
        return (x.data_ptr(), tuple(x.shape), tuple(x.stride()), x.dtype, str(x.device), packing)

    def resize(self, capacity):
        self._capacity = int(capacity)
        self._evict()

    def _drop(self, key):
        entry = self.entries.pop(key, None)
        if entry is not None:
            self.bytes -= entry[3]

    def _evict(self):
        while self.entries and self.bytes > self.capacity:
            _, (_, _, _, nbytes) = self.entries.popitem(last=False)
            self.bytes -= nbytes

    def _valid(self, key):
        entry = self.entries.get(key)
        if entry is None:
            return None
        owner, version, packed, _ = entry
        base = owner()
        if base is None:  # freed (its weak-reference callback drops the entry)
            self._drop(key)
            return None
        if base._version != version:
            self.stale += 1
            self._drop(key)
            return None
        return packed

    def contains(self, x, packing):
        """Whether the packed form of ``x`` is held and current (packs nothing)."""
        return self.capacity > 0 and self._valid(self._key(x, packing)) is not None

    def has_room(self, nbytes):
        """Whether ``nbytes`` more would fit without evicting an entry."""
        return self.bytes + nbytes <= self.capacity

    def lookup(self, x, packing, make):
        if self.capacity <= 0:
            return make()
        key = self._key(x, packing)
        packed = self._valid(key)
        if packed is not None:
            self.entries.move_to_end(key)
            self.hits += 1
            return packed
        self.misses += 1
        base = x._base if x._base is not None else x
        version = base._version
        packed = make()
        nbytes = self._nbytes(packed)
        if nbytes <= self.capacity:
            entries = self.entries

            def forget(_, key=key, entries=entries, cache=self):
                if key in entries and entries[key][0]() is None:
                    cache._drop(key)

            self.entries[key] = (weakref.ref(base, forget), version, packed, nbytes)
            self.bytes += nbytes
            self._evict()
        return packed


def default_cache_bytes():
    """The packed-weight cache's default capacity: ``SMX_WEIGHT_CACHE_BYTES``
    when set (0 turns the cache off), else the smaller of 16 GiB and 1/16 of
    the current device's memory (18 GB of an MI355X's 288 GB: the packed
    Strassen weights of ten Qwen3-32B layers)."""
    env = os.environ.get("SMX_WEIGHT_CACHE_BYTES")
    if env is not None and env.strip() != "":
        return int(env)
    if not torch.cuda.is_available():
        return 16 << 30
    total = torch.cuda.get_device_properties(torch.cuda.current_device()).total_memory
    return int(min(16 << 30, total // 16))


_WEIGHT_CACHE = _WeightCache(None)


def cache_packed_weights(capacity_bytes):
    """Keep the packed forms of plain weights that ``strassen_matmul`` /
    ``cubic_matmul`` calls pack, up to ``capacity_bytes`` of packed data (0
    packs on every call and empties the cache; the default is
    ``default_cache_bytes()``). Returns the previous capacity. The cache
    holds no plain weight: an entry goes when its weight is freed. A working
    set larger than the capacity evicts before reuse and then only adds
    bookkeeping to the per-call packing; packing weights once with
    ``strassen_weight_layout`` / ``cubic_weight_layout`` needs no cache."""
    previous = _WEIGHT_CACHE.capacity
    _WEIGHT_CACHE.resize(capacity_bytes)
    return previous


def packed_weight_cache_info():
    """Hits, misses, stale entries (weights updated in place), entries held,
    bytes held and capacity of the packed-weight cache."""
    c = _WEIGHT_CACHE
    return {"hits": c.hits, "misses": c.misses, "stale": c.stale, "entries": len(c.entries), "bytes": c.bytes,
            "capacity": c.capacity}


def _weight_packing(algo, bn, bk, formula="classical", block_permutation=0, classical_panels=(), exact=None,
                    dot_precision=None):
    return (algo, bn, bk, formula, block_permutation, tuple(classical_panels), exact, dot_precision)


def weight_cached_or_fits(b, *, algo, bn, bk, packed_bytes):
    """Whether a call on the plain weight ``b`` (default packing) finds its
    packed form in the cache, or can add it (``packed_bytes``) without
    evicting another entry."""
    packing = _weight_packing(algo, bn, bk)
    return _WEIGHT_CACHE.contains(b, packing) or (_WEIGHT_CACHE.capacity > 0 and _WEIGHT_CACHE.has_room(packed_bytes))


def pack_weight_for_call(b, *, algo, bn, bk, formula="classical", block_permutation=0, classical_panels=(),
                         panel_schedule=None, dot_precision=None):
    """The packed weight a GEMM call on a plain weight ``b [K, N]`` needs:
    from the packed-weight cache when it holds ``b`` unchanged, else packed
    now (and kept when the cache is enabled)."""
    def make():
        return pack_operand(b, algo=algo, side="rhs", tile_rows=bn, bk=bk, formula=formula,
                            block_permutation=block_permutation, classical_panels=classical_panels,
                            panel_schedule=panel_schedule, dot_precision=dot_precision)

    if panel_schedule is not None and not isinstance(panel_schedule, ExactSchedule):
        return make()  # a schedule still to be read from the device: packed per call
    exact = panel_schedule.exact if panel_schedule is not None else None
    packing = _weight_packing(algo, bn, bk, formula, block_permutation, classical_panels, exact, dot_precision)
    return _WEIGHT_CACHE.lookup(b, packing, make)


def strassen_weight_layout(b, bn, bk, *, formula_variant="classical", block_permutation=0, classical_panels=(),
                           panel_schedule=None, dot_precision=None):
    """Pre-sum and pack a bf16 or float32 ``[K, N]`` weight for
    ``strassen_matmul`` with the tile ``(bn, bk)`` (and the formula, block
    permutation, exact panels and, for float32, ``dot_precision`` the calls
    will use)."""
    return pack_operand(b, algo=_lib.SMX_ALGO_STRASSEN, side="rhs", tile_rows=bn, bk=bk,
                        formula=formula_variant, block_permutation=block_permutation,
                        classical_panels=classical_panels, panel_schedule=panel_schedule,
                        dot_precision=dot_precision)


def cubic_weight_layout(b, bn, bk, *, dot_precision=None):
    """Pack a bf16 or float32 ``[K, N]`` weight's quadrants for
    ``cubic_matmul`` with the tile ``(bn, bk)``."""
    return pack_operand(b, algo=_lib.SMX_ALGO_CUBIC, side="rhs", tile_rows=bn, bk=bk, dot_precision=dot_precision)


def pack_activation(a, algo, bm, bk, *, formula_variant="classical", block_permutation=0, classical_panels=(),
                    panel_schedule=None, dot_precision=None):
    """Pack an activation ``a [M, K]`` once for several GEMMs that share it
    (e.g. the q, k and v projections)."""
    return pack_operand(a, algo=algo, side="lhs", tile_rows=bm, bk=bk, formula=formula_variant,
                        block_permutation=block_permutation, classical_panels=classical_panels,
                        panel_schedule=panel_schedule, dot_precision=dot_precision)
