"""Tile screening and the measured dispatcher (``tuned_matmul``).

Restates two pieces of the reference for gfx950:

* ``tuned_matmul`` (``strassen_pallas.py:1428-1461``): dispatch a bf16 GEMM
  to Strassen only for shapes where Strassen measurably beat the native GEMM
  on this hardware, otherwise to ``native_matmul`` (hipBLASLt). The set of
  winning shapes is data: the reference hard-codes its TPU wins
  (``:49-72``); here the table is produced by ``measure_dispatch`` on an
  MI355X and shipped as ``tuned_shapes.json`` (override with the
  ``SMX_TUNED_TABLE`` environment variable).
* the fixed-budget tile screen of
  ``experiments/qwen3/benchmark_qwen3_scaling_tile_tune.py:103-133``, with the
  same rules: enumerate ``(bm, bn, bk)`` candidates that divide the geometry,
  satisfy the kernels' tile rule and admit the paired gate|up layout; give
  every surviving candidate exactly ``warmups`` + ``runs`` timed calls per
  arm; record failures in-band; the winner per arm is the lowest mean, ties
  to the earlier candidate, with no re-timing. On gfx950 the screen keeps
  the packed kernel's full-tile rule (``bm % 256``, ``bn % 256``,
  ``bk % 64``): thin tilings (``bm % 16``) run as well, but they exist for
  an M that no full-tile bm divides, not as faster candidates; there is no
  VMEM budget to screen against, because the kernel's LDS footprint is fixed
  by its 128 x 128 product-space workgroup tile, not by ``(bm, bn, bk)``.

Timing is per call with HIP events on torch's current stream (the stream
the kernels launch on), so one sample is one whole call: activation packing,
GEMM and fused epilogue.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys

import torch

from . import _lib
from .layouts import swiglu_weight_layout
from .packing import (cache_packed_weights, cubic_weight_layout, pack_activation, pack_operand,
                      packed_weight_cache_info, strassen_weight_layout, weight_cached_or_fits)
from .strassen import cubic_matmul, native_matmul, per_call_packing_expected, strassen_matmul

__all__ = ["TILE_RULE", "enumerate_candidates", "time_calls", "screen_tiles", "measure_dispatch",
           "load_table", "tuned_matmul", "DEFAULT_TABLE"]

HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_TABLE = os.path.join(HERE, "tuned_shapes.json")

# The screened tile rule: bm, bn multiples of 2 x 128 product rows / columns
# (whole product tiles; smx_tile_requirements also admits thin bm % 16), bk of
# 2 x 32 product depth.
TILE_RULE = (256, 256, 64)
BM_CANDIDATES = (512, 1024, 2048)
BN_CANDIDATES = (512, 1024, 2048, 2560)
BK_CANDIDATES = (256, 512, 1024)


def enumerate_candidates(m, k, n, *, paired_width=None, bm_candidates=BM_CANDIDATES, bn_candidates=BN_CANDIDATES,
                         bk_candidates=BK_CANDIDATES):
    """(kept, filtered) tile candidates for a ``[m, k] @ [k, n]`` GEMM, in
    enumeration order. ``paired_width``: the gate (= up) width of a SwiGLU
    weight, which must hold whole ``bn/2`` blocks
    (``benchmark_qwen3_scaling_tile_tune.py:103-133``)."""
    kept, filtered = [], []
    for bm in bm_candidates:
        for bn in bn_candidates:
            for bk in bk_candidates:
                reasons = []
                if m % bm:
                    reasons.append(f"M {m} % bm")
                if n % bn:
                    reasons.append(f"N {n} % bn")
                elif paired_width is not None and paired_width % (bn // 2):
                    reasons.append(f"gate width {paired_width} % (bn//2)")
                if k % bk:
                    reasons.append(f"K {k} % bk")
                if bm % TILE_RULE[0] or bn % TILE_RULE[1] or bk % TILE_RULE[2]:
                    reasons.append("gfx950 tile rule")
                entry = {"tile": [bm, bn, bk]}
                if reasons:
                    entry["filtered_because"] = reasons
                    filtered.append(entry)
                else:
                    kept.append(entry)
    return kept, filtered


def time_calls(function, warmups, runs, batch=1):
    """``warmups`` untimed calls, then ``runs`` samples timed with HIP
    events, each over ``batch`` back-to-back calls; returns milliseconds per
    call of each sample. A batch keeps the device busy while the host issues
    the next call, so short kernels are timed without the host's per-call
    work between them."""
    for _ in range(warmups):
        function()
    torch.cuda.synchronize()
    events = []
    for _ in range(runs):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(batch):
            function()
        stop.record()
        events.append((start, stop))
    torch.cuda.synchronize()
    return [start.elapsed_time(stop) / batch for start, stop in events]


def _device_name(device):
    props = torch.cuda.get_device_properties(device)
    return f"{props.name} ({props.gcnArchName.split(':')[0]})"


def _inputs(m, k, n, seed, device):
    """Activations ~N(0, 1), weight ~N(0, 0.02) stored [n, k] and viewed
    ``[k, n]`` (the layout of an nn.Linear weight), bf16."""
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(m, k, device=device, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, device=device, generator=g) * 0.02).to(torch.bfloat16).t()
    return x, w


def _activate(full):
    gate, up = full.chunk(2, dim=-1)
    return (torch.nn.functional.silu(gate.float()) * up.float()).to(torch.bfloat16)


def screen_tiles(m, k, n, *, swiglu=True, seed=20260907, warmups=2, runs=5, device="cuda", emit=None, **axes):
    """Fixed-budget tile screen for one GEMM geometry; returns the winners.

    Arms: ``strassen`` (packed weight, fused SwiGLU when ``swiglu``) and
    ``cubic`` (the matched cubic, same form); the hipBLASLt GEMM (plus the
    activation) is timed once for context and takes no part in the choice.
    Weights are laid out and packed outside the timed calls, as the
    reference relayouts them offline."""
    emit = emit or (lambda record: None)
    device = torch.device(device)
    kept, filtered = enumerate_candidates(m, k, n, paired_width=n // 2 if swiglu else None, **axes)
    emit({"kind": "metadata", "shape": [m, k, n], "swiglu": swiglu, "device": _device_name(device),
          "candidates": kept, "filtered": filtered, "budget": {"warmups": warmups, "runs": runs,
                                                               "arms": ["strassen", "cubic"]},
          "seed": seed,
          "rule": "identical enumeration and budget per candidate; winner per arm is the lowest mean; failures "
                  "recorded in-band skip only that candidate/arm; no re-timing",
          "scope": "tile screening only; not a registered comparison"})
    if not kept:
        emit({"kind": "verdict", "passes": False, "reason": "no feasible tile candidate"})
        return {}
    x, w = _inputs(m, k, n, seed, device)
    if swiglu:
        context = time_calls(lambda: _activate(native_matmul(x, w)), warmups, runs)
    else:
        context = time_calls(lambda: native_matmul(x, w), warmups, runs)
    emit({"kind": "tune", "arm": "hipblaslt", "tile": None, "mean_ms": statistics.fmean(context),
          "samples_ms": context, "note": "context only; not part of the tile decision"})
    epilogue = "swiglu" if swiglu else None
    results = {"strassen": [], "cubic": []}
    laid_cache = {}
    for entry in kept:
        bm, bn, bk = entry["tile"]
        if bn not in laid_cache:
            laid_cache.clear()
            laid_cache[bn] = swiglu_weight_layout(w, bn) if swiglu else w
        laid = laid_cache[bn]
        for arm in ("strassen", "cubic"):
            try:
                pack = strassen_weight_layout if arm == "strassen" else cubic_weight_layout
                packed = pack(laid, bn, bk)
                gemm = strassen_matmul if arm == "strassen" else cubic_matmul
                values = time_calls(lambda: gemm(x, packed, bm=bm, bn=bn, bk=bk, epilogue=epilogue), warmups, runs)
            except (ValueError, RuntimeError) as error:
                emit({"kind": "tune_failure", "arm": arm, "tile": [bm, bn, bk], "error_type": type(error).__name__,
                      "error": str(error).splitlines()[-1][:2000]})
            else:
                mean = statistics.fmean(values)
                results[arm].append(([bm, bn, bk], mean))
                emit({"kind": "tune", "arm": arm, "tile": [bm, bn, bk], "mean_ms": mean, "samples_ms": values})
            finally:
                packed = None
    chosen = {}
    for arm, rows in results.items():
        if rows:
            tile, mean = min(rows, key=lambda row: row[1])  # min keeps the earliest of equal means
            chosen[arm] = {"tile": tile, "mean_ms": mean}
    emit({"kind": "chosen", "shape": [m, k, n], "winners": chosen,
          "hipblaslt_context_mean_ms": statistics.fmean(context)})
    emit({"kind": "verdict", "passes": "strassen" in chosen and "cubic" in chosen,
          "scope": "tile screening; winners feed the harnesses"})
    return chosen


# Row tiles a dispatched shape may use when M is not a multiple of the
# default tile's bm (prefill chunks and decode batches; bm % 16, as the
# reference allows).
DISPATCH_BM = (1024, 512, 256, 128, 64, 32, 16)


def dispatch_tile(m, k, n, tile=(1024, 1024, 512)):
    """The tile ``measure_dispatch`` times for ``(m, k, n)``: ``tile``, with
    bm lowered to the largest of ``DISPATCH_BM`` not above it that divides M
    when ``tile``'s does not; None when no bm fits or bn, bk do not divide."""
    bm, bn, bk = tile
    if n % bn or k % bk:
        return None
    for b in (bm,) + tuple(v for v in DISPATCH_BM if v < bm):
        if m % b == 0:
            return (b, bn, bk)
    return None


def measure_dispatch(shapes, *, tile=(1024, 1024, 512), margin=0.02, seed=0, warmups=2, runs=10, batch=5,
                     device="cuda", emit=None):
    """Same-run comparison of ``strassen_matmul`` (plain weight, as
    ``tuned_matmul`` calls it: the weight packed for every call) against
    ``native_matmul`` per ``(m, k, n)``, with calls interleaved per sample.
    A third arm, ``strassen_cached``, runs the same call with the
    packed-weight cache holding the weight (only the activation is packed
    per call). The cache's capacity is restored afterwards and its entries
    are dropped. A shape enters the table when either Strassen arm's mean is
    lower than native's by more than ``margin``; the entry says which
    (``per_call``, ``cached``), and ``tuned_matmul`` takes the cached win only
    while the cache can hold the weight. Each shape runs on
    ``dispatch_tile(m, k, n, tile)``. Each sample times ``batch``
    back-to-back calls. Returns the table ``{"shapes": {"m,k,n": {"tile":
    [...], ...}}, ...}``."""
    emit = emit or (lambda record: None)
    device = torch.device(device)
    table = {"device": _device_name(device), "tile": list(tile), "margin": margin,
             "rule": "a Strassen arm's mean below native's by more than margin, same run, interleaved samples; "
                     "per_call: the weight packed for every call, cached: the packed-weight cache holding it",
             "shapes": {}}
    for m, k, n in shapes:
        shape_tile = dispatch_tile(m, k, n, tile)
        if shape_tile is None:
            emit({"kind": "dispatch_skip", "shape": [m, k, n], "reason": f"does not tile by {tuple(tile)}"})
            continue
        bm, bn, bk = shape_tile
        x, w = _inputs(m, k, n, seed, device)

        calls = {"native": lambda: native_matmul(x, w),
                 "strassen": lambda: strassen_matmul(x, w, bm=bm, bn=bn, bk=bk)}
        calls["strassen_cached"] = calls["strassen"]
        samples = {arm: [] for arm in calls}

        def phase(arms, cache_bytes):
            """Interleaved samples of ``arms`` with the packed-weight cache at
            ``cache_bytes`` (0: the weight packed on every call, on purpose,
            so the plain-weight warning is held back)."""
            previous = cache_packed_weights(cache_bytes)
            try:
                with per_call_packing_expected():
                    for _ in range(warmups):
                        for arm in arms:
                            calls[arm]()
                    for r in range(runs):
                        for arm in (arms if r % 2 == 0 else arms[::-1]):
                            samples[arm] += time_calls(calls[arm], 0, 1, batch=batch)
            finally:
                cache_packed_weights(0)
                cache_packed_weights(previous)

        phase(("native", "strassen"), 0)
        # room for the packed weight (7/4 of its bytes): only the activation
        # is packed per call
        phase(("native", "strassen_cached"), 2 * k * n * 2)
        means = {arm: statistics.fmean(v) for arm, v in samples.items()}
        wins = means["strassen"] < (1.0 - margin) * means["native"]
        wins_cached = means["strassen_cached"] < (1.0 - margin) * means["native"]
        record = {"kind": "dispatch", "shape": [m, k, n], "tile": list(shape_tile), "mean_ms": means,
                  "samples_ms": samples, "strassen_wins": wins, "strassen_cached_wins": wins_cached,
                  "flops": 2 * m * k * n}
        emit(record)
        if wins or wins_cached:
            table["shapes"][f"{m},{k},{n}"] = {"tile": list(shape_tile), "strassen_ms": means["strassen"],
                                               "strassen_cached_ms": means["strassen_cached"],
                                               "native_ms": means["native"], "per_call": wins, "cached": wins_cached}
        del x, w
    return table


# Launches of different lengths and fill on a 256-CU MI355X (tiles are 128 x
# 128 product-space workgroups, i.e. 256 x 256 outputs): half a round and one
# round at K = 5120; one round at K = 8192, 16384 and 25600; 1.875, 2.5 and
# 3.125 rounds at K = 8192; 2.5 and 10 rounds at K = 5120.
OCCUPANCY_SHAPES = ((8192, 5120, 1024), (8192, 5120, 2048),
                    (8192, 8192, 2048), (8192, 16384, 2048), (8192, 25600, 2048),
                    (6144, 8192, 5120), (8192, 8192, 5120), (10240, 8192, 5120),
                    (8192, 5120, 5120), (8192, 5120, 20480))


def measure_occupancy(shapes=OCCUPANCY_SHAPES, *, tile=(1024, 1024, 512), seed=0, warmups=3, runs=20, batch=10,
                      device="cuda", emit=None):
    """Strassen and the matched cubic per shape on operands packed once
    (outside the timing), the arms alternating per sample of ``batch``
    back-to-back calls: the time per call, the tile count in rounds of the
    device's CUs, and the time per round of work."""
    emit = emit or (lambda record: None)
    device = torch.device(device)
    bm, bn, bk = tile
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    results = []
    for m, k, n in shapes:
        x, w = _inputs(m, k, n, seed, device)
        operands = {"strassen": (pack_activation(x, _lib.SMX_ALGO_STRASSEN, bm, bk), strassen_weight_layout(w, bn, bk)),
                    "cubic": (pack_activation(x, _lib.SMX_ALGO_CUBIC, bm, bk), cubic_weight_layout(w, bn, bk))}
        calls = {"strassen": lambda: strassen_matmul(*operands["strassen"], bm=bm, bn=bn, bk=bk),
                 "cubic": lambda: cubic_matmul(*operands["cubic"], bm=bm, bn=bn, bk=bk)}
        for call in calls.values():
            time_calls(call, warmups, 0)
        samples = {arm: [] for arm in calls}
        for r in range(runs):
            for arm in (("strassen", "cubic") if r % 2 == 0 else ("cubic", "strassen")):
                samples[arm] += time_calls(calls[arm], 0, 1, batch=batch)
        means = {arm: statistics.fmean(v) for arm, v in samples.items()}
        tiles = (m // 256) * (n // 256)
        rounds = tiles / cus
        record = {"kind": "occupancy", "shape": [m, k, n], "tile": list(tile), "tiles": tiles, "cus": cus,
                  "settings": {name: os.environ.get(name) for name in ("SMX_RASTER", "SMX_TAIL_SPLIT")},
                  "rounds": rounds, "mean_ms": means, "ms_per_round_of_work": {a: v / rounds for a, v in means.items()},
                  "strassen_speed_over_cubic": means["cubic"] / means["strassen"], "samples_ms": samples}
        emit(record)
        results.append(record)
        del operands, x, w
    return results


DECODE_TOKENS = (16, 64, 128)


def measure_decode(tokens=DECODE_TOKENS, *, k=5120, n=51200, bn=1024, bk=512, seed=0, warmups=5, runs=30, batch=10,
                   device="cuda", emit=None):
    """The Qwen3-32B gate|up site with SwiGLU at decode-sized M, a thin
    tiling (bm = 16): Strassen and the cubic on weights packed once against
    hipBLASLt's GEMM followed by torch's SwiGLU, the arms rotating per sample
    of ``batch`` back-to-back calls, with the weight bytes each arm streams
    and the rate they imply."""
    emit = emit or (lambda record: None)
    device = torch.device(device)
    _, w = _inputs(16, k, n, seed, device)
    laid = swiglu_weight_layout(w, bn)
    weights = {"strassen": strassen_weight_layout(laid, bn, bk), "cubic": cubic_weight_layout(laid, bn, bk)}
    weight_bytes = {"strassen": weights["strassen"].data.numel() * 2, "cubic": weights["cubic"].data.numel() * 2,
                    "hipblaslt": w.numel() * 2}
    results = []
    for m in tokens:
        g = torch.Generator(device=device).manual_seed(seed + m)
        x = torch.randn(m, k, device=device, generator=g).to(torch.bfloat16)
        calls = {"strassen": lambda: strassen_matmul(x, weights["strassen"], bm=16, bn=bn, bk=bk, epilogue="swiglu"),
                 "cubic": lambda: cubic_matmul(x, weights["cubic"], bm=16, bn=bn, bk=bk, epilogue="swiglu"),
                 "hipblaslt": lambda: _activate(native_matmul(x, w))}
        for call in calls.values():
            time_calls(call, warmups, 0)
        samples = {arm: [] for arm in calls}
        names = list(calls)
        for r in range(runs):
            for arm in names[r % 3:] + names[:r % 3]:
                samples[arm] += time_calls(calls[arm], 0, 1, batch=batch)
        means = {arm: statistics.fmean(v) for arm, v in samples.items()}
        record = {"kind": "decode", "shape": [m, k, n], "tile": [16, bn, bk], "mean_ms": means,
                  "weight_bytes": weight_bytes,
                  "weight_stream_tb_per_s": {a: weight_bytes[a] / (v * 1e-3) / 1e12 for a, v in means.items()},
                  "samples_ms": samples}
        emit(record)
        results.append(record)
    return results


# Launches with few tiles: the Qwen3-32B down and o projections and the k
# projection at decode-sized and prefill-chunk M ((m, k, n, bm): 20-40 tiles
# on 256 CUs), and the k/v projection at 8192 tokens (128 tiles).
SMALL_LAUNCH_SHAPES = ((16, 25600, 5120, 16), (16, 8192, 5120, 16), (128, 25600, 5120, 128),
                       (256, 25600, 5120, 256), (512, 25600, 5120, 512), (16, 5120, 1024, 16),
                       (8192, 5120, 1024, 256))


def measure_small_launches(shapes=SMALL_LAUNCH_SHAPES, *, bn=256, bk=512, seed=0, warmups=3, runs=10, batch=10,
                           device="cuda", emit=None):
    """Strassen and the cubic on operands packed once (outside the timing),
    no epilogue, against hipBLASLt, on launches whose few tiles leave most
    CUs idle unless the K split spreads them; the arms rotate per sample of
    ``batch`` back-to-back calls. The split's share count comes from the
    library (``smx_gemm_workspace_bytes``); run once as is and once with
    SMX_TAIL_SPLIT=0 to time the whole tiles."""
    emit = emit or (lambda record: None)
    device = torch.device(device)
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    results = []
    for m, k, n, bm in shapes:
        x, w = _inputs(m, k, n, seed, device)
        packed = {algo: (pack_activation(x, algo, bm, bk),
                         (strassen_weight_layout if algo == _lib.SMX_ALGO_STRASSEN else cubic_weight_layout)(w, bn, bk))
                  for algo in (_lib.SMX_ALGO_STRASSEN, _lib.SMX_ALGO_CUBIC)}
        calls = {"strassen": lambda: strassen_matmul(*packed[_lib.SMX_ALGO_STRASSEN], bm=bm, bn=bn, bk=bk),
                 "cubic": lambda: cubic_matmul(*packed[_lib.SMX_ALGO_CUBIC], bm=bm, bn=bn, bk=bk),
                 "hipblaslt": lambda: native_matmul(x, w)}
        for call in calls.values():
            time_calls(call, warmups, 0)
        samples = {arm: [] for arm in calls}
        names = list(calls)
        for r in range(runs):
            for arm in names[r % 3:] + names[:r % 3]:
                samples[arm] += time_calls(calls[arm], 0, 1, batch=batch)
        tiles = -(-(m // 2) // 128) * (n // 256)
        record = {"kind": "small_launch", "shape": [m, k, n], "tile": [bm, bn, bk], "tiles": tiles, "cus": cus,
                  "k_shares": _lib.k_shares(m, k, n, (bm, bn, bk)),
                  "median_ms": {arm: statistics.median(v) for arm, v in samples.items()}, "samples_ms": samples}
        emit(record)
        results.append(record)
        del x, w, packed
    return results


# Kernels one pure GEMM launch can run on (measure_launches).
LAUNCH_ARMS = ("hipblaslt", "cubic", "strassen", "product_major", "product_major_rounds")


def measure_launches(arm, m, k, n, *, tile=(1024, 1024, 512), calls=10, seed=0, device="cuda:0", emit=None):
    """``calls`` timed launches of one pure bf16 GEMM (no epilogue) on one
    kernel, for counter runs under a profiler: ``hipblaslt`` (torch.matmul
    on an ``[in, out]`` view of an ``[out, in]`` weight), or ``cubic`` /
    ``strassen`` / ``product_major`` / ``product_major_rounds`` through
    ``smx_gemm`` on operands packed beforehand (the product-major kernel with
    SMX_FLAG_PRODUCT_MAJOR, or on whole rounds with
    SMX_FLAG_PRODUCT_MAJOR_ROUNDS). One
    untimed launch first; returns the per-launch milliseconds (HIP events)."""
    import ctypes

    if arm not in LAUNCH_ARMS:
        raise ValueError(f"arm must be one of {LAUNCH_ARMS}")
    emit = emit or (lambda record: None)
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    a = torch.randn(m, k, device=dev, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, device=dev, generator=g) * 0.02).to(torch.bfloat16).t()
    if arm == "hipblaslt":
        call = lambda: torch.matmul(a, w)  # noqa: E731
    else:
        algo = _lib.SMX_ALGO_CUBIC if arm == "cubic" else _lib.SMX_ALGO_STRASSEN
        bm, bn, bk = tile
        pa = pack_operand(a, algo=algo, side="lhs", tile_rows=bm, bk=bk)
        pb = pack_operand(w, algo=algo, side="rhs", tile_rows=bn, bk=bk)
        lib = _lib.load()
        d = _lib.SmxGemmDesc()
        d.m, d.n, d.k = m, n, k
        d.lda, d.ldb, d.ldc = k, k, n
        d.bm, d.bn, d.bk = tile
        d.algo, d.epilogue = algo, _lib.SMX_EPI[None]
        d.a_layout, d.b_layout = _lib.SMX_A_PACKED, _lib.SMX_B_PACKED
        d.flags = {"product_major": _lib.SMX_FLAG_PRODUCT_MAJOR,
                   "product_major_rounds": _lib.SMX_FLAG_PRODUCT_MAJOR_ROUNDS}.get(arm, 0)
        need = ctypes.c_int64()
        _lib.check(lib.smx_gemm_workspace_bytes(d, ctypes.byref(need)))
        workspace = None
        if need.value:
            workspace = torch.empty(need.value, dtype=torch.uint8, device=dev)
            d.workspace, d.workspace_bytes = workspace.data_ptr(), need.value
        out = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)

        def call():
            _lib.check(lib.smx_gemm(d, _lib.ptr(pa.data), _lib.ptr(pb.data), _lib.ptr(out), None, None, None, None,
                                    None, stream))
    call()
    torch.cuda.synchronize(dev)
    times = []
    for _ in range(calls):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        call()
        stop.record()
        torch.cuda.synchronize(dev)
        times.append(start.elapsed_time(stop))
    emit({"kind": "launches", "arm": arm, "shape": [m, k, n], "tile": list(tile), "ms": times,
          "tflops": 2.0 * m * n * k / (statistics.fmean(times) * 1e-3) / 1e12})
    return times


_TABLE = None


def load_table(path=None):
    """The dispatch table (``measure_dispatch`` output) from ``path``,
    ``$SMX_TUNED_TABLE`` or the shipped ``tuned_shapes.json``."""
    global _TABLE
    path = path or os.environ.get("SMX_TUNED_TABLE") or DEFAULT_TABLE
    if _TABLE is None or _TABLE[0] != path:
        with open(path) as f:
            _TABLE = (path, json.load(f))
    return _TABLE[1]


def _entry_wins(entry, b):
    """Whether a table entry's measured win holds for a call on the weight
    ``b [K, N]``: a win with the weight packed per call always does; a win
    measured with the packed weight cached holds only when the cache has
    this weight's packed form (7/4 of its bf16 bytes) or can add it without
    evicting another. A working set the cache cannot hold therefore stays on
    the native GEMM for the weights beyond it, instead of packing them on
    every call (the per-call arm, which lost)."""
    if entry.get("per_call", True):
        return True
    if not entry.get("cached"):
        return False
    k, n = b.shape
    _, bn, bk = entry["tile"]
    return weight_cached_or_fits(b, algo=_lib.SMX_ALGO_STRASSEN, bn=bn, bk=bk, packed_bytes=7 * k * n // 2)


def tuned_matmul(a, b, *, interpret=False):
    """Dispatch measured bf16 shapes to Strassen, everything else to the
    native GEMM (``strassen_pallas.py:1428-1461``). A shape goes to Strassen
    only if it is in the measured table with a win that holds for the call
    (per call, or with the weight's packed form cached or fitting in the
    packed-weight cache), both operands are
    2-D bf16 with matching K, and the table's tile divides it."""
    if a.dim() != 2 or b.dim() != 2:
        return native_matmul(a, b)
    m, k = a.shape
    k2, n = b.shape
    entry = load_table()["shapes"].get(f"{m},{k},{n}")
    use_strassen = (entry is not None and k == k2 and a.dtype == torch.bfloat16 and b.dtype == torch.bfloat16
                    and m % entry["tile"][0] == 0 and n % entry["tile"][1] == 0 and k % entry["tile"][2] == 0
                    and _entry_wins(entry, b))
    if not use_strassen:
        return native_matmul(a, b)
    bm, bn, bk = entry["tile"]
    return strassen_matmul(a, b, bm=bm, bn=bn, bk=bk, interpret=interpret)


# Shapes timed for the shipped table: the reference's square crossover and
# projection shapes (strassen_pallas.py:49-72), the Qwen3-32B GEMM sites at
# 8192 tokens, and its q, o, gate-or-up and down projections at 128, 256 and
# 512 tokens (launches that the K split spreads over the chip).
DISPATCH_SHAPES = (
    (4096, 4096, 4096), (8192, 8192, 8192), (16384, 16384, 16384),
    (8192, 4096, 8192), (8192, 4096, 12288), (8192, 4096, 28672), (8192, 14336, 4096),
    (8192, 5120, 8192), (8192, 5120, 1024), (8192, 8192, 5120), (8192, 5120, 25600), (8192, 5120, 51200),
    (8192, 25600, 5120),
) + tuple((m, k, n) for m in (128, 256, 512)
          for k, n in ((5120, 8192), (8192, 5120), (5120, 25600), (25600, 5120)))


def main(argv=None):
    ap = argparse.ArgumentParser(description="gfx950 tile screen and dispatch-table measurement")
    sub = ap.add_subparsers(dest="command", required=True)
    screen = sub.add_parser("screen", help="fixed-budget tile screen of one GEMM geometry")
    screen.add_argument("--shape", default="8192,5120,51200", help="m,k,n (default: Qwen3-32B gate|up)")
    screen.add_argument("--no-swiglu", action="store_true")
    screen.add_argument("--warmups", type=int, default=2)
    screen.add_argument("--runs", type=int, default=5)
    dispatch = sub.add_parser("dispatch", help="measure Strassen against the native GEMM per shape")
    dispatch.add_argument("--runs", type=int, default=10)
    dispatch.add_argument("--table", default=None, help="write the dispatch table here")
    occupancy = sub.add_parser("occupancy", help="Strassen and cubic on launches that fill part of the chip")
    occupancy.add_argument("--runs", type=int, default=20)
    occupancy.add_argument("--shapes", default=None,
                           help="M,K,N shapes separated by ';' (default: OCCUPANCY_SHAPES)")
    decode = sub.add_parser("decode", help="the gate|up site with SwiGLU at decode-sized M (thin tiling)")
    decode.add_argument("--runs", type=int, default=30)
    small = sub.add_parser("small", help="Strassen, cubic and hipBLASLt on launches with few tiles (the K split)")
    small.add_argument("--runs", type=int, default=10)
    launches = sub.add_parser("launches", help="timed launches of one pure GEMM on one kernel (for counter runs)")
    launches.add_argument("--arm", choices=LAUNCH_ARMS, required=True)
    launches.add_argument("--shape", default="8192,5120,25600", help="m,k,n (default: a Qwen3-32B gate or up)")
    launches.add_argument("--calls", type=int, default=10)
    for p in (screen, dispatch, occupancy, decode, small, launches):
        p.add_argument("--out", default=None, help="also append the JSON records to this file")
    args = ap.parse_args(argv)
    sink = open(args.out, "a") if args.out else None

    def emit(record):
        line = json.dumps(record, sort_keys=True)
        print(line, flush=True)
        if sink:
            sink.write(line + "\n")
            sink.flush()

    _lib.load()
    if args.command == "screen":
        m, k, n = (int(v) for v in args.shape.split(","))
        screen_tiles(m, k, n, swiglu=not args.no_swiglu, warmups=args.warmups, runs=args.runs, emit=emit)
    elif args.command == "occupancy":
        shapes = OCCUPANCY_SHAPES
        if args.shapes:
            shapes = tuple(tuple(int(v) for v in shape.split(",")) for shape in args.shapes.split(";"))
        measure_occupancy(shapes, runs=args.runs, emit=emit)
    elif args.command == "decode":
        measure_decode(runs=args.runs, emit=emit)
    elif args.command == "small":
        measure_small_launches(runs=args.runs, emit=emit)
    elif args.command == "launches":
        m, k, n = (int(v) for v in args.shape.split(","))
        measure_launches(args.arm, m, k, n, calls=args.calls, emit=emit)
    else:
        table = measure_dispatch(DISPATCH_SHAPES, runs=args.runs, emit=emit)
        emit({"kind": "table", **table})
        if args.table:
            with open(args.table, "w") as f:
                json.dump(table, f, indent=1, sort_keys=True)
                f.write("\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
