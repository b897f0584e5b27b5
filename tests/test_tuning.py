"""Host logic of the tile screen and the measured dispatcher (no GPU):
candidate enumeration under the gfx950 tile rule and the reference's
screening rules (benchmark_qwen3_scaling_tile_tune.py:103-133), and
tuned_matmul's dispatch conditions (strassen_pallas.py:1428-1461)."""

import json

import pytest
import torch

from strassen_tpu_amd import tuning


def test_enumeration_for_the_qwen3_32b_gate_up_geometry():
    kept, filtered = tuning.enumerate_candidates(8192, 5120, 51200, paired_width=25600)
    tiles = [tuple(e["tile"]) for e in kept]
    # 2560 halves to 1280, which divides the gate width; every bm and bk fits
    assert (1024, 1024, 512) in tiles and (2048, 2560, 1024) in tiles
    assert len(kept) + len(filtered) == 3 * 4 * 3
    # enumeration order is bm-major, then bn, then bk (ties go to the earlier)
    assert tiles == sorted(tiles, key=lambda t: (tuning.BM_CANDIDATES.index(t[0]),
                                                 tuning.BN_CANDIDATES.index(t[1]),
                                                 tuning.BK_CANDIDATES.index(t[2])))
    for e in filtered:
        assert e["filtered_because"]


def test_enumeration_reasons():
    kept, filtered = tuning.enumerate_candidates(1024, 768, 3072, paired_width=1536, bm_candidates=(512, 384),
                                                 bn_candidates=(1024, 2048), bk_candidates=(256, 96))
    assert [tuple(e["tile"]) for e in kept] == [(512, 1024, 256)]
    reasons = {tuple(e["tile"]): e["filtered_because"] for e in filtered}
    assert reasons[(512, 1024, 96)] == ["gfx950 tile rule"]  # 96 divides K but breaks bk % 64
    assert reasons[(512, 2048, 256)] == ["N 3072 % bn"]
    assert reasons[(384, 1024, 256)] == ["M 1024 % bm", "gfx950 tile rule"]
    _, filtered = tuning.enumerate_candidates(1024, 768, 3072, paired_width=1280, bm_candidates=(512,),
                                              bn_candidates=(1024,), bk_candidates=(256,))
    assert filtered[0]["filtered_because"] == ["gate width 1280 % (bn//2)"]


@pytest.fixture
def table(tmp_path, monkeypatch):
    path = tmp_path / "table.json"
    path.write_text(json.dumps({"shapes": {"512,1024,512": {"tile": [256, 256, 512]}}}))
    monkeypatch.setenv("SMX_TUNED_TABLE", str(path))
    calls = []
    monkeypatch.setattr(tuning, "native_matmul", lambda a, b: calls.append("native") or "native")
    monkeypatch.setattr(tuning, "strassen_matmul",
                        lambda a, b, **kw: calls.append(("strassen", kw["bm"], kw["bn"], kw["bk"])) or "strassen")
    return calls


def z(*shape, dtype=torch.bfloat16):
    return torch.zeros(*shape, dtype=dtype)


def test_tuned_matmul_dispatch_rules(table):
    assert tuning.tuned_matmul(z(512, 1024), z(1024, 512)) == "strassen"
    assert table[-1] == ("strassen", 256, 256, 512)
    # not a measured shape, wrong dtype, rank-3, K mismatch: native
    assert tuning.tuned_matmul(z(512, 1024), z(1024, 1024)) == "native"
    assert tuning.tuned_matmul(z(512, 1024, dtype=torch.float32), z(1024, 512, dtype=torch.float32)) == "native"
    assert tuning.tuned_matmul(z(2, 512, 1024), z(1024, 512)) == "native"
    assert tuning.tuned_matmul(z(512, 1024), z(1000, 512)) == "native"


def test_cached_win_needs_the_cache(table, tmp_path, monkeypatch):
    """An entry that won only with the packed-weight cache goes to Strassen
    only while the cache holds the weight's packed form (7/4 of 2 K N bytes)
    or can add it without evicting another: with room for one packed weight
    and calls cycling over two weights, the first weight stays on Strassen
    and the second goes native, instead of both missing and repacking on
    every call."""
    from strassen_tpu_amd import packing

    path = tmp_path / "cached.json"
    path.write_text(json.dumps({"shapes": {"128,1024,512": {"tile": [128, 256, 512], "per_call": False,
                                                            "cached": True}}}))
    monkeypatch.setenv("SMX_TUNED_TABLE", str(path))
    packed_bytes = 7 * 1024 * 512 // 2
    cache = packing._WeightCache(0)
    monkeypatch.setattr(packing, "_WEIGHT_CACHE", cache)

    class Packed:  # stands in for a PackedOperand of packed_bytes
        data = torch.zeros(packed_bytes, dtype=torch.uint8)

    def strassen(a, b, **kw):
        # what strassen_matmul does with a plain weight: the cached lookup
        cache.lookup(b, packing._weight_packing(7, kw["bn"], kw["bk"]), Packed)
        table.append(("strassen", kw["bm"], kw["bn"], kw["bk"]))
        return "strassen"

    monkeypatch.setattr(tuning, "strassen_matmul", strassen)
    w1, w2 = z(1024, 512), z(1024, 512)
    assert tuning.tuned_matmul(z(128, 1024), w1) == "native"  # cache off
    cache.resize(packed_bytes - 1)
    assert tuning.tuned_matmul(z(128, 1024), w1) == "native"  # no room
    cache.resize(packed_bytes)
    assert tuning.tuned_matmul(z(128, 1024), w1) == "strassen"  # room: packed and kept
    assert table[-1] == ("strassen", 128, 256, 512)
    for _ in range(3):
        assert tuning.tuned_matmul(z(128, 1024), w2) == "native"  # would evict w1
        assert tuning.tuned_matmul(z(128, 1024), w1) == "strassen"  # cached
    assert cache.misses == 1 and cache.hits == 3
    assert tuning.tuned_matmul(z(128, 1024), w1.t().contiguous().t()) == "native"  # another tensor, no room


def test_weight_cache_entries_follow_their_weights():
    """Entries hold weak references: freeing a weight (or the base of the
    view passed) drops its entry and its packed bytes; an in-place update
    (the shared version counter) makes the next lookup pack again; contains()
    packs nothing; views of one base share an entry per geometry."""
    from strassen_tpu_amd import packing

    cache = packing._WeightCache(1 << 20)
    made = []

    def make():
        made.append(1)

        class Packed:
            data = torch.zeros(1000, dtype=torch.uint8)
        return Packed

    key = ("k",)
    base = torch.zeros(64, 32, dtype=torch.bfloat16)  # stored [out, in]; the call passes base.t()
    assert not cache.contains(base.t(), key)
    cache.lookup(base.t(), key, make)
    assert cache.contains(base.t(), key) and len(made) == 1
    cache.lookup(base.t(), key, make)  # a fresh view of the same base: a hit
    assert len(made) == 1 and cache.hits == 1 and cache.bytes == 1000
    base.add_(1)  # in place, through the base: the view's entry is stale
    assert not cache.contains(base.t(), key) and cache.stale == 1 and cache.bytes == 0
    cache.lookup(base.t(), key, make)
    assert len(made) == 2 and cache.bytes == 1000
    del base
    import gc
    gc.collect()
    assert len(cache.entries) == 0 and cache.bytes == 0
    assert cache.has_room(1 << 20) and not cache.has_room((1 << 20) + 1)


def test_dispatch_tile():
    assert tuning.dispatch_tile(8192, 5120, 25600) == (1024, 1024, 512)
    assert tuning.dispatch_tile(256, 25600, 5120) == (256, 1024, 512)
    assert tuning.dispatch_tile(384, 1024, 1024) == (128, 1024, 512)
    assert tuning.dispatch_tile(48, 1024, 1024) == (16, 1024, 512)
    assert tuning.dispatch_tile(500, 1024, 1024, (256, 256, 512)) is None  # no bm % 16 divides 500
    assert tuning.dispatch_tile(1024, 1000, 1024) is None and tuning.dispatch_tile(1024, 1024, 1000) is None


def test_shipped_table_is_well_formed():
    table = tuning.load_table(tuning.DEFAULT_TABLE)
    assert {"device", "tile", "margin", "rule", "shapes"} <= set(table)
    for key, entry in table["shapes"].items():
        m, k, n = (int(v) for v in key.split(","))
        bm, bn, bk = entry["tile"]
        assert m % bm == 0 and n % bn == 0 and k % bk == 0
        assert entry["per_call"] or entry["cached"]
        if entry["per_call"]:
            assert entry["strassen_ms"] < entry["native_ms"]
        if entry["cached"]:
            assert entry["strassen_cached_ms"] < entry["native_ms"]
