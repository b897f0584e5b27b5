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
    only while the cache can hold the packed weight (7/4 of 2 K N bytes)."""
    path = tmp_path / "cached.json"
    path.write_text(json.dumps({"shapes": {"128,1024,512": {"tile": [128, 256, 512], "per_call": False,
                                                            "cached": True}}}))
    monkeypatch.setenv("SMX_TUNED_TABLE", str(path))
    capacity = {"capacity": 0}
    monkeypatch.setattr(tuning, "packed_weight_cache_info", lambda: dict(capacity))
    assert tuning.tuned_matmul(z(128, 1024), z(1024, 512)) == "native"
    capacity["capacity"] = 7 * 1024 * 512 // 2 - 1
    assert tuning.tuned_matmul(z(128, 1024), z(1024, 512)) == "native"
    capacity["capacity"] = 7 * 1024 * 512 // 2
    assert tuning.tuned_matmul(z(128, 1024), z(1024, 512)) == "strassen"
    assert table[-1] == ("strassen", 128, 256, 512)


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
