"""The tile screen and the measured dispatcher on the GPU, at a small
geometry: the screen times every kept candidate for both arms and picks a
kept tile; tuned_matmul sends a tabled shape to Strassen (bit-identical to a
direct call) and anything else to the native GEMM."""

import json
import os

import pytest
import torch

import strassen_tpu_amd as smx
from strassen_tpu_amd import tuning

pytestmark = pytest.mark.gpu


def test_small_tile_screen():
    records = []
    chosen = tuning.screen_tiles(1024, 1024, 2048, swiglu=True, warmups=1, runs=2, emit=records.append,
                                 bm_candidates=(512, 1024), bn_candidates=(512, 1024), bk_candidates=(256, 512))
    kept = [tuple(e["tile"]) for e in records[0]["candidates"]]
    assert len(kept) == 8
    tunes = [r for r in records if r["kind"] == "tune" and r["arm"] != "hipblaslt"]
    assert len(tunes) == 2 * len(kept) and all(len(r["samples_ms"]) == 2 for r in tunes)
    for arm in ("strassen", "cubic"):
        assert tuple(chosen[arm]["tile"]) in kept
        best = min((r for r in tunes if r["arm"] == arm), key=lambda r: r["mean_ms"])
        assert chosen[arm]["mean_ms"] == best["mean_ms"]
    assert records[-1] == {"kind": "verdict", "passes": True, "scope": "tile screening; winners feed the harnesses"}


def test_tuned_matmul_dispatch(tmp_path, monkeypatch):
    path = tmp_path / "table.json"
    path.write_text(json.dumps({"shapes": {"512,1024,512": {"tile": [256, 256, 512], "strassen_ms": 1.0,
                                                           "native_ms": 2.0}}}))
    monkeypatch.setenv("SMX_TUNED_TABLE", str(path))
    g = torch.Generator(device="cuda").manual_seed(1)
    a = torch.randn(512, 1024, device="cuda", generator=g).to(torch.bfloat16)
    b = (torch.randn(512, 1024, device="cuda", generator=g) * 0.02).to(torch.bfloat16).t()
    got = tuning.tuned_matmul(a, b)
    assert torch.equal(got, smx.strassen_matmul(a, b, bm=256, bn=256, bk=512))
    c = (torch.randn(1024, 1024, device="cuda", generator=g) * 0.02).to(torch.bfloat16)
    assert torch.equal(tuning.tuned_matmul(a, c), smx.native_matmul(a, c))


def test_dispatch_measurement_records():
    records = []
    table = tuning.measure_dispatch([(512, 1024, 1024), (500, 1024, 1024)], tile=(256, 256, 512), runs=2,
                                    emit=records.append)
    assert records[0]["kind"] == "dispatch"
    samples = records[0]["samples_ms"]
    # hipBLASLt is sampled in both phases (per-call packing, cached weight)
    assert len(samples["native"]) == 4 and len(samples["strassen"]) == 2 and len(samples["strassen_cached"]) == 2
    # the measurement restores the cache's capacity and leaves no entry of its own
    assert smx.packed_weight_cache_info()["entries"] == 0
    assert records[1]["kind"] == "dispatch_skip"
    for key, entry in table["shapes"].items():
        assert entry["per_call"] or entry["cached"]
        assert entry["strassen_ms"] < entry["native_ms"] or entry["strassen_cached_ms"] < entry["native_ms"]


def test_occupancy_and_decode_measurements():
    """The occupancy and decode measurements run and record what they
    claim (small shapes, two samples each)."""
    occ = tuning.measure_occupancy([(512, 1024, 512)], tile=(256, 256, 512), warmups=1, runs=2)
    assert occ[0]["tiles"] == 4 and occ[0]["rounds"] == 4 / occ[0]["cus"]
    assert set(occ[0]["mean_ms"]) == {"strassen", "cubic"} and all(v > 0 for v in occ[0]["mean_ms"].values())
    dec = tuning.measure_decode((16,), k=1024, n=2048, bn=512, bk=512, warmups=1, runs=3)
    assert dec[0]["shape"] == [16, 1024, 2048]
    assert dec[0]["weight_bytes"]["strassen"] == 7 * dec[0]["weight_bytes"]["hipblaslt"] // 4
    assert all(len(v) == 3 for v in dec[0]["samples_ms"].values())


@pytest.mark.parametrize("m", [256, 8192])
def test_shipped_cached_entry_routes_with_the_cache(monkeypatch, m):
    """The shipped table's down projection at 256 and 8192 tokens won with
    the packed-weight cache: tuned_matmul sends it to Strassen (bit-identical
    to the direct call on the entry's tile) while the cache can hold the
    weight, and to the native GEMM without the cache."""
    monkeypatch.delenv("SMX_TUNED_TABLE", raising=False)
    entry = tuning.load_table(tuning.DEFAULT_TABLE)["shapes"].get(f"{m},25600,5120")
    if entry is None:
        pytest.skip("the shipped table was measured without this shape")
    g = torch.Generator(device="cuda").manual_seed(3)
    a = torch.randn(m, 25600, device="cuda", generator=g).to(torch.bfloat16)
    w = (torch.randn(5120, 25600, device="cuda", generator=g) * 0.02).to(torch.bfloat16).t()
    previous = smx.cache_packed_weights(0)
    try:
        assert torch.equal(tuning.tuned_matmul(a, w), smx.native_matmul(a, w))
        smx.cache_packed_weights(1 << 30)
        bm, bn, bk = entry["tile"]
        got = tuning.tuned_matmul(a, w)
        assert torch.equal(got, smx.strassen_matmul(a, w, bm=bm, bn=bn, bk=bk))
        assert smx.packed_weight_cache_info()["hits"] >= 1
    finally:
        smx.cache_packed_weights(0)
        smx.cache_packed_weights(previous)


def test_small_launch_measurement():
    """The small-launch measurement records the library's share count (at
    least two for 20 tiles over K = 4096) and samples every arm."""
    rec = tuning.measure_small_launches([(16, 4096, 5120, 16)], warmups=1, runs=3, batch=2)[0]
    split_off = os.environ.get("SMX_TAIL_SPLIT", "").startswith("0")
    assert rec["tiles"] == 20 and (rec["k_shares"] == 1 if split_off else rec["k_shares"] >= 2)
    assert set(rec["median_ms"]) == {"strassen", "cubic", "hipblaslt"}
    assert all(len(v) == 3 for v in rec["samples_ms"].values())


@pytest.mark.parametrize("arm", tuning.LAUNCH_ARMS)
def test_measure_launches_every_arm(arm):
    """`tuning launches` (the driver of the hipBLASLt comparison's counter
    runs) times each kernel on a pure GEMM: one untimed launch, then the
    asked-for number of positive times, in one emitted record."""
    records = []
    times = tuning.measure_launches(arm, 1024, 1024, 2048, calls=3, emit=records.append)
    assert len(times) == 3 and all(t > 0 for t in times)
    assert len(records) == 1 and records[0]["kind"] == "launches" and records[0]["arm"] == arm
    assert records[0]["shape"] == [1024, 1024, 2048] and records[0]["tflops"] > 0
    with pytest.raises(ValueError, match="arm must be one of"):
        tuning.measure_launches("xla", 1024, 1024, 2048)
