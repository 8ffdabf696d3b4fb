"""The result records of `bench.py --results` against the reference harness's format
(metal_infrence_engine/src/bin/bench.rs:193-226, mlx_baseline/results/engine_metal_m1_ai.json)."""
import json
import os

import harness

# the keys of the reference's engine_metal_m1_ai.json and of its "decode" object
ENGINE_KEYS = {"engine", "label", "timestamp", "commit", "dirty", "chip", "prompt_name", "prompt_tokens",
               "load_ms", "decode", "parity_vs_mlx", "tokens"}
DECODE_KEYS = {"steps", "median_ms", "tps", "achieved_bw_gbs", "mbu", "weight_bytes_per_token", "samples_ms"}


def _record(**kw):
    args = dict(engine="hip", label="t", chip="AMD Instinct MI355X", prompt_name="random130", prompt_tokens=130,
                load_ms=12.5, step_ms=[1.0, 0.5, 0.75, 0.5], tokens=[5, 6, 7, 8, 9], weight_bytes_per_token=1000,
                total_bytes=4000 + 40, peak_bw_gbs=8000.0, ref_tokens=[5, 6, 9, 8], repo_dir="/nonexistent")
    args.update(kw)
    return harness.engine_record(**args)


def test_record_has_the_reference_keys_and_arithmetic():
    r = _record()
    assert set(r) == ENGINE_KEYS and set(r["decode"]) == DECODE_KEYS
    d = r["decode"]
    assert d["steps"] == 4
    assert r["tokens"] == [5, 6, 7, 8]  # truncated to the step count (bench.rs:185)
    assert d["median_ms"] == 0.75  # upper median (bench.rs:123-128)
    assert abs(d["tps"] - 4 / 2.75e-3) < 1e-6
    assert abs(d["achieved_bw_gbs"] - 4040 / 2.75e-3 / 1e9) < 1e-12
    assert abs(d["mbu"] - d["achieved_bw_gbs"] / 8000.0) < 1e-15
    assert r["parity_vs_mlx"] == {"compared": 4, "first_divergence": 2}
    assert r["commit"] == "" and r["dirty"] is False  # no git checkout: as bench.rs's sh() fallback
    assert _record(ref_tokens=[5, 6, 7, 8, 1])["parity_vs_mlx"] == {"compared": 4, "first_divergence": None}


def test_chip_slug_matches_the_reference_rule():
    assert harness.chip_slug("Apple M1 Pro") == "m1_pro"
    assert harness.chip_slug("Apple M1") == "m1"
    assert harness.chip_slug("AMD Instinct MI355X") == "amd_instinct_mi355x"


def test_files_latest_and_history(tmp_path):
    d = str(tmp_path)
    p1 = harness.write_records(d, _record(label="a"))
    p2 = harness.write_records(d, _record(label="b"))
    assert p1 == p2 == os.path.join(d, "engine_hip_amd_instinct_mi355x_random130.json")
    with open(p1) as f:
        assert json.load(f)["label"] == "b"
    with open(os.path.join(d, "history_amd_instinct_mi355x_random130.jsonl")) as f:
        lines = [json.loads(x) for x in f]
    assert [x["label"] for x in lines] == ["a", "b"]
