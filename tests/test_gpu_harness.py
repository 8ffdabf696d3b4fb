"""The measurement path on the GPU: a real decode written through the reference harness's record
format (metal_infrence_engine/src/bin/bench.rs:193-226; keys of
mlx_baseline/results/engine_metal_m1_ai.json), and the read-bandwidth ceiling with the reference's
anti-cache bound (tests/read_bandwidth.rs:139-140)."""
import json
import os
import time

import numpy as np
import pytest

import harness
import qe
from conftest import DECODE_STEPS, PROMPT_LEN, PROMPT_SEED

pytestmark = pytest.mark.gpu

ENGINE_KEYS = {"engine", "label", "timestamp", "commit", "dirty", "chip", "prompt_name", "prompt_tokens",
               "load_ms", "decode", "parity_vs_mlx", "tokens"}
DECODE_KEYS = {"steps", "median_ms", "tps", "achieved_bw_gbs", "mbu", "weight_bytes_per_token", "samples_ms"}


@pytest.mark.slow
def test_real_decode_record(gpu, real_ckpt, tmp_path):
    import torch
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qwen3_0_6b_decode.npz"),
                allow_pickle=False)
    t0 = time.time()
    m = qe.Model.load_model(real_ckpt)
    load_ms = (time.time() - t0) * 1e3
    V = m.config().vocab_size
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, V)
    cache = qe.KVCache(m, PROMPT_LEN + DECODE_STEPS + 1)
    first = int(np.argmax(m.prefill(prompt, 0, cache)))
    gaps, last = [], [time.perf_counter()]

    def on_token(_t):
        now = time.perf_counter()
        gaps.append((now - last[0]) * 1e3)
        last[0] = now

    toks, _ = m.decode(first, PROMPT_LEN, DECODE_STEPS, cache, on_token=on_token)
    wb = m.weight_bytes_per_token()
    total = DECODE_STEPS * wb + sum(m.kv_bytes_at(p) for p in range(PROMPT_LEN, PROMPT_LEN + DECODE_STEPS))
    rec = harness.engine_record(
        engine="hip", label="test", chip=torch.cuda.get_device_name(0), prompt_name="random130",
        prompt_tokens=PROMPT_LEN, load_ms=load_ms, step_ms=gaps, tokens=[first] + toks,
        weight_bytes_per_token=wb, total_bytes=total, peak_bw_gbs=8000.0,
        ref_tokens=[int(t) for t in g["tokens"]], repo_dir=str(tmp_path))
    path = harness.write_records(str(tmp_path), rec)
    with open(path) as f:
        r = json.load(f)
    assert set(r) == ENGINE_KEYS and set(r["decode"]) == DECODE_KEYS
    d = r["decode"]
    assert d["steps"] == DECODE_STEPS and len(d["samples_ms"]) == DECODE_STEPS
    assert r["tokens"] == [int(t) for t in g["tokens"][:DECODE_STEPS]]
    assert r["parity_vs_mlx"] == {"compared": DECODE_STEPS, "first_divergence": None}
    assert d["weight_bytes_per_token"] == 1_192_101_888
    assert d["tps"] > 0 and 0 < d["mbu"] < 1
    assert abs(d["achieved_bw_gbs"] - total / (sum(gaps) / 1e3) / 1e9) < 1e-6 * d["achieved_bw_gbs"]
    hist = os.path.join(str(tmp_path), f"history_{harness.chip_slug(r['chip'])}_random130.jsonl")
    with open(hist) as f:
        assert json.loads(f.readline())["tokens"] == r["tokens"]


def test_read_ceiling_is_below_spec(gpu):
    import torch

    import bench
    gbs = bench.measured_read_ceiling(torch, qe)
    print(f"measured streaming-read ceiling: {gbs:.1f} GB/s")
    assert 0 < gbs <= 1.05 * bench.SPEC_HBM_GBS
