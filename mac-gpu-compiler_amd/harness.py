"""Result records in the reference harness's format (metal_infrence_engine/src/bin/bench.rs:193-226).

The reference's bench writes its latest run to `engine_<engine>_<chip slug>_<prompt>.json` and
appends every run to `history_<chip slug>_<prompt>.jsonl` under `mlx_baseline/results`, which
`mlx_baseline/compare.py` turns into a scoreboard and a history chart. `bench.py --results DIR`
writes the same two files with the same keys, so those tools read this engine's runs beside the
Metal and CPU ones. Differences: the engine name is "hip", `peak` for `mbu` is the MI355X HBM
spec, and `parity_vs_mlx` compares against the token list the caller passes (the CPU
reference's greedy tokens for the same weights and prompt: MLX never ran these random weights).
"""
import json
import os
import subprocess
import time


def chip_slug(chip: str) -> str:
    """bench.rs:94 (and mlx_baseline/bench.py): "Apple M1 Pro" -> "m1_pro"."""
    return chip.replace("Apple ", "").replace(" ", "_").lower()


def median(xs):
    """bench.rs:123-128: the upper median of the samples."""
    s = sorted(xs)
    return s[len(s) // 2]


def _git(args, cwd):
    try:
        return subprocess.run(["git", "-C", cwd] + args, capture_output=True, text=True, timeout=10).stdout.strip()
    except (OSError, subprocess.SubprocessError):
        return ""


def engine_record(*, engine, label, chip, prompt_name, prompt_tokens, load_ms, step_ms, tokens,
                  weight_bytes_per_token, total_bytes, peak_bw_gbs, ref_tokens, repo_dir):
    """The JSON object of bench.rs:198-219 for one run.

    step_ms: the gap before each decode step's token (bench.rs:180-184); tokens: the first token
    then one per step, truncated to the step count (bench.rs:185); total_bytes: weight bytes plus
    the KV bytes at every decoded position (bench.rs:186-188)."""
    steps = len(step_ms)
    tokens = list(tokens)[:steps]
    decode_s = sum(step_ms) / 1e3
    achieved = total_bytes / decode_s
    peak = peak_bw_gbs * 1e9
    compared = min(len(tokens), len(ref_tokens))
    diverge = next((i for i in range(compared) if tokens[i] != ref_tokens[i]), None)
    status = _git(["status", "--porcelain"], repo_dir)
    return {
        "engine": engine,
        "label": label,
        "timestamp": int(time.time()),
        "commit": _git(["rev-parse", "--short", "HEAD"], repo_dir),
        "dirty": bool(status),
        "chip": chip,
        "prompt_name": prompt_name,
        "prompt_tokens": prompt_tokens,
        "load_ms": load_ms,
        "decode": {
            "steps": steps,
            "median_ms": median(step_ms),
            "tps": steps / decode_s,
            "achieved_bw_gbs": achieved / 1e9,
            "mbu": achieved / peak,
            "weight_bytes_per_token": weight_bytes_per_token,
            "samples_ms": list(step_ms),
        },
        "parity_vs_mlx": {"compared": compared, "first_divergence": diverge},
        "tokens": tokens,
    }


def write_records(results_dir: str, record: dict) -> str:
    """bench.rs:221-226: the latest run (pretty JSON) and one history line; returns the latest path."""
    os.makedirs(results_dir, exist_ok=True)
    slug = chip_slug(record["chip"])
    latest = os.path.join(results_dir, f"engine_{record['engine']}_{slug}_{record['prompt_name']}.json")
    with open(latest, "w") as f:
        json.dump(record, f, indent=2)
    with open(os.path.join(results_dir, f"history_{slug}_{record['prompt_name']}.jsonl"), "a") as f:
        f.write(json.dumps(record) + "\n")
    return latest
