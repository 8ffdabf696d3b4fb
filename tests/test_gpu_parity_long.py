"""Full-size parity at the long-context and multi-token workloads, against committed oracle runs.

Long decode (tests/golden/qwen3_0_6b_long_{f32,bf16}.npz): the 130-token random prompt, then
4096 greedy decode steps (positions 130..4225). With an f32 KV cache the bar is the reference's
(tests/metal_parity.rs:14, :35-36): the oracle's greedy tokens and logits within max-abs 1e-2 at
all 4097 steps. The bf16 cache is held to the same bar against the oracle's bf16 mode, which rounds
every appended K/V element to bf16 (nearest, ties to even) and attends with the rounded values;
its drift from the f32 run is printed, as the reference reports its own (README.md:23,90).

With the f32 cache every one of the 4096 steps must pick the oracle's token, both teacher-forced
(segments of 8 pipelined steps from the oracle's token) and in one free-running pipelined decode
from a fresh cache: the engine's logits stay within ~1e-5 of the oracle's, well under the
smallest oracle top-2 gap of the run (1.4e-4).

The bf16 cache rounds K/V in a different order from the oracle's bf16 mode's accumulation, so its
logits move by up to ~1e-3, and random-init weights give a few steps whose oracle top-2 gap is
below that (the reference's real checkpoint does not). Within the logit bar either token of such
a pair is a correct greedy pick: the teacher-forced decode accepts another token only where the
oracle's top-2 gap is below twice the bar and the engine's own logit for the oracle's token is
within that gap of its maximum, and restarts from the oracle's token, so the cache keeps the
oracle's sequence; the free-running decode may leave the oracle only at such a step.

Multi-token forward (tests/golden/qwen3_0_6b_prefill2048.npz): a 2048-token random prompt
prefilled in chunks of 512, a k = 4 verify at position 2048 over the greedy continuation, then
20 decode steps, each against the oracle's sequential forward.

Stored per step: token, top-2 gap, max, L2 norm; every 8th long step (every step of the
prefill run) also the top-16 logits and a fixed sample of logit indices.
"""
import os
import time

import numpy as np
import pytest

import oracle
import qe
from conftest import PROMPT_LEN, PROMPT_SEED, REAL_SEED

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

MAX_ABS_DIFF = 1e-2
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LONG_STEPS = 4096
SEGMENT = 8


def load(name):
    g = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    assert int(g["seed"]) == REAL_SEED
    return g


def check_row(g, j, lg, full_row=None, tol=MAX_ABS_DIFF):
    """logits of fixture step j; full_row: its index among the stored top-k / sampled rows"""
    assert np.all(np.isfinite(lg)), f"step {j}: non-finite logits"
    d = abs(float(lg.max()) - float(g["max"][j]))
    assert d < tol, f"step {j}: max differs by {d}"
    assert abs(np.linalg.norm(lg.astype(np.float64)) - g["l2"][j]) < tol * np.sqrt(lg.size), f"step {j}: L2"
    worst = d
    if full_row is not None:
        ds = float(np.max(np.abs(lg[g["sample_idx"]] - g["sample_val"][full_row])))
        dt = float(np.max(np.abs(lg[g["top_idx"][full_row]] - g["top_val"][full_row])))
        assert ds < tol and dt < tol, f"step {j}: sampled {ds}, top-16 {dt}"
        worst = max(worst, ds, dt)
    return worst


def near_tie(g, j, lg, tok):
    """the engine's pick `tok` at fixture step j differs from the oracle's: a correct pick within
    the logit bar only at an oracle near-tie, with the engine's logit of the oracle's token close
    to its own maximum"""
    gap = float(g["top2_gap"][j])
    ref = int(g["tokens"][j])
    return gap < 2 * MAX_ABS_DIFF and float(lg[tok]) - float(lg[ref]) <= gap + 2 * MAX_ABS_DIFF


@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_long_decode_matches_oracle(gpu, real_ckpt, kv):
    g = load(f"qwen3_0_6b_long_{kv}.npz")
    every = int(g["every"])
    assert every == SEGMENT and len(g["tokens"]) == LONG_STEPS + 1
    m = qe.Model.load_model(real_ckpt)
    V = m.config().vocab_size
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, V)
    np.testing.assert_array_equal(prompt, g["prompt"])
    dtype = qe.QE_KV_BF16 if kv == "bf16" else qe.QE_KV_F32
    cache = qe.KVCache(m, PROMPT_LEN + LONG_STEPS + 1, dtype)
    t0 = time.time()
    logits = m.prefill(prompt, 0, cache)
    ref = [int(t) for t in g["tokens"]]
    worst = check_row(g, 0, logits, 0)
    ties = []
    if oracle.argmax(logits) != ref[0]:
        assert near_tie(g, 0, logits, oracle.argmax(logits)), "step 0: engine and oracle pick different tokens"
        ties.append(0)
    strict = kv == "f32"
    # c steps are done; the next segment feeds the oracle's token ref[c] at position PROMPT_LEN + c
    c, segments = 0, 0
    while c < LONG_STEPS:
        n = min(SEGMENT, LONG_STEPS - c)
        toks, lg = m.decode(ref[c], PROMPT_LEN + c, n, cache, want_logits=True)
        done = n
        for i in range(n):
            j = c + i + 1
            worst = max(worst, check_row(g, j, lg[i], j // every if j % every == 0 else None))
            if toks[i] != ref[j]:
                assert not strict, f"step {j}: engine {toks[i]} oracle {ref[j]} with the f32 cache"
                assert near_tie(g, j, lg[i], toks[i]), (
                    f"step {j}: engine {toks[i]} oracle {ref[j]} (oracle top-2 gap {g['top2_gap'][j]:.2e})")
                ties.append(j)
                done = i + 1  # step j's logits are checked; restart from the oracle's token ref[j]
                break
        c += done
        segments += 1
        if segments % 64 == 0:
            print(f"{kv} cache: step {c}, worst max-abs {worst:.2e} ({time.time() - t0:.1f}s)", flush=True)
    print(f"{kv} cache: 4096 steps, worst max-abs {worst:.2e}, min oracle top-2 gap "
          f"{float(np.min(g['top2_gap'])):.2e}, near-tie steps where the engine picked the other token: {ties}")
    if strict:
        assert ties == [] and worst < 1e-3, f"f32 cache: near-tie flips {ties}, worst max-abs {worst:.2e}"
    # The plain pipelined decode of all 4096 steps from a fresh cache: with the f32 cache it equals
    # the oracle at every step; with the bf16 cache it follows the oracle up to its first near-tie
    # flip, if any (past it the two greedy sequences are different prompts).
    cache2 = qe.KVCache(m, PROMPT_LEN + LONG_STEPS + 1, dtype)
    m.prefill(prompt, 0, cache2, want_logits=False)
    toks, _ = m.decode(ref[0], PROMPT_LEN, LONG_STEPS, cache2)
    diff = [j for j in range(LONG_STEPS) if toks[j] != ref[j + 1]]
    assert not (strict and diff), f"f32 cache: free-running decode leaves the oracle at step {diff[:1]}"
    if diff:
        j = diff[0] + 1
        assert j in ties or float(g["top2_gap"][j]) < 2 * MAX_ABS_DIFF, (
            f"free-running decode leaves the oracle at step {j} (oracle top-2 gap {g['top2_gap'][j]:.2e})")
    print(f"{kv} cache: free-running 4096-step decode equals the oracle for {diff[0] if diff else LONG_STEPS} steps")


def test_bf16_cache_drift_from_f32_oracle(gpu, real_ckpt):
    """the engine's bf16-cache logits against the f32 oracle run, over the steps before the f32 and
    bf16 oracle runs' greedy tokens first differ (the reference reports 0.074 max-abs,
    README.md:90); teacher-forced on the f32 oracle's tokens as in the long decode test"""
    g32, g16 = load("qwen3_0_6b_long_f32.npz"), load("qwen3_0_6b_long_bf16.npz")
    t32 = [int(t) for t in g32["tokens"]]
    diff = np.nonzero(g32["tokens"] != g16["tokens"])[0]
    same = int(diff[0]) if len(diff) else len(t32)
    steps = min(same - 1, 512)
    m = qe.Model.load_model(real_ckpt)
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, m.config().vocab_size)
    cache = qe.KVCache(m, PROMPT_LEN + steps + 1, qe.QE_KV_BF16)
    every = int(g32["every"])

    def drift_of(j, row):
        d = abs(float(row.max()) - float(g32["max"][j]))
        if j % every == 0:
            d = max(d, float(np.max(np.abs(row[g32["sample_idx"]] - g32["sample_val"][j // every]))),
                    float(np.max(np.abs(row[g32["top_idx"][j // every]] - g32["top_val"][j // every]))))
        return d

    drift = drift_of(0, m.prefill(prompt, 0, cache))
    c, flips = 0, []
    while c < steps:
        n = min(SEGMENT, steps - c)
        toks, lg = m.decode(t32[c], PROMPT_LEN + c, n, cache, want_logits=True)
        done = n
        for i in range(n):
            j = c + i + 1
            drift = max(drift, drift_of(j, lg[i]))
            if toks[i] != t32[j]:
                flips.append(j)
                done = i + 1
                break
        c += done
    print(f"bf16 cache vs f32 oracle over {steps} steps (the oracle runs agree for {same} steps): "
          f"max-abs drift {drift:.3e}; steps where the engine picked another token: {flips}")
    assert drift < 0.5
    # a different pick is only possible where the f32 oracle's top-2 gap is within the drift
    assert all(float(g32["top2_gap"][j]) < 2 * drift for j in flips)


def test_prefill_2048_in_chunks_of_512_then_verify_and_decode(gpu, real_ckpt):
    g = load("qwen3_0_6b_prefill2048.npz")
    n = len(g["prompt"])
    assert n == 2048
    m = qe.Model.load_model(real_ckpt)
    prompt = qe.random_prompt(int(g["prompt_seed"]), n, m.config().vocab_size)
    np.testing.assert_array_equal(prompt, g["prompt"])
    ref = [int(t) for t in g["tokens"]]
    steps = len(ref) - 1
    cache = qe.KVCache(m, n + steps + 1)
    logits = m.prefill_batch(prompt, 0, cache, chunk=512)
    assert oracle.argmax(logits) == ref[0]
    worst = check_row(g, 0, logits, 0)
    # k = 4 verify at position 2048 over the greedy continuation: row i is step i + 1
    k = 4
    rows = m.verify(np.array(ref[:k], dtype=np.uint32), n, cache)
    for i in range(k):
        assert oracle.argmax(rows[i]) == ref[i + 1], f"verify row {i}"
        worst = max(worst, check_row(g, i + 1, rows[i], i + 1))
    assert m.verify_greedy(np.array(ref[:k], dtype=np.uint32), n, cache).tolist() == ref[1:k + 1]
    # decode from the chunk-prefilled cache (it rewrites the verified positions)
    toks, lg = m.decode(ref[0], n, steps, cache, want_logits=True)
    assert toks == ref[1:]
    for i in range(steps):
        worst = max(worst, check_row(g, i + 1, lg[i], i + 1))
    print(f"2048-token prefill (chunks of 512), k=4 verify, {steps} decode steps: worst max-abs {worst:.2e}")


def test_prefill_2048_token_by_token_matches_chunked(gpu, real_ckpt):
    """the reference's prompt loop (one forward per token, bench.rs:174-176) on the same prompt"""
    g = load("qwen3_0_6b_prefill2048.npz")
    m = qe.Model.load_model(real_ckpt)
    prompt = g["prompt"].astype(np.uint32)
    cache = qe.KVCache(m, len(prompt) + 1)
    logits = m.prefill(prompt, 0, cache)
    assert oracle.argmax(logits) == int(g["tokens"][0])
    check_row(g, 0, logits, 0)


def test_prefill_prefetch_changes_no_result(gpu, real_ckpt, monkeypatch):
    """the causal attention launch's L2 prefetch of o_proj's weights (chunks of 65..1024 tokens)
    only loads: bit-identical last-token logits with QE_PREFILL_PREFETCH=0"""
    g = load("qwen3_0_6b_prefill2048.npz")
    prompt = g["prompt"].astype(np.uint32)

    def run():
        m = qe.Model.load_model(real_ckpt)  # QE_PREFILL_PREFETCH is read here
        return m.prefill_batch(prompt, 0, qe.KVCache(m, len(prompt) + 1), chunk=512)

    on = run()
    monkeypatch.setenv("QE_PREFILL_PREFETCH", "0")
    off = run()
    np.testing.assert_array_equal(on, off)


@pytest.mark.parametrize("streams", ["2", "3"])
def test_prefill_two_streams_change_no_result(gpu, real_ckpt, monkeypatch, streams):
    """consecutive chunks go round-robin over 2 (the default) or 3 streams, each chunk's attention
    ordered after the earlier chunks' K/V rows of the same layer: bit-identical logits and cache to
    one stream (QE_PREFILL_STREAMS=1), here for a prompt that ends in a short chunk"""
    g = load("qwen3_0_6b_prefill2048.npz")
    prompt = g["prompt"].astype(np.uint32)[:1800]

    def run():
        m = qe.Model.load_model(real_ckpt)  # QE_PREFILL_STREAMS is read here
        c = qe.KVCache(m, len(prompt) + 4)
        lg = m.prefill_batch(prompt, 0, c, chunk=256)
        toks, _ = m.decode(oracle.argmax(lg), len(prompt), 4, c)
        return lg, toks

    monkeypatch.setenv("QE_PREFILL_STREAMS", streams)
    lgn, tn = run()
    monkeypatch.setenv("QE_PREFILL_STREAMS", "1")
    lg1, t1 = run()
    np.testing.assert_array_equal(lgn, lg1)
    assert tn == t1
