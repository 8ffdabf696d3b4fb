"""Full-size parity: the decode workload on the Qwen3-0.6B-architecture random-init model.

130-token random prompt, then 128 greedy decode steps with an f32 KV cache. The bar is the
reference's (tests/metal_parity.rs:14, :35-36): at every step the logits are within max-abs 1e-2
of the CPU oracle and the greedy tokens are identical -- here for all 130 prompt positions and
all 128 decode steps, with the oracle run live in lockstep (teacher-forced on the GPU's tokens),
plus the committed oracle fixture tests/golden/qwen3_0_6b_decode.npz.
"""
import os
import time

import numpy as np
import pytest

import oracle
import qe
from conftest import DECODE_STEPS, PROMPT_LEN, PROMPT_SEED, REAL_SEED

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

MAX_ABS_DIFF = 1e-2
FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qwen3_0_6b_decode.npz")


@pytest.fixture(scope="module")
def golden():
    g = np.load(FIXTURE, allow_pickle=False)
    assert int(g["seed"]) == REAL_SEED and int(g["prompt_seed"]) == PROMPT_SEED
    return g


def test_weight_bytes_match_reference_formula(gpu, real_ckpt, golden):
    m = qe.Model.load_model(real_ckpt)
    # bench.rs:106-116 on this checkpoint; the reference records 1,192,101,888 for Qwen3-0.6B
    assert m.weight_bytes_per_token() == 1_192_101_888 == int(golden["weight_bytes_per_token"])


def test_decode_matches_oracle_fixture(gpu, real_ckpt, golden):
    m = qe.Model.load_model(real_ckpt)
    V = m.config().vocab_size
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, V)
    np.testing.assert_array_equal(prompt, golden["prompt"])
    cache = qe.KVCache(m, PROMPT_LEN + DECODE_STEPS + 1)
    logits = m.prefill(prompt, 0, cache)
    first = oracle.argmax(logits)
    toks, step_logits = m.decode(first, PROMPT_LEN, DECODE_STEPS, cache, want_logits=True)
    got = [first] + toks
    ref = [int(t) for t in golden["tokens"]]
    div = next((i for i in range(len(ref)) if got[i] != ref[i]), None)
    assert div is None, f"greedy tokens diverge at step {div}: gpu {got[div]} oracle {ref[div]}"
    all_logits = np.concatenate([logits[None], step_logits])
    idx = golden["sample_idx"]
    for i, lg in enumerate(all_logits):
        assert np.all(np.isfinite(lg))
        d_sample = np.max(np.abs(lg[idx] - golden["sample_val"][i]))
        d_top = np.max(np.abs(lg[golden["top_idx"][i]] - golden["top_val"][i]))
        assert d_sample < MAX_ABS_DIFF and d_top < MAX_ABS_DIFF, f"step {i}: {d_sample} {d_top}"
        assert abs(np.linalg.norm(lg.astype(np.float64)) - golden["l2"][i]) < 1e-2 * np.sqrt(V)


def test_lockstep_every_step_against_live_oracle(gpu, real_ckpt):
    m = qe.Model.load_model(real_ckpt)
    om = oracle.Model(real_ckpt)
    V = m.config().vocab_size
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, V)
    cache = qe.KVCache(m, PROMPT_LEN + DECODE_STEPS + 1)
    oc = om.new_cache()
    t0 = time.time()
    worst = 0.0
    for pos, tok in enumerate(prompt):
        a = om.forward(int(tok), pos, oc)
        b = m.forward(int(tok), pos, cache)
        d = float(np.max(np.abs(a - b)))
        worst = max(worst, d)
        assert np.all(np.isfinite(b)) and d < MAX_ABS_DIFF, f"prefill pos {pos}: {d}"
        assert oracle.argmax(a) == oracle.argmax(b), f"prefill pos {pos}: different greedy token"
    print(f"prefill lockstep done in {time.time() - t0:.1f}s, worst max-abs {worst:.2e}", flush=True)
    first = oracle.argmax(a)
    toks, step_logits = m.decode(first, PROMPT_LEN, DECODE_STEPS, cache, want_logits=True)
    tok = first
    gaps = []
    for i in range(DECODE_STEPS):
        a = om.forward(tok, PROMPT_LEN + i, oc)  # teacher-forced on the GPU's previous token
        d = float(np.max(np.abs(a - step_logits[i])))
        worst = max(worst, d)
        assert d < MAX_ABS_DIFF, f"decode step {i}: logits diverge by {d}"
        srt = np.sort(a)
        gaps.append(float(srt[-1] - srt[-2]))
        assert toks[i] == oracle.argmax(a), f"decode step {i}: gpu {toks[i]} oracle {oracle.argmax(a)} (top-2 gap {gaps[-1]:.2e})"
        tok = toks[i]
        if i % 32 == 0:
            print(f"decode step {i}: max-abs {d:.2e} ({time.time() - t0:.1f}s)", flush=True)
    print(f"lockstep: 130 prompt + 128 decode steps, worst max-abs {worst:.2e}, min top-2 gap {min(gaps):.2e}")
