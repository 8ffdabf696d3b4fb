"""Writes tests/golden/qwen3_0_6b_decode.npz: the oracle's greedy run of the decode workload.

Workload: the seeded random-init Qwen3-0.6B-architecture checkpoint (seed 20260101), a 130-token
prompt of uniform-random ids (seed 7), then 128 greedy decode steps at positions 130..257 with an
f32 KV cache -- the reference's bench protocol (bench.rs:172-191) on synthetic weights.

Stored per step (the prompt's last position, then each decode step): the greedy token, the top-2
gap, the logits' max / L2 norm, the top-16 (index, value) pairs and 512 logits at fixed sampled
indices. Run from the repo root: python tests/golden/make_real_fixture.py [workdir]
"""
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mac-gpu-compiler_amd")]

import oracle  # noqa: E402
import qe  # noqa: E402

SEED = 20260101
PROMPT_SEED = 7
PROMPT_LEN = 130
STEPS = 128
N_SAMPLE = 512
TOPK = 16


def sample_indices(vocab: int) -> np.ndarray:
    return np.sort(np.random.default_rng(99).choice(vocab, size=N_SAMPLE, replace=False)).astype(np.int64)


def digest(logits: np.ndarray, idx: np.ndarray):
    order = np.argsort(-logits, kind="stable")[:TOPK]
    return order.astype(np.int64), logits[order].astype(np.float32), logits[idx].astype(np.float32)


def main():
    work = sys.argv[1] if len(sys.argv) > 1 else "/tmp/qe_fixture"
    d = os.path.join(work, "qwen3_0_6b")
    path = os.path.join(d, "model.safetensors")
    if not os.path.exists(path):
        qe.write_random_checkpoint(d, SEED, qe.QWEN3_0_6B)
    m = oracle.Model(path)
    V = m.config["vocab_size"]
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, V)
    idx = sample_indices(V)
    cache = m.new_cache()
    t0 = time.time()
    for pos, tok in enumerate(prompt):
        logits = m.forward(int(tok), pos, cache)
    print(f"prefill {time.time() - t0:.1f}s", flush=True)
    tokens, gaps, maxes, norms, top_i, top_v, samples = [], [], [], [], [], [], []

    def record(lg):
        t = oracle.argmax(lg)
        ti, tv, s = digest(lg, idx)
        tokens.append(t)
        gaps.append(float(tv[0] - tv[1]))
        maxes.append(float(lg.max()))
        norms.append(float(np.linalg.norm(lg.astype(np.float64))))
        top_i.append(ti)
        top_v.append(tv)
        samples.append(s)
        return t

    tok = record(logits)
    for i in range(STEPS):
        logits = m.forward(tok, PROMPT_LEN + i, cache)
        tok = record(logits)
        if i % 16 == 0:
            print(f"step {i} token {tok} gap {gaps[-1]:.4f} ({time.time() - t0:.1f}s)", flush=True)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "qwen3_0_6b_decode.npz")
    np.savez_compressed(
        out, seed=SEED, prompt_seed=PROMPT_SEED, prompt=prompt.astype(np.int64), tokens=np.array(tokens, np.int64),
        top2_gap=np.array(gaps, np.float32), max=np.array(maxes, np.float32), l2=np.array(norms, np.float64),
        top_idx=np.stack(top_i), top_val=np.stack(top_v), sample_idx=idx, sample_val=np.stack(samples),
        weight_bytes_per_token=np.int64(m.weight_bytes_per_token()))
    print(f"wrote {out}: tokens {tokens[:8]}..., min top-2 gap {min(gaps):.5f}")


if __name__ == "__main__":
    main()
