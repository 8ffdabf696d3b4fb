"""Writes the oracle's golden runs on the seeded random-init Qwen3-0.6B-architecture checkpoint.

Every workload uses the checkpoint of seed 20260101 and runs the CPU oracle (the C restatement of
cpu_inference.rs) token by token, as the reference's bench does (bench.rs:172-191):

  decode   tests/golden/qwen3_0_6b_decode.npz: a 130-token prompt of uniform-random ids (seed 7),
           then 128 greedy decode steps at positions 130..257 with an f32 KV cache. Stored per
           step (the prompt's last position, then each decode step): the greedy token, the top-2
           gap, the logits' max / L2 norm, the top-16 (index, value) pairs and 512 logits at
           fixed sampled indices.
  long     tests/golden/qwen3_0_6b_long_<kv>.npz (kv = f32 or bf16): the same prompt, then 4096
           greedy steps (positions 130..4225). With --kv bf16 the oracle's cache rounds every
           appended K/V element to bf16 (nearest, ties to even) and attends with the rounded
           values. Stored per step: token, top-2 gap, max, L2; every 8th step also the top-16
           pairs and 256 sampled logits.
  prefill  tests/golden/qwen3_0_6b_prefill2048.npz: a 2048-token prompt (seed 11), then 20 greedy
           steps. Stored for the prompt's last position and each greedy step: token, top-2 gap,
           max, L2, top-16 pairs and 512 sampled logits. The logits of a k-token verify pass at
           position 2048 over the greedy continuation are rows 1..k of these.

Run from the repo root: python tests/golden/make_real_fixture.py [decode|long|prefill] [--kv f32|bf16]
[--workdir DIR]
"""
import argparse
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mac-gpu-compiler_amd")]

import oracle  # noqa: E402
import qe  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
SEED = 20260101
PROMPT_SEED = 7
PROMPT_LEN = 130
STEPS = 128
LONG_STEPS = 4096
LONG_EVERY = 8          # long runs: top-k and sampled logits every LONG_EVERY-th step
LONG_SAMPLES = 256
PREFILL_SEED = 11
PREFILL_LEN = 2048
PREFILL_STEPS = 20
N_SAMPLE = 512
TOPK = 16


def sample_indices(vocab: int, n: int = N_SAMPLE) -> np.ndarray:
    return np.sort(np.random.default_rng(99).choice(vocab, size=n, replace=False)).astype(np.int64)


def digest(logits: np.ndarray, idx: np.ndarray):
    order = np.argsort(-logits, kind="stable")[:TOPK]
    return order.astype(np.int64), logits[order].astype(np.float32), logits[idx].astype(np.float32)


class Recorder:
    """Per-step token / top-2 gap / max / L2, and the top-k and sampled logits of chosen steps."""

    def __init__(self, idx):
        self.idx = idx
        self.tokens, self.gaps, self.maxes, self.norms = [], [], [], []
        self.top_i, self.top_v, self.samples = [], [], []

    def __call__(self, lg, full=True):
        t = oracle.argmax(lg)
        ti, tv, s = digest(lg, self.idx)
        self.tokens.append(t)
        self.gaps.append(float(tv[0] - tv[1]))
        self.maxes.append(float(lg.max()))
        self.norms.append(float(np.linalg.norm(lg.astype(np.float64))))
        if full:
            self.top_i.append(ti)
            self.top_v.append(tv)
            self.samples.append(s)
        return t

    def arrays(self):
        return dict(tokens=np.array(self.tokens, np.int64), top2_gap=np.array(self.gaps, np.float32),
                    max=np.array(self.maxes, np.float32), l2=np.array(self.norms, np.float64),
                    top_idx=np.stack(self.top_i), top_val=np.stack(self.top_v), sample_idx=self.idx,
                    sample_val=np.stack(self.samples))


def checkpoint(work):
    d = os.path.join(work, "qwen3_0_6b")
    path = os.path.join(d, "model.safetensors")
    if not os.path.exists(path):
        qe.write_random_checkpoint(d, SEED, qe.QWEN3_0_6B)
    return path


def prefill(m, cache, prompt, t0):
    for pos, tok in enumerate(prompt):
        logits = m.forward(int(tok), pos, cache)
        if pos % 256 == 255:
            print(f"prompt position {pos} ({time.time() - t0:.1f}s)", flush=True)
    print(f"prefill of {len(prompt)} tokens {time.time() - t0:.1f}s", flush=True)
    return logits


def run_decode(m, work):
    V = m.config["vocab_size"]
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, V)
    rec = Recorder(sample_indices(V))
    cache = m.new_cache()
    t0 = time.time()
    tok = rec(prefill(m, cache, prompt, t0))
    for i in range(STEPS):
        tok = rec(m.forward(tok, PROMPT_LEN + i, cache))
        if i % 16 == 0:
            print(f"step {i} token {tok} gap {rec.gaps[-1]:.4f} ({time.time() - t0:.1f}s)", flush=True)
    out = os.path.join(HERE, "qwen3_0_6b_decode.npz")
    np.savez_compressed(out, seed=SEED, prompt_seed=PROMPT_SEED, prompt=prompt.astype(np.int64),
                        weight_bytes_per_token=np.int64(m.weight_bytes_per_token()), **rec.arrays())
    return out, rec


def run_long(m, work, kv):
    V = m.config["vocab_size"]
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, V)
    rec = Recorder(sample_indices(V, LONG_SAMPLES))
    cache = m.new_cache(bf16=kv == "bf16")
    t0 = time.time()
    tok = rec(prefill(m, cache, prompt, t0))
    for i in range(LONG_STEPS):
        tok = rec(m.forward(tok, PROMPT_LEN + i, cache), full=(i + 1) % LONG_EVERY == 0)
        if i % 128 == 0:
            print(f"step {i} token {tok} gap {rec.gaps[-1]:.4f} ({time.time() - t0:.1f}s)", flush=True)
    out = os.path.join(HERE, f"qwen3_0_6b_long_{kv}.npz")
    np.savez_compressed(out, seed=SEED, prompt_seed=PROMPT_SEED, prompt=prompt.astype(np.int64), kv=kv,
                        every=np.int64(LONG_EVERY), **rec.arrays())
    return out, rec


def run_prefill(m, work):
    V = m.config["vocab_size"]
    prompt = qe.random_prompt(PREFILL_SEED, PREFILL_LEN, V)
    rec = Recorder(sample_indices(V))
    cache = m.new_cache()
    t0 = time.time()
    tok = rec(prefill(m, cache, prompt, t0))
    for i in range(PREFILL_STEPS):
        tok = rec(m.forward(tok, PREFILL_LEN + i, cache))
    out = os.path.join(HERE, "qwen3_0_6b_prefill2048.npz")
    np.savez_compressed(out, seed=SEED, prompt_seed=PREFILL_SEED, prompt=prompt.astype(np.int64), **rec.arrays())
    return out, rec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("workload", nargs="?", default="decode", choices=["decode", "long", "prefill"])
    ap.add_argument("--kv", choices=["f32", "bf16"], default="f32")
    ap.add_argument("--workdir", default="/tmp/qe_fixture")
    args = ap.parse_args()
    m = oracle.Model(checkpoint(args.workdir))
    if args.workload == "decode":
        out, rec = run_decode(m, args.workdir)
    elif args.workload == "long":
        out, rec = run_long(m, args.workdir, args.kv)
    else:
        out, rec = run_prefill(m, args.workdir)
    print(f"wrote {out}: tokens {rec.tokens[:8]}..., {len(set(rec.tokens))} distinct, "
          f"min top-2 gap {min(rec.gaps):.3e}")


if __name__ == "__main__":
    main()
