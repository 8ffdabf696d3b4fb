"""Two-row verify passes through the decode step's two launches per layer (qe_verify /
qe_verify_greedy with k = 2 on the Qwen3-0.6B shape): each row must give the greedy token and the
logits of token-by-token decoding -- the committed oracle fixture at positions 130..257, and the
batch path (QE_VERIFY_FUSED=0, itself checked against the oracle in test_gpu_batch.py) at every
attention shape the fused pass takes (4, 8 and 16 runs of 32 or 64 positions, f32 and bf16
caches, the pass's second row in the next run)."""
import os

import numpy as np
import pytest

import oracle
import qe
from conftest import DECODE_STEPS, PROMPT_LEN, PROMPT_SEED

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qwen3_0_6b_decode.npz")


def test_two_row_passes_follow_the_fixture(gpu, real_ckpt):
    g = np.load(FIXTURE, allow_pickle=False)
    m = qe.Model.load_model(real_ckpt)
    assert m.fused_layers() == 1
    V = m.config().vocab_size
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, V)
    c = qe.KVCache(m, PROMPT_LEN + DECODE_STEPS + 2)
    first = oracle.argmax(m.prefill(prompt, 0, c))
    ref = [int(t) for t in g["tokens"]]  # ref[0] = first
    assert first == ref[0]
    idx = g["sample_idx"]
    worst = 0.0
    # passes [ref[i], ref[i + 1]] at positions P + i, P + i + 1: both drafts right, so the rows'
    # greedy tokens are ref[i + 1], ref[i + 2]; logits on the fixture's sample within 1e-2
    for i in range(0, DECODE_STEPS - 1, 2):
        ids = [ref[i], ref[i + 1]]
        if i % 8 == 0:
            rows = m.verify(ids, PROMPT_LEN + i, c)
            for r in range(2):
                # sample_val[j]: the logits that gave ref[j]
                worst = max(worst, float(np.abs(rows[r][idx] - g["sample_val"][i + 1 + r]).max()))
                assert oracle.argmax(rows[r]) == ref[i + 1 + r]
        else:
            toks = m.verify_greedy(ids, PROMPT_LEN + i, c)
            assert [int(t) for t in toks] == [ref[i + 1], ref[i + 2]], f"pass at {PROMPT_LEN + i}"
    assert worst < 1e-2, worst
    print(f"two-row fused verify: worst sampled logit difference {worst:.3g}")
    # a rejected draft: row 0 still gives the greedy token, row 1 that of the wrong draft
    wrong = (ref[2] + 1) % V
    toks = m.verify_greedy([ref[1], wrong], PROMPT_LEN + 1, c)
    assert int(toks[0]) == ref[2]


@pytest.mark.parametrize("kv", [qe.QE_KV_F32, qe.QE_KV_BF16])
def test_two_row_passes_match_the_batch_path(gpu, real_ckpt, monkeypatch, kv):
    m = qe.Model.load_model(real_ckpt)
    monkeypatch.setenv("QE_VERIFY_FUSED", "0")
    b = qe.Model.load_model(real_ckpt)  # QE_VERIFY_FUSED is read here
    monkeypatch.delenv("QE_VERIFY_FUSED")
    V = m.config().vocab_size
    n = 1030
    prompt = qe.random_prompt(11, n, V)
    # pass positions: 4, 8 and 16 runs of 32 (up to 256 positions) and of 64 (up to 1024), the
    # second row opening a new run (pos + 1 a multiple of the run), and the last position a pass
    # takes on this path (its rows end at position 1023)
    positions = [3, 31, 63, 100, 127, 200, 255, 256, 300, 511, 700, 1022]
    cm, cb = qe.KVCache(m, n + 2, kv), qe.KVCache(b, n + 2, kv)
    # the two paths sum in different orders (f32 FMA here, split-bf16 matrix cores there); with a
    # bf16 cache such differences can round a K/V element the other way (2^-9 relative), so that
    # cache is held to the reference's own bar
    tol = 1e-3 if kv == qe.QE_KV_F32 else 1e-2
    m.prefill_batch(prompt[:3], 0, cm, want_logits=False)
    b.prefill_batch(prompt[:3], 0, cb, want_logits=False)
    done = 3
    for pos in positions:
        if pos > done:
            m.prefill_batch(prompt[done:pos], done, cm, want_logits=False)
            b.prefill_batch(prompt[done:pos], done, cb, want_logits=False)
            done = pos
        ids = prompt[pos:pos + 2]
        rm, rb = m.verify(ids, pos, cm), b.verify(ids, pos, cb)
        diff = float(np.abs(rm - rb).max())
        assert diff < tol, (pos, diff)
        assert [oracle.argmax(r) for r in rm] == [int(t) for t in m.verify_greedy(ids, pos, cm)]
        assert [oracle.argmax(r) for r in rm] == [oracle.argmax(r) for r in rb], pos
        # the K/V rows the pass wrote are those of the batch path: a decode step after it agrees
        nxt = int(prompt[pos + 2])
        lm, lb = m.forward(nxt, pos + 2, cm), b.forward(nxt, pos + 2, cb)
        assert float(np.abs(lm - lb).max()) < tol, pos
        done = pos + 3
