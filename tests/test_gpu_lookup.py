"""Speculative greedy decode by prompt lookup (qe_decode_lookup) through the C ABI: it must emit
exactly the greedy tokens of token-by-token decoding (the oracle's on the tiny model, the
committed decode fixture on the real one) and leave the cache as qe_decode would."""
import os

import numpy as np
import pytest

import oracle
import qe
from conftest import DECODE_STEPS, PROMPT_LEN, PROMPT_SEED, TINY

pytestmark = pytest.mark.gpu


def test_verify_greedy_is_the_argmax_of_verify(gpu, tiny_ckpt):
    m = qe.Model.load_model(tiny_ckpt)
    prefix = qe.random_prompt(51, 30, TINY.vocab_size)
    draft = qe.random_prompt(53, 9, TINY.vocab_size)
    c = qe.KVCache(m, 48)
    m.prefill(prefix, 0, c, want_logits=False)
    rows = m.verify(draft, 30, c)
    toks = m.verify_greedy(draft, 30, c)
    assert [int(t) for t in toks] == [oracle.argmax(r) for r in rows]


@pytest.mark.parametrize("k_max,ngram", [(1, 1), (4, 3), (8, 2)])
def test_tiny_lookup_decode_matches_oracle(gpu, tiny_ckpt, k_max, ngram):
    m = qe.Model.load_model(tiny_ckpt)
    om = oracle.Model(tiny_ckpt)
    # a prompt that repeats, so drafts exist and some are rejected
    base = [int(t) for t in qe.random_prompt(57, 12, TINY.vocab_size)]
    prompt = np.array(base * 3 + base[:5], dtype=np.uint32)
    P, steps = len(prompt), 40
    c = qe.KVCache(m, P + steps + 8)
    logits = m.prefill(prompt, 0, c)
    oc = om.new_cache()
    for pos, tok in enumerate(prompt):
        ref = om.forward(int(tok), pos, oc)
    first = oracle.argmax(ref)
    assert oracle.argmax(logits) == first
    got, st = m.decode_lookup(first, P, steps, c, context=prompt, k_max=k_max, ngram=ngram)
    want, tok = [], first
    for i in range(steps):
        tok = oracle.argmax(om.forward(tok, P + i, oc))
        want.append(tok)
    assert got == want
    assert st["accepted"] <= st["drafted"] and st["passes"] + st["single_steps"] >= 1
    assert st["passes"] + st["single_steps"] + st["accepted"] + st["plain_steps"] == steps
    assert len(c) == P + steps
    # the cache continues like the oracle's after the rejected drafts
    more, _ = m.decode(got[-1], P + steps, 5, c)
    for i in range(5):
        tok = oracle.argmax(om.forward(tok, P + steps + i, oc))
        assert more[i] == tok


@pytest.mark.parametrize("adaptive", [True, False])
@pytest.mark.parametrize("quality", ["right", "wrong", "every_third"])
def test_tiny_drafted_decode_matches_plain(gpu, tiny_ckpt, adaptive, quality):
    """qe_decode_drafted with a caller's draft source: the tokens of plain decode whatever the
    drafts; with drafts that never pay (always wrong) the adaptive rule decodes plain blocks"""
    m = qe.Model.load_model(tiny_ckpt)
    prompt = qe.random_prompt(61, 20, TINY.vocab_size)
    P, steps, k_max = len(prompt), 80, 3
    c = qe.KVCache(m, P + steps + 8)
    first = oracle.argmax(m.prefill(prompt, 0, c))
    want, _ = m.decode(first, P, steps, c)
    seq = [first] + want
    calls = [0]

    def draft(hist, k):
        i = len(hist) - P - 1  # seq index of the last token
        assert list(hist[P:]) == seq[:i + 1]
        calls[0] += 1
        good = quality == "right" or (quality == "every_third" and calls[0] % 3 == 0)
        return [seq[i + 1 + j] if good else (seq[i + 1 + j] + 1) % TINY.vocab_size for j in range(k)]

    got, st = m.decode_drafted(first, P, steps, c, draft, context=prompt, k_max=k_max, adaptive=adaptive)
    assert got == want
    assert st["passes"] + st["single_steps"] + st["accepted"] + st["plain_steps"] == steps
    assert len(c) == P + steps
    if quality == "right":
        assert st["accepted"] == st["drafted"] > 0
    if quality == "wrong":
        assert st["accepted"] == 0
        assert (st["plain_steps"] > 0) == adaptive
    if not adaptive:
        assert st["plain_steps"] == 0
    more, _ = m.decode(got[-1], P + steps, 3, c)  # the cache continues after rejected drafts
    c2 = qe.KVCache(m, P + steps + 8)
    m.prefill(prompt, 0, c2, want_logits=False)
    ref, _ = m.decode(first, P, steps + 3, c2)
    assert more == ref[steps:]


def test_drafted_decode_reports_a_draft_source_error(gpu, tiny_ckpt):
    m = qe.Model.load_model(tiny_ckpt)
    prompt = qe.random_prompt(63, 10, TINY.vocab_size)
    c = qe.KVCache(m, 40)
    first = oracle.argmax(m.prefill(prompt, 0, c))

    P = len(prompt)
    calls, emitted = [0], []

    def bad(hist, k):  # drafts nothing twice (two single steps), then fails
        calls[0] += 1
        if calls[0] == 3:
            raise ValueError("draft source failed")
        return []

    with pytest.raises(ValueError, match="draft source failed"):
        m.decode_drafted(first, P, 20, c, bad, context=prompt, k_max=2, adaptive=False, on_token=emitted.append)
    # the decode stopped at the failing call: two tokens out, the cache valid up to the next position
    assert calls[0] == 3 and len(emitted) == 2 and len(c) == P + 2
    want, _ = m.decode(first, P, 2, c)
    assert want == emitted
    with pytest.raises(qe.QeError):  # a draft token outside the vocabulary
        m.decode_drafted(first, len(prompt), 5, c, lambda h, k: [TINY.vocab_size] * k, context=prompt, k_max=2)


@pytest.mark.slow
def test_real_lookup_decode_matches_fixture(gpu, real_ckpt):
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qwen3_0_6b_decode.npz"),
                allow_pickle=False)
    m = qe.Model.load_model(real_ckpt)
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, m.config().vocab_size)
    c = qe.KVCache(m, PROMPT_LEN + DECODE_STEPS + 1)
    first = oracle.argmax(m.prefill(prompt, 0, c))
    toks, st = m.decode_lookup(first, PROMPT_LEN, DECODE_STEPS, c, context=prompt, k_max=4, ngram=3)
    ref = [int(t) for t in g["tokens"]]
    got = [first] + toks
    assert got == ref, f"diverges at {next(i for i in range(len(ref)) if got[i] != ref[i])}"
    print(f"lookup decode: {st}, {DECODE_STEPS / (st['passes'] + st['single_steps']):.2f} tokens per pass")


def test_lookup_argument_errors(gpu, tiny_ckpt):
    m = qe.Model.load_model(tiny_ckpt)
    c = qe.KVCache(m, 16)
    m.prefill(np.arange(4, dtype=np.uint32), 0, c, want_logits=False)
    for kw, code in (({"k_max": 0}, qe.QE_ERR_ARG), ({"k_max": 64}, qe.QE_ERR_ARG), ({"ngram": 0}, qe.QE_ERR_ARG)):
        with pytest.raises(qe.QeError) as e:
            m.decode_lookup(1, 4, 4, c, context=[0, 1, 2, 3], **kw)
        assert e.value.code == code
    with pytest.raises(qe.QeError) as e:
        m.decode_lookup(1, 5, 4, c)  # nothing cached at position 4
    assert e.value.code == qe.QE_ERR_POS
    with pytest.raises(qe.QeError) as e:
        m.decode_lookup(1, 4, 13, c)  # runs past max_seq
    assert e.value.code == qe.QE_ERR_POS
    with pytest.raises(qe.QeError) as e:
        m.decode_lookup(TINY.vocab_size, 4, 2, c)
    assert e.value.code == qe.QE_ERR_ARG
    with pytest.raises(qe.QeError) as e:
        m.verify_greedy(np.zeros(65, dtype=np.uint32), 0, qe.KVCache(m, 80))
    assert e.value.code == qe.QE_ERR_ARG
