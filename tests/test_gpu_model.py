"""Whole-model parity on the GPU against the CPU oracle (the reference's own bar:
tests/metal_parity.rs -- logits max-abs < 1e-2 and equal greedy tokens at every step)."""
import numpy as np
import pytest

import oracle
import qe
from conftest import TINY

pytestmark = pytest.mark.gpu

MAX_ABS_DIFF = 1e-2  # tests/metal_parity.rs:14


def test_tiny_forward_matches_oracle(gpu, tiny_ckpt):
    m = qe.Model.load_model(tiny_ckpt)
    om = oracle.Model(tiny_ckpt)
    cache = qe.KVCache(m, 64)
    oc = om.new_cache()
    prompt = qe.random_prompt(3, 40, TINY.vocab_size)
    worst = 0.0
    for pos, tok in enumerate(prompt):
        a = om.forward(int(tok), pos, oc)
        b = m.forward(int(tok), pos, cache)
        assert np.all(np.isfinite(b)), f"non-finite logits at pos {pos}"
        d = float(np.max(np.abs(a - b)))
        worst = max(worst, d)
        assert d < 1e-4, f"pos {pos}: logits diverge by {d}"
        assert oracle.argmax(a) == oracle.argmax(b), f"pos {pos}: different greedy token"
    assert len(cache) == len(prompt)
    print(f"tiny forward: worst max-abs {worst:.2e}")


def test_tiny_decode_matches_forward(gpu, tiny_ckpt):
    # tests/metal_parity.rs:42-71: pipelined decode with the GPU argmax == forward + CPU argmax
    m = qe.Model.load_model(tiny_ckpt)
    steps = 48
    prompt = qe.random_prompt(11, 5, TINY.vocab_size)
    max_seq = len(prompt) + steps + 1
    cache = qe.KVCache(m, max_seq)
    for pos, tok in enumerate(prompt):
        logits = m.forward(int(tok), pos, cache)
    first = oracle.argmax(logits)
    expected = []
    tok = first
    for i in range(steps):
        tok = oracle.argmax(m.forward(tok, len(prompt) + i, cache))
        expected.append(tok)
    cache2 = qe.KVCache(m, max_seq)
    m.prefill(prompt, 0, cache2, want_logits=False)
    got = []
    toks, _ = m.decode(first, len(prompt), steps, cache2, on_token=got.append)
    assert got == expected
    assert toks == expected


def test_tiny_decode_matches_oracle(gpu, tiny_ckpt):
    m = qe.Model.load_model(tiny_ckpt)
    om = oracle.Model(tiny_ckpt)
    steps = 60
    prompt = qe.random_prompt(13, 9, TINY.vocab_size)
    cache = qe.KVCache(m, len(prompt) + steps)
    oc = om.new_cache()
    for pos, tok in enumerate(prompt):
        ol = om.forward(int(tok), pos, oc)
    gl = m.prefill(prompt, 0, cache)
    assert np.max(np.abs(gl - ol)) < 1e-4
    first = oracle.argmax(ol)
    toks, logits = m.decode(first, len(prompt), steps, cache, want_logits=True)
    tok = first
    for i in range(steps):
        ol = om.forward(tok, len(prompt) + i, oc)
        assert np.max(np.abs(ol - logits[i])) < 1e-4, f"step {i}"
        tok = oracle.argmax(ol)
        assert toks[i] == tok, f"step {i}: gpu {toks[i]} oracle {tok}"


@pytest.mark.parametrize("max_seq,n_pos,kv", [(300, 290, "f32"), (2100, 2050, "f32"), (2100, 2050, "bf16")])
def test_tiny_long_cache_matches_oracle(gpu, tiny_ckpt, max_seq, n_pos, kv):
    # Every position replays the step graph of its attention shape. A cache of 300 positions
    # allows 5 runs per KV head: steps use 4 or 5 runs of 64 positions. 2100 positions allow 16:
    # runs of 64 in groups of 4, 8 and 16, then runs of 128 and 192 positions (two and three
    # tiles, so the double-buffered tile loop runs), with o_proj merging 4, 8 and 16 partials.
    # The bf16 cache is compared with the oracle's bf16 mode (K/V rounded to bf16 on append).
    m = qe.Model.load_model(tiny_ckpt)
    om = oracle.Model(tiny_ckpt)
    cache = qe.KVCache(m, max_seq, qe.QE_KV_BF16 if kv == "bf16" else qe.QE_KV_F32)
    oc = om.new_cache(bf16=kv == "bf16")
    tol = 1e-3 if kv == "bf16" else 1e-4
    prompt = qe.random_prompt(23, n_pos, TINY.vocab_size)
    worst = 0.0
    for pos, tok in enumerate(prompt):
        a = om.forward(int(tok), pos, oc)
        b = m.forward(int(tok), pos, cache)
        d = float(np.max(np.abs(a - b)))
        worst = max(worst, d)
        assert d < tol, f"pos {pos}: logits diverge by {d}"
        assert oracle.argmax(a) == oracle.argmax(b), f"pos {pos}: different greedy token"
    print(f"tiny model, {kv} cache {max_seq}, {n_pos} positions: worst max-abs {worst:.2e}")


def test_prefill_equals_forward_loop(gpu, tiny_ckpt):
    m = qe.Model.load_model(tiny_ckpt)
    prompt = qe.random_prompt(17, 23, TINY.vocab_size)
    c1 = qe.KVCache(m, 32)
    for pos, tok in enumerate(prompt):
        a = m.forward(int(tok), pos, c1)
    c2 = qe.KVCache(m, 32)
    b = m.prefill(prompt, 0, c2)
    np.testing.assert_array_equal(a, b)


def test_profile_step_stages_and_next_step(gpu, tiny_ckpt):
    """qe_profile_step times every stage (and each layer's q|k|v + attention pair) and leaves a
    cache from which the next forward still matches the oracle"""
    m = qe.Model.load_model(tiny_ckpt)
    om = oracle.Model(tiny_ckpt)
    prompt = qe.random_prompt(19, 9, TINY.vocab_size)
    c = qe.KVCache(m, 16)
    m.prefill(prompt[:8], 0, c, want_logits=False)
    stages = {name: (us, n) for name, us, n in m.profile_step(int(prompt[8]), 8, c)}
    L = TINY.num_hidden_layers
    prefixes = ["qkv+attention+o_proj", "qkv+attention+o_proj+gate_up", "qkv+attention+o_proj+gate_up+down",
                "qkv+attention+o_proj+gate_up+down+lm_head"]
    assert set(stages) == {"qkv", "attention", "qkv+attention", "o_proj", "gate_up", "down", "lm_head", "argmax",
                           *prefixes}
    assert stages["qkv+attention"][1] == 2 * L and stages["attention"][1] == L
    assert [stages[p][1] for p in prefixes] == [3 * L, 4 * L, 5 * L, 5 * L + 1]
    assert all(us > 0 for us, _ in stages.values())
    oc = om.new_cache()
    for pos, tok in enumerate(prompt):
        om.forward(int(tok), pos, oc)
    ref = om.forward(3, 9, oc)
    got = m.forward(3, 9, c)
    assert float(np.max(np.abs(got - ref))) < MAX_ABS_DIFF


@pytest.mark.parametrize("env", [{"QE_L2_PREFETCH": "0"}, {"QE_LAUNCH": "eager"}])
def test_switches_change_no_result(gpu, tiny_ckpt, env, monkeypatch):
    """the L2 weight prefetch and graph replay change timing only: the same tokens and bit-identical
    logits as the default path"""
    prompt = qe.random_prompt(23, 12, TINY.vocab_size)

    def run():
        m = qe.Model.load_model(tiny_ckpt)  # QE_L2_PREFETCH is read here
        c = qe.KVCache(m, 48)               # QE_LAUNCH here
        first = oracle.argmax(m.prefill(prompt, 0, c))
        return m.decode(first, len(prompt), 30, c, want_logits=True)

    toks0, logits0 = run()
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    toks1, logits1 = run()
    assert list(toks1) == list(toks0)
    np.testing.assert_array_equal(logits1, logits0)


# Past 1024 positions a decode step splits each KV head's positions over up to 64 runs and
# merges them in a launch of its own; QE_WIDE_ATTN=0 keeps 16 longer runs merged in the o_proj
# prologue. Creating the cache enumerates every step shape up to max_seq (a loop that must end);
# the two paths agree to the rounding of their merge order.
@pytest.mark.parametrize("max_seq", [1100, 4227, 9000, 33000])
def test_wide_attention_matches_prologue_merge(gpu, tiny_ckpt, max_seq, monkeypatch):
    m = qe.Model.load_model(tiny_ckpt)
    prompt = qe.random_prompt(41, max_seq - 4, TINY.vocab_size)

    def run():
        c = qe.KVCache(m, max_seq)  # QE_WIDE_ATTN is read here
        first = oracle.argmax(m.prefill_batch(prompt, 0, c, chunk=2048))
        return m.decode(first, len(prompt), 3, c, want_logits=True)

    toks1, lg1 = run()
    monkeypatch.setenv("QE_WIDE_ATTN", "0")
    toks0, lg0 = run()
    d = float(np.max(np.abs(lg1 - lg0)))
    assert d < 1e-4, f"wide and prologue-merged attention differ by {d}"
    for i in range(3):
        top2 = np.sort(lg0[i])[-2:]
        if top2[1] - top2[0] > 1e-3:
            assert toks1[i] == toks0[i]
        else:
            break  # a near-tie: the two greedy continuations may part here


def test_empty_inputs_do_nothing(gpu, tiny_ckpt):
    """an empty prompt and a zero-step decode leave the cache as it was; a one-position cache
    holds exactly one forward"""
    m = qe.Model.load_model(tiny_ckpt)
    c = qe.KVCache(m, 8)
    assert m.prefill([], 0, c) is None and len(c) == 0
    assert m.prefill_batch(np.zeros(0, dtype=np.uint32), 0, c) is None and len(c) == 0
    toks, logits = m.decode(1, 0, 0, c, want_logits=True)
    assert list(toks) == [] and logits.shape == (0, TINY.vocab_size) and len(c) == 0
    one = qe.KVCache(m, 1)
    a = m.forward(5, 0, one)
    om = oracle.Model(tiny_ckpt)
    assert float(np.max(np.abs(a - om.forward(5, 0, om.new_cache())))) < MAX_ABS_DIFF
    with pytest.raises(qe.QeError) as e:
        m.decode(oracle.argmax(a), 1, 1, one)  # no room for a second position
    assert e.value.code == qe.QE_ERR_POS


def test_position_contract(gpu, tiny_ckpt):
    m = qe.Model.load_model(tiny_ckpt)
    cache = qe.KVCache(m, 4)
    with pytest.raises(qe.QeError) as e:
        m.forward(1, 1, cache)  # nothing cached yet
    assert e.value.code == qe.QE_ERR_POS
    for pos in range(4):
        m.forward(pos, pos, cache)
    with pytest.raises(qe.QeError) as e:
        m.forward(1, 4, cache)  # pos >= max_seq (metal_inference.rs:321)
    assert e.value.code == qe.QE_ERR_POS
    with pytest.raises(qe.QeError) as e:
        m.forward(TINY.vocab_size, 0, cache)
    assert e.value.code == qe.QE_ERR_ARG
    with pytest.raises(qe.QeError) as e:
        m.decode(1, 2, 3, cache)  # runs past max_seq
    assert e.value.code == qe.QE_ERR_POS
    # rewriting an earlier position is allowed, as in the reference's Metal engine
    a = m.forward(7, 2, cache)
    assert np.all(np.isfinite(a)) and len(cache) == 3


def test_bf16_kv_cache_matches_bf16_oracle(gpu, tiny_ckpt):
    """a bf16 cache against the oracle's bf16 mode (each appended K/V element rounded to nearest
    bf16, ties to even): forward over a prompt, then pipelined decode, within 1e-3; the drift from
    the f32 cache is printed"""
    m = qe.Model.load_model(tiny_ckpt)
    om = oracle.Model(tiny_ckpt)
    prompt = qe.random_prompt(19, 30, TINY.vocab_size)
    steps = 40
    c16 = qe.KVCache(m, len(prompt) + steps, qe.QE_KV_BF16)
    c32 = qe.KVCache(m, len(prompt) + steps)
    o16 = om.new_cache(bf16=True)
    worst = drift = 0.0
    for pos, tok in enumerate(prompt):
        a = om.forward(int(tok), pos, o16)
        b = m.forward(int(tok), pos, c16)
        worst = max(worst, float(np.max(np.abs(a - b))))
        drift = max(drift, float(np.max(np.abs(m.forward(int(tok), pos, c32) - b))))
        assert oracle.argmax(a) == oracle.argmax(b), f"pos {pos}"
    first = oracle.argmax(a)
    toks, logits = m.decode(first, len(prompt), steps, c16, want_logits=True)
    tok = first
    for i in range(steps):
        a = om.forward(tok, len(prompt) + i, o16)
        worst = max(worst, float(np.max(np.abs(a - logits[i]))))
        tok = oracle.argmax(a)
        assert toks[i] == tok, f"step {i}"
    print(f"bf16 cache vs bf16 oracle: worst max-abs {worst:.2e}; bf16 vs f32 cache drift {drift:.2e}")
    assert worst < 1e-3
