"""CPU checks of the synthetic checkpoint and of the oracle against an independent Qwen3.

- the seeded random-init writer produces a safetensors file the `safetensors` library reads,
  with the HF Qwen3 names/shapes, bf16 ~ N(0, 0.02), unit norm gains and a tied lm_head;
- the oracle (C restatement of cpu_inference.rs) matches transformers' Qwen3ForCausalLM on the
  tiny checkpoint (committed fixture tests/golden/tiny_qwen3_transformers.npz, and live when
  transformers is importable): logits at every position and the greedy continuation.
"""
import os

import numpy as np
import pytest

import oracle
import qe

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TINY = qe.Config(256, 512, 2, 4, 2, 128, 1000, 1e-6, 1e6, 999)


@pytest.fixture(scope="module")
def tiny_fixture(tmp_path_factory):
    g = np.load(os.path.join(GOLDEN, "tiny_qwen3_transformers.npz"), allow_pickle=False)
    d = tmp_path_factory.mktemp("tiny_golden")
    path = qe.write_random_checkpoint(str(d), int(g["seed"]), TINY)
    return path, g


def test_checkpoint_format_and_statistics(tmp_path):
    torch = pytest.importorskip("torch")
    from safetensors.torch import load_file

    path = qe.write_random_checkpoint(str(tmp_path), 99, TINY)
    sd = load_file(path)
    H, I, QD, KD = 256, 512, 512, 256
    want = {"model.embed_tokens.weight": (1000, H), "lm_head.weight": (1000, H), "model.norm.weight": (H,)}
    for l in range(2):
        p = f"model.layers.{l}."
        want.update({p + "input_layernorm.weight": (H,), p + "post_attention_layernorm.weight": (H,),
                     p + "self_attn.q_proj.weight": (QD, H), p + "self_attn.k_proj.weight": (KD, H),
                     p + "self_attn.v_proj.weight": (KD, H), p + "self_attn.o_proj.weight": (H, QD),
                     p + "self_attn.q_norm.weight": (128,), p + "self_attn.k_norm.weight": (128,),
                     p + "mlp.gate_proj.weight": (I, H), p + "mlp.up_proj.weight": (I, H),
                     p + "mlp.down_proj.weight": (H, I)})
    assert set(sd) == set(want)
    for k, shape in want.items():
        assert tuple(sd[k].shape) == shape and sd[k].dtype == torch.bfloat16, k
        if k.endswith("norm.weight") or "layernorm" in k:
            assert bool((sd[k] == 1.0).all()), k
    assert torch.equal(sd["lm_head.weight"], sd["model.embed_tokens.weight"])  # tied
    w = torch.cat([sd[k].float().flatten() for k in want if k.endswith("proj.weight")])
    assert abs(float(w.mean())) < 1e-3 and abs(float(w.std()) - 0.02) < 5e-4
    # 8-byte aligned data section
    hl = int.from_bytes(open(path, "rb").read(8), "little")
    assert (8 + hl) % 8 == 0


def test_checkpoint_is_deterministic(tmp_path):
    a = qe.write_random_checkpoint(str(tmp_path / "a"), 5, TINY)
    b = qe.write_random_checkpoint(str(tmp_path / "b"), 5, TINY)
    c = qe.write_random_checkpoint(str(tmp_path / "c"), 6, TINY)
    da, db, dc = (open(p, "rb").read() for p in (a, b, c))
    assert da == db and da != dc


def test_random_prompt():
    p1 = qe.random_prompt(7, 130, 151936)
    p2 = qe.random_prompt(7, 130, 151936)
    assert p1.dtype == np.uint32 and (p1 == p2).all() and p1.max() < 151936 and len(set(p1.tolist())) > 120


def test_oracle_matches_transformers_fixture(tiny_fixture):
    path, g = tiny_fixture
    m = oracle.Model(path)
    c = m.new_cache()
    prompt = g["prompt"]
    for pos, tok in enumerate(prompt):
        lg = m.forward(int(tok), pos, c)
        np.testing.assert_allclose(lg, g["logits"][pos], atol=2e-5, rtol=0)
    # greedy continuation (the fixture's transformers run re-encodes the whole sequence each step)
    tok = oracle.argmax(lg)
    got = []
    for i in range(len(g["greedy"])):
        got.append(tok)
        lg = m.forward(tok, len(prompt) + i, c)
        tok = oracle.argmax(lg)
    assert got == g["greedy"].tolist()


def test_oracle_bf16_cache_matches_transformers_fixture(tiny_fixture):
    """the oracle's bf16 KV cache mode against transformers with a cache that rounds every stored
    key and value to bf16 (torch's conversion): logits at every prompt position and the greedy
    continuation. The tolerance is wider than the f32 run's 2e-5 because the two implementations'
    f32 keys differ in their last bits, and a key element near a bf16 rounding boundary then rounds
    to a neighbouring bf16 value in one of them (observed 8.5e-5); the oracle's f32 cache misses
    the same fixture by over 2e-3, so the bound still tells the two modes apart."""
    path, g = tiny_fixture
    m = oracle.Model(path)
    c = m.new_cache(bf16=True)
    c32 = m.new_cache()
    prompt = g["prompt"]
    miss32 = 0.0
    for pos, tok in enumerate(prompt):
        lg = m.forward(int(tok), pos, c)
        np.testing.assert_allclose(lg, g["logits_bf16kv"][pos], atol=3e-4, rtol=0)
        miss32 = max(miss32, float(np.max(np.abs(m.forward(int(tok), pos, c32) - g["logits_bf16kv"][pos]))))
    assert miss32 > 1e-3
    tok = oracle.argmax(lg)
    got = []
    for i in range(len(g["greedy_bf16kv"])):
        got.append(tok)
        lg = m.forward(tok, len(prompt) + i, c)
        tok = oracle.argmax(lg)
    assert got == g["greedy_bf16kv"].tolist()


def test_oracle_matches_transformers_live(tiny_fixture):
    pytest.importorskip("transformers")
    import sys

    sys.path.insert(0, GOLDEN)
    import make_tiny_fixture as mk

    path, g = tiny_fixture
    prompt, logits, gen = mk.run(path)
    np.testing.assert_array_equal(prompt, g["prompt"])
    np.testing.assert_allclose(logits, g["logits"], atol=1e-6, rtol=0)
    assert gen.tolist() == g["greedy"].tolist()
    _, logits16, gen16 = mk.run(path, kv_bf16=True)
    np.testing.assert_allclose(logits16, g["logits_bf16kv"], atol=1e-6, rtol=0)
    assert gen16.tolist() == g["greedy_bf16kv"].tolist()


def test_weight_bytes_formula_on_real_header(real_ckpt):
    # bench.rs:106-116 applied to the real-architecture checkpoint's header reproduces the value
    # the reference records for Qwen3-0.6B (mlx_baseline/results/mlx_m1_ai.json:287)
    m = oracle.Model(real_ckpt)
    assert m.weight_bytes_per_token() == 1_192_101_888
    assert m.kv_bytes_at(130) == 229_376 * 131
    assert len(m.tensors()) == 311
