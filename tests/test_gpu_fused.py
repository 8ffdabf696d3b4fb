"""The decode step with fused layers against the one-launch-per-stage step on the same checkpoint,
and against the oracle. Two forms (QE_FUSED at model load): 1 = two launches per layer (attention
block, MLP block), 2 = one persistent launch for all layers; both serve one KV head per XCD.

The fused layers split o_proj and down over the 8 XCDs by input columns and add the 8 partial
vectors to the residual stream, so their sums are ordered differently from the per-stage step's:
logits agree to float rounding (bound 1e-3 here, measured ~1e-5), greedy tokens exactly.
QE_FUSED=0 selects the per-stage step.
"""
import os

import numpy as np
import pytest

import oracle
import qe
from conftest import PROMPT_LEN, PROMPT_SEED

pytestmark = pytest.mark.gpu

# a checkpoint with the real widths (hidden 1024, 16/8 heads of 128, SwiGLU 3072) but 2 layers
# and a 4096-token vocabulary, so that the oracle runs it in seconds
NARROW = qe.Config(1024, 3072, 2, 16, 8, 128, 4096, 1e-6, 1e6, 4095)
NARROW_SEED = 4321
MODES = [1, 2]


@pytest.fixture(scope="module")
def narrow_ckpt(workdir):
    return qe.write_random_checkpoint(os.path.join(workdir, "narrow"), NARROW_SEED, NARROW)


def load(path, mode: int):
    old = os.environ.get("QE_FUSED")
    os.environ["QE_FUSED"] = str(mode)
    try:
        return qe.Model.load_model(path)
    finally:
        if old is None:
            del os.environ["QE_FUSED"]
        else:
            os.environ["QE_FUSED"] = old


def test_fused_path_selected_for_the_qwen3_shape(gpu, narrow_ckpt, tiny_ckpt):
    for mode in (0, 1, 2):
        assert load(narrow_ckpt, mode).fused_layers() == mode
    assert load(tiny_ckpt, 2).fused_layers() == 0  # other shapes keep the per-stage step


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("kv", [qe.QE_KV_F32, qe.QE_KV_BF16])
def test_fused_decode_matches_oracle_lockstep(gpu, narrow_ckpt, kv, mode):
    m = load(narrow_ckpt, mode)
    assert m.fused_layers() == mode
    om = oracle.Model(narrow_ckpt)
    V = NARROW.vocab_size
    prompt = qe.random_prompt(5, 40, V)
    cache = qe.KVCache(m, 400, kv)
    oc = om.new_cache(bf16=kv == qe.QE_KV_BF16)
    worst = 0.0
    for pos, tok in enumerate(prompt):
        a = om.forward(int(tok), pos, oc)
        b = m.forward(int(tok), pos, cache)
        worst = max(worst, float(np.max(np.abs(a - b))))
        assert oracle.argmax(a) == oracle.argmax(b), f"pos {pos}"
    first = oracle.argmax(a)
    steps = 300  # past 256 positions: 4, 8 and 16 attention runs per KV head
    toks, lg = m.decode(first, len(prompt), steps, cache, want_logits=True)
    tok = first
    for i in range(steps):
        a = om.forward(tok, len(prompt) + i, oc)
        worst = max(worst, float(np.max(np.abs(a - lg[i]))))
        assert toks[i] == oracle.argmax(a), f"decode step {i}"
        tok = toks[i]
    assert worst < 1e-3, worst
    print(f"fused mode {mode} lockstep kv={kv}: worst max-abs {worst:.2e}")


@pytest.mark.parametrize("mode", MODES)
def test_fused_matches_per_stage_step_long(gpu, narrow_ckpt, mode):
    """2600 positions: runs of 64 in 4..32 runs, then 32 runs of 128 (past 2048 positions)."""
    mf, ms = load(narrow_ckpt, mode), load(narrow_ckpt, 0)
    assert mf.fused_layers() == mode and ms.fused_layers() == 0
    V = NARROW.vocab_size
    prompt = qe.random_prompt(9, 24, V)
    out = []
    for m in (mf, ms):
        c = qe.KVCache(m, 2700)
        lg = m.prefill(prompt, 0, c)
        first = int(np.argmax(lg))
        toks, _ = m.decode(first, len(prompt), 2600, c)
        last = m.forward(toks[-1], len(prompt) + 2600, c)
        out.append((toks, last))
    assert out[0][0] == out[1][0]
    assert float(np.max(np.abs(out[0][1] - out[1][1]))) < 1e-3


@pytest.mark.parametrize("mode", MODES)
def test_fused_real_model_matches_fixture_tokens(gpu, real_ckpt, mode):
    """The bench workload: 130-token prompt + 128 greedy steps against the oracle's committed run
    (the per-stage step's own test is test_gpu_parity_real)."""
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qwen3_0_6b_decode.npz"),
                allow_pickle=False)
    m = load(real_ckpt, mode)
    assert m.fused_layers() == mode
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, m.config().vocab_size)
    cache = qe.KVCache(m, PROMPT_LEN + 129)
    logits = m.prefill(prompt, 0, cache)
    first = oracle.argmax(logits)
    toks, lg = m.decode(first, PROMPT_LEN, 128, cache, want_logits=True)
    got = [first] + toks
    ref = [int(t) for t in g["tokens"]]
    assert got == ref[:len(got)]
    idx = g["sample_idx"]
    worst = max(float(np.max(np.abs(l[idx] - g["sample_val"][i + 1]))) for i, l in enumerate(lg))
    assert worst < 1e-2, worst


@pytest.mark.parametrize("env", ["QE_FUSED_PF_IDLE", "QE_FUSED_PF_RUN", "QE_FUSED_PF_QKV", "QE_FUSED_PF_DOWN",
                                 "QE_FUSED_PF_ATTN", "QE_FUSED_PF_MLP"])
def test_fused_prefetch_switches_change_no_result(gpu, narrow_ckpt, monkeypatch, env):
    """the two-launch layer's L2 prefetches only load: turning the idle-slot, run-workgroup,
    next-layer q|k|v or down-column prefetch off, or adding prefetch workgroups, gives the same tokens and
    bit-identical logits, at 4, 8 and 16 attention runs per KV head (positions 40..339)"""
    prompt = qe.random_prompt(9, 40, NARROW.vocab_size)

    def run():
        m = load(narrow_ckpt, 1)
        assert m.fused_layers() == 1
        c = qe.KVCache(m, 400)
        lg0 = m.prefill(prompt, 0, c)
        toks, lg = m.decode(oracle.argmax(lg0), len(prompt), 300, c, want_logits=True)
        return toks, lg

    want_toks, want_lg = run()
    monkeypatch.setenv(env, "8" if env in ("QE_FUSED_PF_ATTN", "QE_FUSED_PF_MLP") else "0")
    toks, lg = run()
    assert toks == want_toks
    np.testing.assert_array_equal(lg, want_lg)


def test_fused_profile_step_times_layer_launches_in_step(gpu, narrow_ckpt):
    """qe_profile_step times the two-launch layer's launches inside the whole step from the clock
    stamps of their workgroups (the stamping compilation of the same kernels): a launch's share of
    the step (to the next layer launch's start; the step's last layer launch has none) is at least
    its own execution window, and the next forward still matches the oracle"""
    m = load(narrow_ckpt, 1)
    om = oracle.Model(narrow_ckpt)
    L = NARROW.num_hidden_layers
    prompt = qe.random_prompt(13, 41, NARROW.vocab_size)
    c = qe.KVCache(m, 400)
    m.prefill(prompt[:40], 0, c, want_logits=False)
    stages = {name: (us, n) for name, us, n in m.profile_step(int(prompt[40]), 40, c)}
    assert stages["in_step:attn_block"][1] == L and stages["in_step:mlp_block"][1] == L - 1
    assert stages["in_exec:attn_block"][1] == L and stages["in_exec:mlp_block"][1] == L
    for name in ("attn_block", "mlp_block"):
        share, window = stages["in_step:" + name][0], stages["in_exec:" + name][0]
        assert 0 < window <= share * 1.001, (name, window, share)
        assert share < stages["step"][0] * stages["step"][1]
    oc = om.new_cache()
    for pos, tok in enumerate(prompt):
        om.forward(int(tok), pos, oc)
    ref = om.forward(3, 41, oc)
    got = m.forward(3, 41, c)
    assert int(np.argmax(got)) == int(np.argmax(ref))
    assert float(np.max(np.abs(got - ref))) < 1e-3
