"""Multi-token forward (chunked prefill, k-token verify) on the matrix cores, through the C ABI.

The reference has only token-by-token prefill (bench.rs:174-176), so its own invariant is the
oracle: chunked logits must equal sequential forward logits within the parity bar
(tests/metal_parity.rs:14), and decoding must continue from a chunk-prefilled cache exactly as from
a sequentially prefilled one.
"""
import numpy as np
import pytest

import oracle
import qe
from conftest import DECODE_STEPS, PROMPT_LEN, PROMPT_SEED, TINY

pytestmark = pytest.mark.gpu

MAX_ABS_DIFF = 1e-2  # tests/metal_parity.rs:14


def bf16_round(a: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits (round to nearest even), as uint16"""
    u = a.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


# m <= 32 runs the skinny (split over k) kernel: one m-tile on 16 or 8 waves, or two m-tiles;
# m <= 64 the LDS-tiled 64 x 64 kernel (k % 64 == 0) or the register-only one (k = 96); larger m
# the 64-row kernel up to 1024 rows (192-column tiles where that fills the CUs more evenly: 512 x
# 6144, 1000 x 6144), then the 128-row tile kernel with 64 columns per tile, or 128 once that gives
# 256 tiles (2048 x 6144);
# odd stage counts (k = 32, 96), ragged rows and columns (n = 1000) included
@pytest.mark.parametrize("m,n,k", [(1, 64, 32), (5, 128, 64), (64, 1024, 1024), (100, 4096, 1024),
                                   (512, 1024, 3072), (37, 6144, 1024), (4, 32768, 1024), (3, 1000, 256),
                                   (16, 2048, 1024), (8, 4096, 3072), (17, 6144, 1024), (32, 1024, 3072),
                                   (2, 4096, 160), (40, 512, 96), (65, 64, 32), (128, 128, 32),
                                   (200, 4096, 1024), (300, 1000, 96), (513, 6144, 1024), (2048, 6144, 1024),
                                   (512, 6144, 1024), (1000, 6144, 64)])
def test_gemm_matches_float64(gpu, m, n, k):
    import torch
    rng = np.random.default_rng(m * 7 + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w16 = bf16_round(rng.standard_normal((n, k)).astype(np.float32) * 0.05)
    wf = (w16.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    ref = a.astype(np.float64) @ wf.T
    at, wt = torch.from_numpy(a).cuda(), torch.from_numpy(w16.view(np.int16)).cuda()
    ct = torch.full((m, n), float("nan"), device="cuda")
    qe.op_gemm_bf16(at, wt, ct)
    torch.cuda.synchronize()
    got = ct.cpu().numpy().astype(np.float64)
    # a is split into two bf16 halves (|error| <= 2^-17 |a|); f32 accumulation over k terms
    bound = (2.0 ** -16 + k * 2.0 ** -24) * (np.abs(a).astype(np.float64) @ np.abs(wf).T) + 1e-30
    assert np.all(np.abs(got - ref) <= bound), f"max excess {np.max(np.abs(got - ref) / bound)}"


# chunks of up to 4 tokens run their projections as multi-row matvecs (11 in chunks of 4: 4, 4, 3)
@pytest.mark.parametrize("n_prompt,chunk", [(1, 0), (11, 4), (100, 32), (300, 0), (513, 512), (700, 2048)])
def test_tiny_prefill_batch_matches_oracle(gpu, tiny_ckpt, n_prompt, chunk):
    m = qe.Model.load_model(tiny_ckpt)
    om = oracle.Model(tiny_ckpt)
    prompt = qe.random_prompt(29, n_prompt, TINY.vocab_size)
    cache = qe.KVCache(m, n_prompt + 24)
    got = m.prefill_batch(prompt, 0, cache, chunk=chunk)
    oc = om.new_cache()
    for pos, tok in enumerate(prompt):
        ref = om.forward(int(tok), pos, oc)
    d = float(np.max(np.abs(got - ref)))
    assert d < 1e-3, f"last-token logits diverge by {d}"
    assert oracle.argmax(got) == oracle.argmax(ref)
    assert len(cache) == n_prompt
    # decoding continues from the chunk-filled cache like the oracle does
    tok = oracle.argmax(ref)
    toks, logits = m.decode(tok, n_prompt, 20, cache, want_logits=True)
    for i in range(20):
        ref = om.forward(tok, n_prompt + i, oc)
        d = float(np.max(np.abs(logits[i] - ref)))
        assert d < 1e-3, f"decode step {i} after chunked prefill: {d}"
        tok = oracle.argmax(ref)
        assert toks[i] == tok


# k <= 4: the projections are multi-row matvecs over the k token rows; k = 5, 9, 17: the skinny
# GEMM; "skinny": k = 4 with the multi-row matvec switched off
@pytest.mark.parametrize("k,path", [(1, "rows"), (2, "rows"), (3, "rows"), (4, "rows"), (5, "rows"), (9, "rows"),
                                    (17, "rows"), (4, "skinny")])
def test_tiny_verify_matches_oracle(gpu, tiny_ckpt, k, path, monkeypatch):
    if path == "skinny":
        monkeypatch.setenv("QE_MV_ROWS", "0")  # read when the model loads
    m = qe.Model.load_model(tiny_ckpt)
    om = oracle.Model(tiny_ckpt)
    prefix = qe.random_prompt(31, 40, TINY.vocab_size)
    draft = qe.random_prompt(37, k, TINY.vocab_size)
    cache = qe.KVCache(m, 40 + k)
    m.prefill(prefix, 0, cache, want_logits=False)
    rows = m.verify(draft, 40, cache)
    oc = om.new_cache()
    for pos, tok in enumerate(prefix):
        om.forward(int(tok), pos, oc)
    for i, tok in enumerate(draft):
        ref = om.forward(int(tok), 40 + i, oc)
        d = float(np.max(np.abs(rows[i] - ref)))
        assert d < 1e-3, f"verify row {i}: {d}"
        assert oracle.argmax(rows[i]) == oracle.argmax(ref)
    assert len(cache) == 40 + k


@pytest.mark.parametrize("n_prompt,chunk", [(3, 0), (100, 32), (300, 0)])
def test_tiny_prefill_batch_bf16_kv_matches_bf16_oracle(gpu, tiny_ckpt, n_prompt, chunk):
    """bf16 cache: chunked prefill, a k = 4 verify and decode against the oracle's bf16 mode (each
    appended K/V element rounded to nearest bf16, ties to even) within 1e-3"""
    m = qe.Model.load_model(tiny_ckpt)
    om = oracle.Model(tiny_ckpt)
    prompt = qe.random_prompt(41, n_prompt, TINY.vocab_size)
    cb = qe.KVCache(m, n_prompt + 16, qe.QE_KV_BF16)
    oc = om.new_cache(bf16=True)
    got = m.prefill_batch(prompt, 0, cb, chunk=chunk)
    for pos, tok in enumerate(prompt):
        ref = om.forward(int(tok), pos, oc)
    assert float(np.max(np.abs(got - ref))) < 1e-3
    draft = qe.random_prompt(43, 4, TINY.vocab_size)
    rows = m.verify(draft, n_prompt, cb)
    for i, tok in enumerate(draft):
        ref = om.forward(int(tok), n_prompt + i, oc)
        assert float(np.max(np.abs(rows[i] - ref))) < 1e-3, f"verify row {i}"
    tok = oracle.argmax(ref)
    toks, logits = m.decode(tok, n_prompt + 4, 8, cb, want_logits=True)
    for i in range(8):
        ref = om.forward(tok, n_prompt + 4 + i, oc)
        assert float(np.max(np.abs(logits[i] - ref))) < 1e-3, f"decode step {i}"
        tok = oracle.argmax(ref)
        assert toks[i] == tok


def test_tiny_prefill_batch_continues_a_cache(gpu, tiny_ckpt):
    """chunked prefill from start_pos > 0 onto a cache filled token by token"""
    m = qe.Model.load_model(tiny_ckpt)
    om = oracle.Model(tiny_ckpt)
    prompt = qe.random_prompt(61, 150, TINY.vocab_size)
    cache = qe.KVCache(m, 160)
    m.prefill(prompt[:50], 0, cache, want_logits=False)
    got = m.prefill_batch(prompt[50:], 50, cache, chunk=64)
    oc = om.new_cache()
    for pos, tok in enumerate(prompt):
        ref = om.forward(int(tok), pos, oc)
    assert float(np.max(np.abs(got - ref))) < 1e-3
    assert len(cache) == 150


@pytest.mark.parametrize("chunk", [64, 128])
def test_tiny_prefill_streams_change_no_result(gpu, tiny_ckpt, monkeypatch, chunk):
    """chunks of more than 32 tokens go round-robin over QE_PREFILL_STREAMS streams, each chunk's
    attention ordered after the earlier chunks' K/V rows of the same layer: with 2, 3 and 4
    streams over ten or five GEMM-path chunks (and a short tail) the last token's logits equal one
    stream's bit for bit, and decoding from the filled cache gives the same tokens"""
    prompt = qe.random_prompt(71, 600, TINY.vocab_size)

    def run(streams):
        monkeypatch.setenv("QE_PREFILL_STREAMS", streams)
        m = qe.Model.load_model(tiny_ckpt)  # QE_PREFILL_STREAMS is read here
        c = qe.KVCache(m, len(prompt) + 8)
        lg = m.prefill_batch(prompt, 0, c, chunk=chunk)
        toks, _ = m.decode(oracle.argmax(lg), len(prompt), 6, c)
        return lg, toks

    lg1, t1 = run("1")
    for streams in ("2", "3", "4"):
        lgn, tn = run(streams)
        np.testing.assert_array_equal(lgn, lg1, err_msg=f"{streams} streams")
        assert tn == t1, f"{streams} streams"


def test_batch_argument_errors(gpu, tiny_ckpt):
    m = qe.Model.load_model(tiny_ckpt)
    cache = qe.KVCache(m, 8)
    with pytest.raises(qe.QeError) as e:
        m.prefill_batch(np.arange(9, dtype=np.uint32), 0, cache)  # past max_seq
    assert e.value.code == qe.QE_ERR_POS
    with pytest.raises(qe.QeError) as e:
        m.prefill_batch(np.arange(4, dtype=np.uint32), 0, cache, chunk=2049)
    assert e.value.code == qe.QE_ERR_ARG
    with pytest.raises(qe.QeError) as e:
        m.verify(np.zeros(65, dtype=np.uint32), 0, qe.KVCache(m, 80))
    assert e.value.code == qe.QE_ERR_ARG
    with pytest.raises(qe.QeError) as e:
        m.verify(np.zeros(2, dtype=np.uint32), 3, cache)  # nothing cached at 0..2
    assert e.value.code == qe.QE_ERR_POS


@pytest.mark.slow
def test_real_prefill_batch_then_decode_matches_fixture(gpu, real_ckpt):
    import os
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qwen3_0_6b_decode.npz"),
                allow_pickle=False)
    m = qe.Model.load_model(real_ckpt)
    V = m.config().vocab_size
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, V)
    cache = qe.KVCache(m, PROMPT_LEN + DECODE_STEPS + 1)
    logits = m.prefill_batch(prompt, 0, cache, chunk=64)  # three chunks, the last one partial
    first = oracle.argmax(logits)
    toks, step_logits = m.decode(first, PROMPT_LEN, DECODE_STEPS, cache, want_logits=True)
    got = [first] + toks
    ref = [int(t) for t in g["tokens"]]
    assert got == ref, f"greedy tokens diverge at {next(i for i in range(len(ref)) if got[i] != ref[i])}"
    idx = g["sample_idx"]
    for i, lg in enumerate(np.concatenate([logits[None], step_logits])):
        assert np.max(np.abs(lg[idx] - g["sample_val"][i])) < MAX_ABS_DIFF, f"step {i}"
        assert np.max(np.abs(lg[g["top_idx"][i]] - g["top_val"][i])) < MAX_ABS_DIFF, f"step {i}"


@pytest.mark.slow
@pytest.mark.parametrize("k", [2, 3, 4, 20])
def test_real_verify_matches_fixture(gpu, real_ckpt, k):
    """verify of the greedy continuation: row i is the oracle's logits after token i + 1"""
    import os
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qwen3_0_6b_decode.npz"),
                allow_pickle=False)
    m = qe.Model.load_model(real_ckpt)
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, m.config().vocab_size)
    cache = qe.KVCache(m, PROMPT_LEN + k)
    m.prefill_batch(prompt, 0, cache, want_logits=False)
    ref = [int(t) for t in g["tokens"]]
    rows = m.verify(np.array(ref[:k], dtype=np.uint32), PROMPT_LEN, cache)
    idx = g["sample_idx"]
    for i in range(k):
        assert oracle.argmax(rows[i]) == ref[i + 1], f"row {i}"
        assert np.max(np.abs(rows[i][idx] - g["sample_val"][i + 1])) < MAX_ABS_DIFF, f"row {i}"
        assert np.max(np.abs(rows[i][g["top_idx"][i + 1]] - g["top_val"][i + 1])) < MAX_ABS_DIFF, f"row {i}"
