"""The device argmax rules against the reference's scan (main.rs:37-42; the GPU kernel
inference.metal:300-321): the first maximum wins, so ties go to the lowest index and -0.0 ties
+0.0; NaN never wins, except that a NaN at index 0 keeps the scan at 0; a row with nothing above
-inf gives 0.

Two device paths take greedy tokens: the verify pass's row argmax (qe_op_argmax runs that kernel
on caller-made rows), and the decode step's per-workgroup candidates in the lm_head launch plus the
reduction that feeds the next step. The second is driven through qe_decode and qe_verify_greedy on
tiny checkpoints whose lm_head and final-norm gains are set so that the logits hold exact ties,
NaNs and infinities at chosen rows.
"""
import json
import os

import numpy as np
import pytest

import oracle
import qe
from conftest import TINY

pytestmark = pytest.mark.gpu

BF16_NAN, BF16_ONE, BF16_MINUS_ONE, BF16_NINF = 0x7FC0, 0x3F80, 0xBF80, 0xFF80


def run_argmax(rows: np.ndarray) -> np.ndarray:
    import torch
    x = torch.from_numpy(np.ascontiguousarray(rows, dtype=np.float32)).cuda()
    out = torch.full((rows.shape[0],), -1, dtype=torch.int32, device="cuda")
    qe.op_argmax(x, out)
    torch.cuda.synchronize()
    return out.cpu().numpy().astype(np.int64)


def crafted_rows(n: int) -> list:
    rng = np.random.default_rng(5)
    rows = []
    base = rng.standard_normal(n).astype(np.float32)
    for i, j in [(3, 9), (0, 63), (64, 65), (900, 1023), (1024, 8191), (5000, n - 1), (8192, 8193)]:
        r = base.copy()
        r[i] = r[j] = 50.0  # exact tie across lanes, waves, load rounds and the thread block
        rows.append(r)
    r = base.copy(); r[0] = np.nan; r[77] = 99.0; rows.append(r)           # NaN at index 0 -> 0
    r = base.copy(); r[10] = np.nan; r[11] = 7.0; rows.append(r)           # NaN elsewhere skipped
    r = base.copy(); r[::3] = np.nan; rows.append(r)                      # many NaNs
    rows.append(np.full(n, -np.inf, np.float32))                          # all -inf -> 0
    rows.append(np.full(n, np.nan, np.float32))                           # all NaN -> 0
    r = np.full(n, -1.0, np.float32); r[0] = np.nan; rows.append(r)
    r = np.full(n, -1.0, np.float32); r[40] = -0.0; r[41] = 0.0; rows.append(r)    # -0.0 first
    r = np.full(n, -1.0, np.float32); r[40] = 0.0; r[4000] = -0.0; rows.append(r)  # +0.0 first
    r = np.full(n, -np.inf, np.float32); r[123] = np.inf; r[7] = np.inf; rows.append(r)
    r = np.full(n, -np.inf, np.float32); r[n - 1] = -3.0; rows.append(r)
    rows.append(np.zeros(n, np.float32))                                  # every entry ties
    for _ in range(4):
        rows.append(rng.standard_normal(n).astype(np.float32))
    return rows


@pytest.mark.parametrize("n", [1, 2, 63, 1000, 10000, 151936])
def test_row_argmax_rules(gpu, n):
    rows = [r for r in crafted_rows(max(n, 8194))]
    rows = np.stack([r[:n] for r in rows])
    got = run_argmax(rows)
    want = np.array([oracle.argmax(r) for r in rows])
    np.testing.assert_array_equal(got, want)


def test_row_argmax_many_rows(gpu):
    """more rows than one launch takes (65535): the op works through them in batches"""
    rng = np.random.default_rng(9)
    rows = rng.standard_normal((70000, 7)).astype(np.float32)
    rows[65534:65537, :] = 1.0  # all-equal rows at the batch edge: index 0 wins
    rows[69999, 3] = np.nan
    got = run_argmax(rows)
    want = np.array([oracle.argmax(r) for r in rows])
    np.testing.assert_array_equal(got, want)


def patch_tensor(path: str, name: str, values: np.ndarray) -> None:
    """Overwrites one bf16 tensor's bytes in a safetensors file in place."""
    with open(path, "r+b") as f:
        hl = int.from_bytes(f.read(8), "little")
        hdr = json.loads(f.read(hl))
        a, b = hdr[name]["data_offsets"]
        data = np.ascontiguousarray(values, dtype=np.uint16).tobytes()
        assert len(data) == b - a, name
        f.seek(8 + hl + a)
        f.write(data)


def crafted_model(d: str, lm_col0: dict) -> str:
    """Tiny checkpoint whose final norm keeps only hidden dim 0 (gain 1 there, 0 elsewhere) and
    whose lm_head is zero except column 0 of the given rows: logit r = lm_col0[r] * xn0 exactly,
    and 0 (or 0 * inf = NaN) for the others."""
    path = qe.write_random_checkpoint(d, 4321, TINY)
    H, V = TINY.hidden_size, TINY.vocab_size
    g = np.zeros(H, np.uint16)
    g[0] = BF16_ONE
    patch_tensor(path, "model.norm.weight", g)
    lm = np.zeros((V, H), np.uint16)
    for r, v in lm_col0.items():
        lm[r, 0] = v
    patch_tensor(path, "lm_head.weight", lm)
    return path


CASES = {
    # exact ties between two pairs of rows in different lm_head workgroups; which pair holds the
    # maximum depends on the sign of the normalized x[0], so both tie directions occur
    "ties": {37: BF16_ONE, 901: BF16_ONE, 120: BF16_MINUS_ONE, 500: BF16_MINUS_ONE},
    "nan_at_0": {0: BF16_NAN, 5: BF16_ONE, 6: BF16_MINUS_ONE},
    "nan_elsewhere": {3: BF16_NAN, 37: BF16_ONE, 901: BF16_ONE, 120: BF16_MINUS_ONE, 500: BF16_MINUS_ONE},
    # every logit is -inf or +inf (all equal), or NaN where 0 * inf arises
    "all_inf": {r: BF16_NINF for r in range(TINY.vocab_size)},
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_decode_and_verify_argmax_rules(gpu, tmp_path, case):
    path = crafted_model(str(tmp_path), CASES[case])
    m = qe.Model.load_model(path)
    om = oracle.Model(path)
    prompt = qe.random_prompt(29, 6, TINY.vocab_size)
    steps = 12
    c = qe.KVCache(m, len(prompt) + steps + 1)
    oc = om.new_cache()
    for pos, tok in enumerate(prompt):
        ol = om.forward(int(tok), pos, oc)
    gl = m.prefill(prompt, 0, c)
    first = oracle.argmax(ol)
    assert oracle.argmax(gl) == first
    toks, logits = m.decode(first, len(prompt), steps, c, want_logits=True)
    tok, want = first, []
    for i in range(steps):
        ol = om.forward(tok, len(prompt) + i, oc)
        tok = oracle.argmax(ol)
        want.append(tok)
        # the decode step's device argmax applies the rule to its own logits
        assert toks[i] == oracle.argmax(logits[i]), f"step {i}"
    assert toks == want
    if case == "nan_at_0" or case == "all_inf":
        assert set(toks) == {0}
    elif case == "ties":
        assert set(toks) <= {37, 120} and len(set(toks)) >= 1
    # the verify pass's device argmax on the same sequence
    ids = [first] + toks[:3]
    c2 = qe.KVCache(m, len(prompt) + steps + 1)
    m.prefill(prompt, 0, c2, want_logits=False)
    got = m.verify_greedy(ids, len(prompt), c2)
    assert got.tolist() == toks[:4]
