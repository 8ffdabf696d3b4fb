"""Batch-1 greedy decode benchmark of the Qwen3-0.6B-architecture bf16 model on one MI355X.

Workload (the reference's bench protocol, metal_infrence_engine/src/bin/bench.rs:165-191, on
synthetic weights): a seeded random-init checkpoint, a 130-token prompt of uniform-random ids,
an untimed prefill, then one greedy decode of 128 steps (positions 130..257) with an f32 KV cache.
A "step" of this benchmark is that whole 128-token decode: --steps K times K of them back to back
(each from position 130 of the prefilled cache, which rewrites positions 130..257 before reading
them, so every step sees the state of a freshly prefilled cache) after --warmup W untimed ones.
value = 128 K / timed seconds. Every decode's 129 greedy tokens are checked against the oracle's
committed run. Prints ONE JSON line (the last line of stdout).

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--kv f32|bf16] [--decode-steps 128]
                  [--no-cpu-baseline]
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "mac-gpu-compiler_amd")
sys.path[:0] = [ROOT, PKG]

SEED = 20260101
PROMPT_SEED = 7
PROMPT_LEN = 130
SPEC_HBM_GBS = 8000.0  # MI355X HBM3E spec


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


READ_FORMS = {}  # form -> best GB/s of the last measured_read_ceiling() call


def measured_read_ceiling(torch, qe) -> float:
    """Best streaming-read GB/s over 1 and 2 GiB buffers (past the 256 MB MALL), as in
    tests/read_bandwidth.rs:69-141: sum-checked, best of 5 trials of ~8 GiB each. Two kernel forms
    are timed: the reference's grid-strided plain loads (qe_op_read_sum) and contiguous ranges per
    workgroup with non-temporal loads (qe_op_read_sum_nt), which read faster on gfx950; the ceiling
    is the better of the two (both are kept in READ_FORMS)."""
    forms = {"plain": qe.op_read_sum, "nt": qe.op_read_sum_nt}
    best_of = {f: 0.0 for f in forms}
    for gib in (1, 2):
        n = (gib << 30) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        part = torch.zeros(8192, dtype=torch.float32, device="cuda")
        grid = 8192
        for form, op in forms.items():
            part.zero_()
            op(src, part, grid)
            torch.cuda.synchronize()
            total = float(part[:grid].double().sum())
            if total != float(n):
                raise RuntimeError(f"read_sum ({form}) checksum {total} != {n}")
        reps = max(1, 8 // gib)
        for _ in range(5):
            for form, op in forms.items():
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(reps):
                    op(src, part, grid)
                e1.record()
                e1.synchronize()
                best_of[form] = max(best_of[form], (gib << 30) * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9)
        del src, part
    torch.cuda.empty_cache()
    READ_FORMS.clear()
    READ_FORMS.update({f: round(v, 1) for f, v in best_of.items()})
    best = max(best_of.values())
    # tests/read_bandwidth.rs:139-140: a reading above the spec means the buffer was served from
    # a cache, and the figure cannot be a DRAM ceiling
    if not 0.0 < best <= 1.05 * SPEC_HBM_GBS:
        raise RuntimeError(f"read ceiling {best:.1f} GB/s is outside (0, 1.05 x {SPEC_HBM_GBS:.0f}] GB/s: "
                           "the buffer is probably being served from cache")
    return best


def measured_copy(torch) -> float:
    """A plain 1 GiB device copy (torch's elementwise copy kernel): GB/s moved (read + write).
    Its known size (1 GiB read, 1 GiB written per launch) is also the scale for the rocprofv3
    FETCH_SIZE / WRITE_SIZE counters of the traffic summary."""
    n = (1 << 30) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    best = 0.0
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        dst.copy_(src)
        e1.record()
        e1.synchronize()
        best = max(best, 2 * (1 << 30) / (e0.elapsed_time(e1) * 1e-3) / 1e9)
    del src, dst
    torch.cuda.empty_cache()
    return best


def pmc_traffic(stage: str):
    """HBM bytes per launch of `stage` from the committed rocprofv3 counter summary
    (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by the same counter's reading for the
    1 GiB copy), or None when the summary does not cover that stage. The attention's figure is
    from the counter runs without the L2 prefetch, so that it covers the same bytes as the
    attention's algorithmic bytes (its own K/V, q/k/v and output); the two-launch layer's stages
    (attn_block, mlp_block, final_reduce) are from the counter runs of those launches. On gfx950
    FETCH_SIZE counts L2 read requests to the memory fabric: these are L2-miss bytes, an upper
    bound on HBM bytes."""
    if stage in ("attn_block", "mlp_block", "final_reduce"):
        name = "decode_step_fused_qwen3_0_6b_pmc.json"
    elif stage == "attention":
        name = "decode_step_qwen3_0_6b_pmc_no_prefetch.json"
    else:
        name = "decode_step_qwen3_0_6b_pmc.json"
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            summary = json.load(f)
    except (OSError, ValueError):
        return None
    row = summary.get("stages", {}).get(stage)
    return int(row["traffic_bytes"]) if row and "traffic_bytes" in row else None


def pmc_prefetch(stage: str):
    """bytes of a later launch's weights that one launch of `stage` loads into L2, as counted in the
    same counter summary (0 when it loads none), or None when the summary does not cover `stage`"""
    if stage not in ("attn_block", "mlp_block", "final_reduce"):
        return None
    try:
        with open(os.path.join(ROOT, "profiles", "decode_step_fused_qwen3_0_6b_pmc.json")) as f:
            row = json.load(f).get("stages", {}).get(stage)
    except (OSError, ValueError):
        return None
    return int(row.get("prefetch_bytes", 0)) if row else None


def cpu_baseline(ckpt: str, prompt, target_s: float = 15.0, min_steps: int = 16):
    """The oracle (C restatement of cpu_inference.rs) on this host at the benchmark's own
    positions: an untimed prefill of the whole prompt, then greedy decode steps from the prompt's
    end until ~target_s of decode work (at least min_steps); tok/s over the decode steps."""
    import oracle

    m = oracle.Model(ckpt)
    cache = m.new_cache()
    t0 = time.perf_counter()
    for pos, tok in enumerate(prompt):
        logits = m.forward(int(tok), pos, cache)
    prefill_s = time.perf_counter() - t0
    tok = oracle.argmax(logits)
    times = []
    t_start = time.perf_counter()
    pos = len(prompt)
    while len(times) < min_steps or (time.perf_counter() - t_start < target_s and len(times) < 128):
        t0 = time.perf_counter()
        logits = m.forward(tok, pos, cache)
        tok = oracle.argmax(logits)
        times.append(time.perf_counter() - t0)
        pos += 1
    tps = len(times) / sum(times)
    return {
        "value": round(tps, 3),
        "unit": "tok/s",
        "cores": oracle.get_threads(),
        "kind": "port",
        "sample": f"oracle forward (C restatement of cpu_inference.rs, rows split over {oracle.get_threads()} threads "
                  f"per matvec, attention single-threaded), untimed {len(prompt)}-token prefill ({prefill_s:.1f} s), "
                  f"then {len(times)} greedy decode steps at positions {len(prompt)}..{pos - 1}; median "
                  f"{sorted(times)[len(times) // 2] * 1e3:.1f} ms/token; host {cpu_model()}",
    }


def by_position(gaps, start: int, window: int):
    """tok/s per window of `window` decode steps (from the host-side gaps between tokens)."""
    out = []
    for i in range(0, len(gaps), window):
        w = gaps[i:i + window]
        out.append({"positions": f"{start + i}..{start + i + len(w) - 1}", "tok_s": round(len(w) / sum(w), 1)})
    return out


def graph_time_us(torch, launch, n: int, reps: int = 3) -> float:
    """Mean duration of one of n back-to-back launches: launch(i) for i < n captured as one
    graph on a side stream, replayed between two events; best of `reps` replays."""
    stream = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        launch(0)  # warm-up outside the capture (first launch, lazy setup)
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=stream):
            for i in range(n):
                launch(i)
    best = float("inf")
    with torch.cuda.stream(stream):  # replay() launches on the current stream: time it there
        g.replay()
        torch.cuda.synchronize()
        for _ in range(reps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            g.replay()
            e1.record(stream)
            e1.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e3 / n)
    del g
    return best


MALL_BYTES = 256 << 20


def sweep_matvec(torch, qe, ceiling: float, repeats: int):
    """The isolated matvec at the model's shapes (in -> out; 4096 and 6144 are the fused q|k|v and gate|up), bf16 W ~ N(0, 0.02), f32 x;
    `repeats` launches per shape rotating over distinct W copies worth >= 2x the 256 MB MALL, so
    every launch streams its weights from HBM (bench.rs-style bytes: out*in*2 + in*4 + out*4)."""
    rows = []
    shapes = [(1024, 2048), (1024, 1024), (2048, 1024), (1024, 3072), (3072, 1024), (1024, 4096), (1024, 6144), (1024, 151936)]
    # one GPU's share of each projection under 8-way tensor parallelism by KV head: q 2 heads,
    # k / v 1 head, o 2 heads in, gate|up 384 + 384 rows, down 384 in, lm_head 18,992 rows
    shard = [(1024, 256), (1024, 128), (256, 1024), (1024, 768), (384, 1024), (1024, 18992)]
    for cin, cout in shapes + shard:
        wbytes = cout * cin * 2
        copies = max(2, -(-2 * MALL_BYTES // wbytes))
        W = (torch.randn(copies, cout, cin, device="cuda") * 0.02).to(torch.bfloat16)
        x = torch.randn(cin, device="cuda")
        out = torch.empty(cout, device="cuda")
        us = graph_time_us(torch, lambda i: qe.op_matvec_bf16(W[i % copies], x, out,
                                                              stream=torch.cuda.current_stream()), repeats)
        b = wbytes + cin * 4 + cout * 4
        gbs = b / (us * 1e-6) / 1e9
        rows.append({"in": cin, "out": cout, "tp8_shard": (cin, cout) in shard, "us": round(us, 3), "bytes": b,
                     "gb_s": round(gbs, 1),
                     "frac_of_measured": round(gbs / ceiling, 4), "frac_of_spec": round(gbs / SPEC_HBM_GBS, 4),
                     "w_copies": copies})
        log(f"matvec {cin:5d} -> {cout:6d}: {us:8.3f} us  {gbs:7.1f} GB/s ({gbs / ceiling:.1%} of measured)")
        del W, x, out
        torch.cuda.empty_cache()
    return rows


def sweep_attention(torch, qe, ceiling: float, repeats: int):
    """The isolated decode attention (16 q heads, 8 KV heads, head_dim 128) over L cached
    positions, f32 q/K/V ~ N(0, 1); launches rotate over at least two K/V copies worth at least
    twice the 256 MB MALL, so every figure is an HBM one (tests/read_bandwidth.rs:139-140). Split into runs
    of 64 positions (the default) and single-pass (one workgroup per KV head).
    Bytes = 8192 L (K and V) + 2 * 16 * 128 * 4 (q in, out)."""
    rows = []
    n_heads, n_kv, D = 16, 8, 128
    for L in (128, 512, 2048, 8192, 32768):
        kvbytes = 2 * n_kv * L * D * 4
        copies = max(2, -(-2 * MALL_BYTES // kvbytes))
        K = torch.randn(copies, n_kv, L, D, device="cuda")
        V = torch.randn(copies, n_kv, L, D, device="cuda")
        q = torch.randn(n_heads * D, device="cuda")
        out = torch.empty(n_heads * D, device="cuda")
        work = torch.empty(qe.op_attention_work_bytes(n_heads, n_kv, L), dtype=torch.uint8, device="cuda")
        b = 8192 * L + 2 * n_heads * D * 4
        row = {"positions": L, "bytes": b, "kv_copies": copies}
        for name, splits in (("split", 0), ("single_pass", 1)):
            us = graph_time_us(torch, lambda i: qe.op_attention(q, K[i % copies], V[i % copies], out, L, n_heads, n_kv,
                                                               work, n_splits=splits,
                                                               stream=torch.cuda.current_stream()),
                               repeats if splits == 0 or L <= 2048 else max(4, repeats // 16))
            gbs = b / (us * 1e-6) / 1e9
            row[name] = {"us": round(us, 3), "gb_s": round(gbs, 1), "frac_of_measured": round(gbs / ceiling, 4)}
            log(f"attention L={L:6d} {name:11s}: {us:9.3f} us  {gbs:7.1f} GB/s")
        rows.append(row)
        del K, V, q, out, work
        torch.cuda.empty_cache()
    return rows


def prefill_bench(torch, qe, model, cfg, args):
    """Config 5: a 2048-token random prompt prefilled in chunks of 512 on the matrix cores
    (qe_prefill_batch), then k = 4 verify passes (qe_verify) against single decode steps.
    GEMM work per chunk = 2 M x (all projection weights) FLOP; the kernels issue it twice (the
    activations are split into two bf16 halves). Causal attention = 8192 x sum(p + 1) x L FLOP."""
    n, chunk = args.prefill_tokens, args.chunk
    ids = qe.random_prompt(11, n, cfg.vocab_size)
    cache = qe.KVCache(model, n + 8)
    H, I, L = cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers
    QD, KD = cfg.num_attention_heads * cfg.head_dim, cfg.num_key_value_heads * cfg.head_dim
    # on-box bf16 GEMM ceiling: torch (hipBLASLt) at the largest projection shape of a chunk
    a = torch.randn(chunk, H, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(2 * I, H, device="cuda", dtype=torch.bfloat16)
    wt = w.t().contiguous()
    for _ in range(3):
        torch.matmul(a, wt)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(50):
        torch.matmul(a, wt)
    e1.record()
    e1.synchronize()
    lib_tflops = 2.0 * chunk * 2 * I * H * 50 / (e0.elapsed_time(e1) * 1e-3) / 1e12
    model.prefill_batch(ids[:chunk], 0, cache, chunk=chunk, want_logits=False)  # warm-up, buffers
    best = float("inf")
    for _ in range(3):
        cache = qe.KVCache(model, n + 8)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        model.prefill_batch(ids, 0, cache, chunk=chunk, want_logits=False)
        torch.cuda.synchronize()
        best = min(best, time.perf_counter() - t0)
    # the same prompt in one chunk of n tokens (the largest chunk qe_prefill_batch takes)
    best_one = float("inf")
    if n <= 2048:
        model.prefill_batch(ids, 0, qe.KVCache(model, n + 8), chunk=n, want_logits=False)
        for _ in range(3):
            cache = qe.KVCache(model, n + 8)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            model.prefill_batch(ids, 0, cache, chunk=n, want_logits=False)
            torch.cuda.synchronize()
            best_one = min(best_one, time.perf_counter() - t0)
    proj = L * ((QD + 2 * KD) * H + H * QD + 2 * I * H + H * I)
    gemm_flop = 2.0 * n * proj
    attn_flop = 8192.0 * sum(p + 1 for p in range(n)) * L
    # the engine's matrix-core work: both bf16 halves of every GEMM
    mfma_flop = 2 * gemm_flop
    # k = 4 verify vs one decode step, on a cache holding the prompt
    draft = qe.random_prompt(13, 4, cfg.vocab_size)
    vcache = qe.KVCache(model, n + 16)
    model.prefill_batch(ids, 0, vcache, chunk=chunk, want_logits=False)
    model.verify(draft, n, vcache)
    t0 = time.perf_counter()
    reps = 20
    for _ in range(reps):
        model.verify(draft, n, vcache)
    verify_ms = (time.perf_counter() - t0) / reps * 1e3
    # the same pass with each row's greedy token taken on the device (qe_verify_greedy, what
    # prompt-lookup decoding calls): no logits leave the device
    t0 = time.perf_counter()
    for _ in range(reps):
        model.verify_greedy(draft, n, vcache)
    verify_greedy_ms = (time.perf_counter() - t0) / reps * 1e3
    t0 = time.perf_counter()
    for _ in range(reps):
        model.forward(int(draft[0]), n, vcache)
    forward_ms = (time.perf_counter() - t0) / reps * 1e3
    return {
        "metric": "prefill tok/s (2048-token prompt, chunks of 512, bf16 MFMA)",
        "value": round(n / best, 1),
        "unit": "tok/s",
        "ms": round(best * 1e3, 3),
        "prompt_tokens": n,
        "chunk": chunk,
        "gemm_flop": gemm_flop,
        "attention_flop": attn_flop,
        "achieved_tflops_algorithmic": round((gemm_flop + attn_flop) / best / 1e12, 2),
        "mfma_tflops_issued": round(mfma_flop / best / 1e12, 2),
        "mfma_peak_tflops": 2500.0,
        "hipblaslt_bf16_tflops_same_shape": round(lib_tflops, 1),
        "one_chunk_ms": round(best_one * 1e3, 3) if best_one < float("inf") else None,
        "one_chunk_tok_s": round(n / best_one, 1) if best_one < float("inf") else None,
        "verify_k4_ms": round(verify_ms, 3),
        "verify_greedy_k4_ms": round(verify_greedy_ms, 3),
        "forward_1_ms": round(forward_ms, 3),
        "verify_k4_tokens_per_s_if_all_accepted": round(4 / verify_ms * 1e3, 1),
    }


def lookup_bench(qe, model, cfg, args):
    """Prompt-lookup speculative decode (qe_decode_lookup) against plain greedy decode on the
    decode workload: the 130-token prompt, then --decode-steps greedy tokens. Both must give the same
    tokens; reports tok/s of each, verify passes and tokens per pass for k_max = 1 (a verify of 2
    rows, through the decode step's two launches per layer), 3 (4 rows, on the multi-row matvec),
    4 and 8."""
    import numpy as np
    P, K = args.prompt_len, args.decode_steps
    prompt = qe.random_prompt(PROMPT_SEED, P, cfg.vocab_size)

    def run(fn):
        best, out = float("inf"), None
        for _ in range(3):
            c = qe.KVCache(model, P + K + 1)
            first = int(np.argmax(model.prefill(prompt, 0, c)))
            t0 = time.perf_counter()
            out = fn(first, c)
            best = min(best, time.perf_counter() - t0)
        return best, first, out

    t_plain, first, (plain, _) = run(lambda f, c: model.decode(f, P, K, c))
    res = {"metric": f"greedy decode tok/s with prompt-lookup drafts ({P}-token prompt, {K} steps)", "unit": "tok/s",
           "plain_tok_s": round(K / t_plain, 1)}
    for k_max in (1, 3, 4, 8):
        t, _, (toks, st) = run(lambda f, c: model.decode_lookup(f, P, K, c, context=prompt, k_max=k_max, ngram=3))
        passes = st["passes"] + st["single_steps"]
        res[f"k{k_max}"] = {"tok_s": round(K / t, 1), "speedup": round(t_plain / t, 3), "same_tokens": toks == plain,
                            "tokens_per_pass": round(K / passes, 3), **st}

    # The random-init model's greedy output repeats itself far more than text does, so lookup
    # drafts are accepted more often than on text (the reference's MLX replay saw 1.22-1.32
    # tokens per pass, README.md:109-111). To time the speculative loop at those rates, a draft
    # source (qe_decode_drafted) makes its drafts from the known greedy continuation: on a
    # fraction a of its drafts the first token is the true next token (accepted), every other
    # draft token is wrong (rejected), so a pass emits 1 + a tokens on average. The loop is the
    # engine's own, with its adaptive rule (plain blocks while passes do not pay) and without it;
    # the emitted tokens are checked against the plain decode.
    seq = [first] + list(plain)

    def emulate(accept: float, kd: int, adaptive: bool):
        best, stats = float("inf"), None
        for _ in range(3):
            c = qe.KVCache(model, P + K + 1)
            model.prefill(prompt, 0, c, want_logits=False)
            credit = [0.0]

            def draft(hist, k):
                i = len(hist) - P - 1  # index of the last token in seq
                credit[0] += accept
                a = 1 if credit[0] >= 1.0 else 0
                credit[0] -= a
                return seq[i + 1:i + 1 + a] + [(seq[i + 1 + j] + 1) % cfg.vocab_size for j in range(a, min(kd, k))]

            t0 = time.perf_counter()
            out, st = model.decode_drafted(first, P, K, c, draft, context=prompt, k_max=kd, adaptive=adaptive)
            dt = time.perf_counter() - t0
            if out != list(plain):
                raise RuntimeError("drafted decode left the greedy sequence")
            if dt < best:
                passes = st["passes"] + st["single_steps"]
                best, stats = dt, {"tok_s": round(K / dt, 1), "speedup": round(t_plain / dt, 3),
                                   "tokens_per_pass": round((K - st["plain_steps"]) / max(passes, 1), 3),
                                   "ms_per_pass": round(dt / max(passes, 1) * 1e3, 3) if not st["plain_steps"] else None,
                                   **st}
        return stats

    res["emulated_text_acceptance"] = {
        f"{1 + a:.2f}_tokens_per_pass_k{kd}" + ("" if ad else "_always_draft"): emulate(a, kd, ad)
        for a in (0.22, 0.32) for kd in (1, 3) for ad in (True, False)}
    return res


def other_configs(torch, qe, model, cfg, ceiling: float, args) -> dict:
    """Short runs of the other workloads, so that one default `bench.py` run also measures them
    (outside the timed decode): the isolated matvec and attention sweeps (100 launches per shape
    instead of 1000), the 4096-step decode with an f32 cache (one untimed decode that captures its
    step graphs, then one timed), its tokens against the oracle's committed run, the
    2048-token chunked prefill with the k = 4 verify, and prompt-lookup decode (plain against
    k_max = 1, and one draft at the emulated text acceptance rates)."""
    import numpy as np
    out = {}
    t0 = time.time()
    # config 5 first: the two-stream chunked prefill runs slower once this process has run the
    # sweeps' launches on torch's streams (13.3 vs 11.0 ms for 2048 tokens in chunks of 512; the
    # streams then share hardware queues)
    pf = prefill_bench(torch, qe, model, cfg, args)
    out["prefill"] = {k: pf[k] for k in ("ms", "value", "chunk", "achieved_tflops_algorithmic", "mfma_tflops_issued",
                                         "one_chunk_ms", "verify_k4_ms", "verify_greedy_k4_ms", "forward_1_ms")
                      if k in pf}
    mv = sweep_matvec(torch, qe, ceiling, 100)
    out["matvec_sweep"] = {f"{r['in']}->{r['out']}" + (" (tp8 shard)" if r["tp8_shard"] else ""):
                           {"us": r["us"], "gb_s": r["gb_s"], "frac_of_measured": r["frac_of_measured"]} for r in mv}
    at = sweep_attention(torch, qe, ceiling, 100)
    out["attention_sweep"] = {str(r["positions"]): {k: r[k] for k in ("split", "single_pass")} for r in at}
    # config 4: 4096 greedy steps after the 130-token prompt, f32 cache
    P, DS = PROMPT_LEN, 4096
    prompt = qe.random_prompt(PROMPT_SEED, P, cfg.vocab_size)
    cache = qe.KVCache(model, P + DS + 1, qe.QE_KV_F32)
    first = int(np.argmax(model.prefill(prompt, 0, cache)))
    model.decode(first, P, DS, cache)
    torch.cuda.synchronize()
    gaps, last = [], [time.perf_counter()]

    def on_token(_t):
        now = time.perf_counter()
        gaps.append(now - last[0])
        last[0] = now

    t1 = time.perf_counter()
    last[0] = t1
    toks, _ = model.decode(first, P, DS, cache, on_token=on_token)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t1
    got = [first] + toks
    fx = os.path.join(ROOT, "tests", "golden", "qwen3_0_6b_long_f32.npz")
    ref = [int(t) for t in np.load(fx, allow_pickle=False)["tokens"]] if os.path.exists(fx) else []
    n = min(len(ref), len(got))
    out["long_decode_f32"] = {
        "tok_s": round(DS / wall, 1),
        "by_position": [by_position(gaps, P, 512)[i] for i in (0, -1)],
        "parity_vs_oracle_fixture": {"compared": n, "first_divergence": next((i for i in range(n) if got[i] != ref[i]), None)}
        if ref else None}
    del cache
    # prompt-lookup decode (f3): plain vs k_max = 1 (two-row verify passes), and the emulated
    # text acceptance rates with one draft, the emitted tokens checked against plain decode
    lk = lookup_bench(qe, model, cfg, args)
    out["lookup"] = {"plain_tok_s": lk["plain_tok_s"],
                     "k1": {k: lk["k1"][k] for k in ("tok_s", "speedup", "same_tokens", "tokens_per_pass")},
                     "emulated_text_acceptance_k1": {k: {"speedup": v["speedup"], "ms_per_pass": v["ms_per_pass"]}
                                                     for k, v in lk["emulated_text_acceptance"].items() if "_k1" in k}}
    out["seconds"] = round(time.time() - t0, 1)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10,
                    help="timed benchmark steps; one step is a whole --decode-steps greedy decode")
    ap.add_argument("--warmup", type=int, default=2, help="untimed decodes before the timed ones")
    ap.add_argument("--decode-steps", type=int, default=128, help="greedy decode steps (tokens) per benchmark step")
    ap.add_argument("--kv", choices=["f32", "bf16"], default="f32")
    ap.add_argument("--prompt-len", type=int, default=PROMPT_LEN)
    ap.add_argument("--workdir", default=os.environ.get("QE_BENCH_DIR", "/tmp/qe_bench"))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-profile", action="store_true",
                    help="skip the per-stage timing graphs (for counter-collection runs under QE_LAUNCH=eager)")
    ap.add_argument("--json-out", default=None, help="also write a detailed result JSON here")
    ap.add_argument("--prefill-tokens", type=int, default=2048)
    ap.add_argument("--chunk", type=int, default=512)
    ap.add_argument("--mode", choices=["decode", "matvec-sweep", "attention-sweep", "prefill", "lookup"],
                    default="decode",
                    help="decode: the batch-1 decode benchmark (one JSON line); the sweeps time the isolated "
                         "matvec at every model shape or the isolated attention at 128..32768 positions")
    ap.add_argument("--repeats", type=int, default=1000, help="launches per shape in the sweeps")
    ap.add_argument("--results", default=None,
                    help="decode mode: also write engine_hip_<chip>_<prompt>.json and append to "
                         "history_<chip>_<prompt>.jsonl here, in the reference harness's format")
    ap.add_argument("--label", default="", help="label stored in the --results record")
    ap.add_argument("--prompt-name", default="random130", help="prompt name in the --results file names")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="decode mode: skip the short runs of the other workloads (sweeps, 4096-step decode, "
                         "prefill) that the default run adds as other_configs")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this engine runs batch-1 decode on one GPU; --gpus {args.gpus} is not supported "
              "(how the path would shard across GPUs is a design note, not code)", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import qe

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    ckdir = os.path.join(args.workdir, f"qwen3_0_6b_seed{SEED}")
    ckpt = os.path.join(ckdir, "model.safetensors")
    if not os.path.exists(ckpt):
        t0 = time.time()
        qe.write_random_checkpoint(ckdir, SEED, qe.QWEN3_0_6B)
        log(f"wrote random-init checkpoint in {time.time() - t0:.1f}s")

    ceiling = measured_read_ceiling(torch, qe)
    log(f"measured HBM read ceiling: {ceiling:.1f} GB/s (plain loads {READ_FORMS['plain']:.1f}, "
        f"non-temporal {READ_FORMS['nt']:.1f})")
    if args.mode in ("matvec-sweep", "attention-sweep"):
        sweep = sweep_matvec if args.mode == "matvec-sweep" else sweep_attention
        rows = sweep(torch, qe, ceiling, args.repeats)
        result = {"metric": f"isolated {args.mode.split('-')[0]} GB/s (algorithmic bytes / launch time)",
                  "unit": "GB/s", "n_gpus": 1, "repeats": args.repeats, "measured_ceiling_gbs": round(ceiling, 1),
                  "peak": SPEC_HBM_GBS, "data": "synthetic", "rows": rows}
        if args.json_out:
            with open(args.json_out, "w") as f:
                json.dump(result, f, indent=1)
        print(json.dumps(result), flush=True)
        return
    copy_gbs = measured_copy(torch)
    log(f"measured 1 GiB device copy: {copy_gbs:.1f} GB/s (read + write)")

    t0 = time.time()
    model = qe.Model.load_model(ckpt)
    load_ms = (time.time() - t0) * 1e3
    log(f"loaded model in {load_ms / 1e3:.1f}s")
    cfg = model.config()
    if args.mode in ("prefill", "lookup"):
        if args.mode == "prefill":
            result = dict(prefill_bench(torch, qe, model, cfg, args), measured_ceiling_gbs=round(ceiling, 1))
        else:
            result = lookup_bench(qe, model, cfg, args)
        result.update(n_gpus=1, data="synthetic")
        if args.json_out:
            with open(args.json_out, "w") as f:
                json.dump(result, f, indent=1)
        print(json.dumps(result), flush=True)
        return
    kv_dtype = qe.QE_KV_BF16 if args.kv == "bf16" else qe.QE_KV_F32
    prompt = qe.random_prompt(PROMPT_SEED, args.prompt_len, cfg.vocab_size)
    K, W, DS = args.steps, args.warmup, args.decode_steps
    P = args.prompt_len
    el = 2 if kv_dtype == qe.QE_KV_BF16 else 4

    # the oracle's committed greedy run of this workload, if there is one
    ref = []
    fx = {(128, "f32"): "qwen3_0_6b_decode.npz", (4096, "f32"): "qwen3_0_6b_long_f32.npz",
          (4096, "bf16"): "qwen3_0_6b_long_bf16.npz"}.get((DS, args.kv))
    if fx and P == PROMPT_LEN and os.path.exists(os.path.join(ROOT, "tests", "golden", fx)):
        ref = [int(t) for t in np.load(os.path.join(ROOT, "tests", "golden", fx), allow_pickle=False)["tokens"]]

    # untimed: the prompt's prefill. Each decode below starts at position P of this cache and
    # rewrites positions P..P+DS-1 before reading them, so every one sees a freshly prefilled cache.
    cache = qe.KVCache(model, P + DS + 1, kv_dtype)
    logits = model.prefill(prompt, 0, cache)
    first = int(np.argmax(logits))
    stream = torch.cuda.ExternalStream(model.stream_handle())
    runs = []  # per timed decode: tokens, host gaps between tokens

    def decode_once():
        gaps, last = [], [time.perf_counter()]

        def on_token(_t):
            now = time.perf_counter()
            gaps.append(now - last[0])
            last[0] = now

        toks, _ = model.decode(first, P, DS, cache, on_token=on_token)
        return [first] + toks, gaps

    for _ in range(W):
        decode_once()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    t_start = time.perf_counter()
    for _ in range(K):
        runs.append(decode_once())
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    gpu_s = ev0.elapsed_time(ev1) * 1e-3
    tokens = runs[0][0]
    gaps = [g for _, gs in runs for g in gs]

    # every timed decode against the oracle's run (and against each other)
    parity = None
    if ref:
        n = min(len(ref), len(tokens))
        divs = [next((i for i in range(n) if r[i] != ref[i]), None) for r, _ in runs]
        parity = {"compared": n, "decodes": len(runs), "first_divergence": next((d for d in divs if d is not None), None)}
    if any(r != tokens for r, _ in runs):
        raise RuntimeError("the timed decodes produced different tokens")

    weight_bytes = model.weight_bytes_per_token()
    kv_bytes = [model.kv_bytes_at(p, kv_dtype) for p in range(P, P + DS)]
    bytes_per_decode = DS * weight_bytes + sum(kv_bytes)
    avg_bytes = bytes_per_decode / DS
    n_tok = K * DS
    tps = n_tok / wall
    per_token_gpu_s = gpu_s / n_tok
    achieved_gbs = avg_bytes / per_token_gpu_s / 1e9

    # per-stage launch durations: each stage's launches alone as a graph, replayed between two
    # HIP events on the engine stream (qe_profile_step), at 8 positions around the decode's mean
    # position, on the benchmark's cache (outside the timed region)
    n_prof = 8
    mid = P + DS // 2 - n_prof // 2
    prof_positions = list(range(mid, mid + n_prof))
    stages = {}
    for pos in ([] if args.no_profile else prof_positions):
        for name, us, launches in model.profile_step(tokens[pos - P], pos, cache):
            stages.setdefault(name, ([], launches))[0].append(us)
    mean_pos = sum(prof_positions) / n_prof
    stage_bytes = qe.stage_bytes(cfg, mean_pos, el)
    # Each stage's cost inside the step: the step's prefixes (for one launch per stage: q|k|v;
    # + attention; + o_proj; ...; + lm_head) are timed as graphs, and a stage costs the difference
    # between the prefix that ends with it and the one before; the argmax (the step's last launch,
    # which advances the step state and so cannot end a shorter prefix) costs the whole step minus
    # the prefix that ends with the lm_head. The costs add up to the step, which `reconciliation`
    # compares with the timed decode. Each stage replayed alone (its launches back to back, no
    # producer in front) is reported beside it as isolated_mean_us.
    mode = model.fused_layers()
    order = {2: ["layers", "lm_head", "argmax"],
             1: ["attn_block", "mlp_block", "final_reduce", "lm_head", "argmax"]}.get(
                 mode, ["qkv", "attention", "o_proj", "gate_up", "down", "lm_head", "argmax"])
    prefix_names = ["+".join(order[:i + 1]) for i in range(len(order) - 1)] + ["step"]
    kernel_table, prev = {}, None
    for name, pref in zip(order, prefix_names):
        if pref not in stages or name not in stages:
            break
        durs, launches = stages[pref]
        tot = [us * launches for us in durs]  # µs per step of the prefix, per profiled position
        inc = [t - p for t, p in zip(tot, prev)] if prev else tot
        prev = tot
        per_step = stages[name][1]
        mean_us = sum(inc) / len(inc) / per_step
        iso = sum(stages[name][0]) / len(stages[name][0])
        b = stage_bytes.get(name, 0)
        kernel_table[name] = {"launches_per_step": per_step, "mean_us": round(mean_us, 3),
                              "us_per_step": round(mean_us * per_step, 2), "isolated_mean_us": round(iso, 3),
                              "bytes_per_launch": int(b),
                              "achieved_gbs": round(b / (mean_us * 1e-6) / 1e9, 1) if mean_us > 0 else None}
        # two-launch layers: the same launches timed inside the whole step's graph from their
        # workgroups' clock stamps. in_step_us is a launch's share of the step (its first
        # workgroup's start to the next launch's; dispatch and drain included, as a kernel trace
        # counts a dispatch), in_exec_us its first workgroup's start to its last one's exit.
        share, window = stages.get("in_step:" + name), stages.get("in_exec:" + name)
        if share:
            ins = sum(share[0]) / len(share[0])
            kernel_table[name]["in_step_us"] = round(ins, 3)
            kernel_table[name]["in_step_gbs"] = round(b / (ins * 1e-6) / 1e9, 1) if ins > 0 else None
        if window:
            kernel_table[name]["in_exec_us"] = round(sum(window[0]) / len(window[0]), 3)
    pf = qe.prefetch_bytes(cfg, mean_pos, el) if qe.l2_prefetch_enabled() and mode == 0 else 0
    if "attention" in kernel_table:
        # the gate/up and down weights this launch also pulls into L2 (counted with those stages)
        kernel_table["attention"]["prefetch_bytes"] = int(pf)
    if kernel_table:
        dom_name = max(kernel_table, key=lambda k: kernel_table[k].get("in_step_us", kernel_table[k]["mean_us"])
                       * kernel_table[k]["launches_per_step"])
        dom = dict(kernel_table[dom_name])
        if "in_step_us" in dom:  # the launch's share of the step, as a kernel trace times each dispatch
            dom["mean_us"], dom["achieved_gbs"] = dom["in_step_us"], dom["in_step_gbs"]
    else:
        dom_name, dom = None, {"achieved_gbs": None, "bytes_per_launch": None, "mean_us": None,
                               "launches_per_step": None}

    result = {
        "metric": "decode tok/s @ batch 1, Qwen3-0.6B-arch bf16; achieved HBM GB/s vs roofline",
        "value": round(tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(wall / K * 1e3, 3),
        "ms_per_token": round(wall / n_tok * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        # what the kernels do with that type: the weights stream as bf16 and are unpacked exactly to
        # f32 (cpu_inference.rs:182-183), and every product, sum, norm and softmax runs in f32
        "arithmetic": "bf16 weights, f32 activations, f32 FMA and accumulation; KV cache " + args.kv,
        "data": "synthetic",
        "config": {
            "workload": f"Qwen3-0.6B-architecture decoder, seeded random-init bf16 weights (seed {SEED}), "
                        f"{P}-token random prompt (seed {PROMPT_SEED}) prefilled untimed, then {DS} greedy decode "
                        f"steps at batch 1 (positions {P}..{P + DS - 1}) per benchmark step, {args.kv} KV cache",
            "prompt_tokens": P,
            "decode_steps": DS,
            "kv_cache": args.kv,
            "batch": 1,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": dom["achieved_gbs"],
            "peak": SPEC_HBM_GBS,
            "unit": "GB/s",
            "frac": round(dom["achieved_gbs"] / SPEC_HBM_GBS, 4) if dom["achieved_gbs"] else None,
            "traffic": pmc_traffic(dom_name),
            "traffic_prefetch_bytes": pmc_prefetch(dom_name),
            "kernel": dom_name,
            "bytes_per_launch": dom["bytes_per_launch"],
            "mean_position": mean_pos,
            "launch_us": dom["mean_us"],
            "exec_us": dom.get("in_exec_us"),
            "launches_per_step": dom["launches_per_step"],
            "measured_ceiling_gbs": round(ceiling, 1),
            "measured_ceiling_forms_gbs": dict(READ_FORMS),
            "measured_copy_gbs": round(copy_gbs, 1),
        },
        "roofline_step": {
            "bound": "hbm",
            "achieved": round(achieved_gbs, 1),
            "peak": SPEC_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved_gbs / SPEC_HBM_GBS, 4),
            "frac_of_measured": round(achieved_gbs / ceiling, 4),
            "frac_of_measured_plain": round(achieved_gbs / READ_FORMS["plain"], 4),
            "bytes_per_token": int(round(avg_bytes)),
            "gpu_us_per_token": round(per_token_gpu_s * 1e6, 2),
        },
        "kernels": kernel_table,
        # the stages' in-step costs add up to the whole-step graph (timed at the profiled
        # positions); the decode's own GPU time per token is over positions 130..257
        "reconciliation": {
            "stages_us_per_token": round(sum(k["us_per_step"] for k in kernel_table.values()), 2) if kernel_table else None,
            "decode_gpu_us_per_token": round(per_token_gpu_s * 1e6, 2),
        },
        "median_ms_per_token": round(sorted(gaps)[len(gaps) // 2] * 1e3, 4) if gaps else None,
        "by_position": by_position(runs[0][1], P, 512) if DS >= 1024 else None,
        "gpu_ms_per_token": round(per_token_gpu_s * 1e3, 4),
        # 2: one persistent launch for all layers, 1: two launches per layer, 0: one per stage
        "layer_launches": {2: "persistent", 1: "two per layer", 0: "one per stage"}[mode],
        "weight_bytes_per_token": weight_bytes,
        "parity_vs_oracle_fixture": parity,
    }
    if not args.no_other_configs and DS == 128 and P == PROMPT_LEN and args.kv == "f32":
        result["other_configs"] = other_configs(torch, qe, model, cfg, ceiling, args)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(ckpt, prompt)
    if args.results:
        import harness
        rec = harness.engine_record(
            engine="hip", label=args.label, chip=torch.cuda.get_device_name(0), prompt_name=args.prompt_name,
            prompt_tokens=P, load_ms=load_ms, step_ms=[g * 1e3 for g in runs[0][1]], tokens=tokens,
            weight_bytes_per_token=weight_bytes, total_bytes=bytes_per_decode, peak_bw_gbs=SPEC_HBM_GBS,
            ref_tokens=ref, repo_dir=ROOT)
        log(f"wrote {harness.write_records(args.results, rec)}")
    if args.json_out:
        detail = dict(result, tokens=tokens, samples_ms=[round(g * 1e3, 4) for g in gaps])
        with open(args.json_out, "w") as f:
            json.dump(detail, f, indent=1)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
