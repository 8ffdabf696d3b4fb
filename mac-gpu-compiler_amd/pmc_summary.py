"""Memory traffic beyond L2 per decode-step stage from rocprofv3 counter runs of qe_stage_pmc.

  python mac-gpu-compiler_amd/pmc_summary.py --fetch F.csv --write W.csv [--l2 L.csv] [--fused] \\
      [--copy-mib 1024] [--attn-pos 193] --out-json profiles/X.json --out-md profiles/X.md [--command TEXT]

F.csv / W.csv are the counter_collection CSVs of `rocprofv3 --pmc FETCH_SIZE` and
`rocprofv3 --pmc WRITE_SIZE` over `qe_stage_pmc` (every decode-step kernel at the Qwen3-0.6B
shapes, after a 1 GiB copy; --fused: the two-launch layer). On gfx950 FETCH_SIZE is built from the
L2's read requests to the memory fabric (TCC_EA0_RDREQ, 32/64/128-byte), so it counts bytes that
missed L2, which the MALL or HBM then serve; WRITE_SIZE counts L2 writes to the fabric. Each
counter is read in KiB per dispatch and scaled by what the same counter reads for the copy (N MiB
read, N MiB written, all of it through HBM), so `traffic_bytes` is L2-miss bytes per launch in
the copy kernel's units: an upper bound on the launch's HBM bytes.
L.csv (optional): `rocprofv3 --pmc TCC_HIT_sum TCC_MISS_sum TCC_EA0_RDREQ_sum` of the same
program, for each stage's L2 hit rate.
"""
import argparse
import csv
import json
import os
import re
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))

import qe  # noqa: E402  (stage_bytes, QWEN3_0_6B)

# k_mv_wide<TPR, CPT, RR, PRO, EPI, SM>: prologue / epilogue -> stage
_WIDE = {(2, 0): "qkv", (1, 0): "qkv", (3, 1): "o_proj", (1, 2): "gate_up", (0, 1): "down"}


def stage_of(kernel: str):
    for name, st in (("k_fused_attn", "attn_block"), ("k_fused_mlp", "mlp_block"), ("k_fused_reduce", "final_reduce")):
        if name in kernel:
            return st
    if "k_attn_split" in kernel:
        return "attention"
    if "k_argmax" in kernel:
        return "argmax"
    m = re.search(r"k_mv_wide<(\d+), (\d+), (\d+), (\d+), (\d+)", kernel)
    if m:
        return _WIDE.get((int(m.group(4)), int(m.group(5))))
    m = re.search(r"k_matvec<(\d+), (\d+), (\d+), (\d+)>", kernel)
    if m and int(m.group(4)) == 3:
        return "lm_head"
    return None


def read(path: str, counter: str):
    """[(kernel name, value)] for every dispatch of `counter` in a counter_collection CSV."""
    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter:
                rows.append((r["Kernel_Name"], float(r["Counter_Value"])))
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--copy-mib", type=int, default=1024)
    ap.add_argument("--copy-kernel", default="k_copy", help="substring naming the calibration copy kernel")
    ap.add_argument("--attn-pos", type=int, default=193, help="position the attention dispatches ran at")
    ap.add_argument("--out-json", required=True)
    ap.add_argument("--out-md", required=True)
    ap.add_argument("--command", default="")
    ap.add_argument("--no-prefetch", action="store_true",
                    help="the counter runs used qe_stage_pmc --no-prefetch (attention without the L2 prefetch)")
    ap.add_argument("--fused", action="store_true", help="the counter runs used qe_stage_pmc --fused")
    ap.add_argument("--pf-idle", action="store_true",
                    help="... --fused --pf-idle: the attention block's idle and run workgroups load the MLP block's gate|up"
                         " rows, the MLP block the next layer's q|k|v rows")
    ap.add_argument("--l2", default=None, help="counter CSV of TCC_HIT_sum, TCC_MISS_sum, TCC_EA0_RDREQ_sum")
    ap.add_argument("--persist-log", default=None, help="output of qe_stage_pmc --l2-persist (timings, no counters)")
    a = ap.parse_args()
    if a.fused:
        a.no_prefetch = True  # the fused launches carry no prefetch workgroups by default

    fetch, write = read(a.fetch, "FETCH_SIZE"), read(a.write, "WRITE_SIZE")
    l2 = {c: read(a.l2, c) for c in ("TCC_HIT_sum", "TCC_MISS_sum", "TCC_EA0_RDREQ_sum")} if a.l2 else {}
    copy_kib = a.copy_mib * 1024.0

    def copy_reading(rows):
        vals = [v for k, v in rows if a.copy_kernel in k]
        return max(vals) if vals else None

    cf, cw = copy_reading(fetch), copy_reading(write)
    if not cf or not cw:
        sys.exit(f"no '{a.copy_kernel}' dispatch in the counter files")
    ff, fw = copy_kib / cf, copy_kib / cw

    mean_pos = float(a.attn_pos)
    algo = qe.stage_bytes(qe.QWEN3_0_6B, mean_pos, 4)
    # the attention launch's own HBM traffic also holds the weights it prefetches into L2
    pf = 0 if a.no_prefetch else qe.prefetch_bytes(qe.QWEN3_0_6B, mean_pos, 4)
    stages = {}
    for rows, key in ((fetch, "fetch_kib"), (write, "write_kib"), *((l2[c], c) for c in l2)):
        for kernel, v in rows:
            st = stage_of(kernel)
            if st is None:
                continue
            m = re.search(r"k_\w+(<[^>]*>)?", kernel)
            d = stages.setdefault(st, {"kernel": m.group(0) if m else kernel})
            d.setdefault(key, []).append(v)
    out = {"copy_mib": a.copy_mib, "copy_fetch_kib": cf, "copy_write_kib": cw, "fetch_scale": round(ff, 4),
           "write_scale": round(fw, 4), "mean_position": mean_pos, "stages": {}}
    for st, d in stages.items():
        if "fetch_kib" not in d or "write_kib" not in d:
            continue
        fk = sum(d["fetch_kib"]) / len(d["fetch_kib"])
        wk = sum(d["write_kib"]) / len(d["write_kib"])
        traffic = (fk * ff + wk * fw) * 1024.0
        extra = pf if st == "attention" else 0
        cfg = qe.QWEN3_0_6B
        if a.pf_idle and st == "attn_block":
            # with fewer than 16 runs (up to 1024 positions) the idle and run slots load all 24
            # gate|up rows of each MLP workgroup, and the o_proj slots the down columns
            extra = 3 * cfg.intermediate_size * cfg.hidden_size * 2 if a.attn_pos < 1024 else 0
        if a.pf_idle and st == "mlp_block":
            # the MLP block loads the next layer's q|k|v rows
            qd = cfg.num_attention_heads * cfg.head_dim
            kd = cfg.num_key_value_heads * cfg.head_dim
            extra = (qd + 2 * kd) * cfg.hidden_size * 2
        out["stages"][st] = {
            "kernel": d["kernel"],
            "dispatches": len(d["fetch_kib"]),
            "fetch_kib": round(fk, 2),
            "write_kib": round(wk, 2),
            "traffic_bytes": int(round(traffic)),
            "algorithmic_bytes": int(round(algo[st])),
            "prefetch_bytes": int(extra),
            "traffic_over_algorithmic": round(traffic / (algo[st] + extra), 4),
        }
        if all(c in d for c in l2) and l2:
            hit = sum(d["TCC_HIT_sum"]) / len(d["TCC_HIT_sum"])
            miss = sum(d["TCC_MISS_sum"]) / len(d["TCC_MISS_sum"])
            out["stages"][st].update({
                "l2_hits": int(round(hit)), "l2_misses": int(round(miss)),
                "l2_hit_rate": round(hit / (hit + miss), 4) if hit + miss else None,
                "ea_read_requests": int(round(sum(d["TCC_EA0_RDREQ_sum"]) / len(d["TCC_EA0_RDREQ_sum"]))),
            })
    # the reread probe: two launches that each read the same 2 MiB from all 256 workgroups
    reread = [v for k, v in fetch if "k_reread" in k]
    if len(reread) >= 2:
        out["reread_probe_fetch_bytes"] = [int(round(v * ff * 1024.0)) for v in reread[:2]]
    persist = []
    if a.persist_log:
        persist = [l.strip() for l in open(a.persist_log) if l.startswith("l2-persist:")]
        out["l2_persist"] = persist
    with open(a.out_json, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")

    order = (["attn_block", "mlp_block", "final_reduce"] if a.fused else ["qkv", "attention", "o_proj", "gate_up", "down"]) \
        + ["lm_head", "argmax"]
    what = ("the two-launch decode layer (attention block, MLP block) in step order, then the final reduce, lm_head "
            "and argmax" if a.fused else "each decode-step kernel of the Qwen3-0.6B shapes")
    lines = [
        "# Memory traffic beyond L2 per launch: batch-1 decode step, Qwen3-0.6B architecture"
        + (", two launches per layer" if a.fused else ", one launch per stage"),
        "",
        "Counters: `FETCH_SIZE` then `WRITE_SIZE` (KiB per dispatch)" + (", then `TCC_HIT_sum`, `TCC_MISS_sum`, "
        "`TCC_EA0_RDREQ_sum`" if l2 else "") + ", one rocprofv3 run each, over",
        f"`qe_stage_pmc` ({what} on synthetic inputs, weights",
        "rotating over four copies; f32 KV). On gfx950 `FETCH_SIZE` counts the L2's read requests to the memory",
        "fabric, so these are L2-miss bytes (served by the MALL or HBM), an upper bound on HBM bytes.",
        "Scale: each counter divided into what it reads for the",
        f"{a.copy_mib} MiB copy kernel (read {a.copy_mib} MiB, write {a.copy_mib} MiB): FETCH_SIZE x {ff:.4f},",
        f"WRITE_SIZE x {fw:.4f}. Attention runs at position {a.attn_pos} ({a.attn_pos + 1} cached positions).",
        "Algorithmic bytes: weights + f32 input + f32 output per matvec; K/V history + q/k/v + output",
        "for attention (the figures `bench.py` divides by the launch time)." +
        (" The attention block's idle and run workgroups also load the MLP block's gate|up rows into L2, its"
         " o_proj workgroups the down columns, and the MLP block the next layer's q|k|v rows (prefetch bytes;"
         " the ratio is traffic over own + prefetch bytes)."
         if a.pf_idle else "") +
        ("" if a.no_prefetch else " The attention launch also streams the layer's gate/up and down weights into"
         " L2 (prefetch bytes, counted with those stages); its ratio is traffic over own + prefetch bytes."),
        "",
        "Commands (MI355X, one GPU; committed files only):",
        "",
        "```",
        a.command.strip(),
        "```",
        "",
        "| Stage | Kernel | Dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | L2-miss bytes/launch | Algorithmic bytes | Prefetch bytes | Ratio |"
        + (" L2 hits | L2 misses | L2 hit rate |" if l2 else ""),
        "|---|---|---|---|---|---|---|---|---|" + ("---|---|---|" if l2 else ""),
    ]
    for st in order:
        r = out["stages"].get(st)
        if r:
            row = (f"| {st} | `{r['kernel']}` | {r['dispatches']} | {r['fetch_kib']:.1f} | {r['write_kib']:.1f} | "
                   f"{r['traffic_bytes']:,} | {r['algorithmic_bytes']:,} | {r['prefetch_bytes']:,} | "
                   f"{r['traffic_over_algorithmic']:.3f} |")
            if l2 and "l2_hits" in r:
                row += f" {r['l2_hits']:,} | {r['l2_misses']:,} | {r['l2_hit_rate']:.3f} |"
            lines.append(row)
    if "reread_probe_fetch_bytes" in out:
        r1, r2 = out["reread_probe_fetch_bytes"]
        lines += [
            "",
            "**L2 between dispatches under this collection.** Two back-to-back launches of `k_reread` (every one of",
            f"256 workgroups reads the same 2 MiB) fetch {r1:,} and {r2:,} bytes beyond L2: each XCD's L2",
            "misses on the whole buffer again in the second launch. Per-dispatch counter collection does not",
            "keep L2 contents from one dispatch to the next, so no stage here can show L2 hits on lines an",
            "earlier launch loaded (the attention launch's prefetch of the gate/up and down weights included).",
        ]
    if persist:
        lines += [
            "",
            "Without the profiler L2 does keep them: `qe_stage_pmc --l2-persist` (graphs of 64 launches, each",
            "workgroup reading 64 KiB of its own XCD's 2 MiB share of a 16 MiB chunk):",
            "",
            "```",
            *persist,
            "```",
            "",
            "Re-reading the XCD's own lines runs well above the measured HBM read ceiling (~5.7 TB/s); rotating",
            "within the MALL or past it does not. So an earlier launch's loads serve a later launch from L2 in the engine's",
            "graphs, but only through the XCD that loaded them, and these counter tables cannot show it:",
            "that effect is measured by time only.",
        ]
    with open(a.out_md, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(json.dumps(out["stages"], indent=1))


if __name__ == "__main__":
    main()
