"""HBM traffic per decode-step stage from two rocprofv3 counter runs of qe_stage_pmc.

  python mac-gpu-compiler_amd/pmc_summary.py --fetch F.csv --write W.csv [--copy-mib 1024] \\
      [--attn-pos 193] --out-json profiles/X.json --out-md profiles/X.md [--command TEXT]

F.csv / W.csv are the counter_collection CSVs of `rocprofv3 --pmc FETCH_SIZE` and
`rocprofv3 --pmc WRITE_SIZE` over `qe_stage_pmc` (every decode-step kernel at the Qwen3-0.6B
shapes, after a 1 GiB copy). Each counter is read in KiB per dispatch and scaled by what the same
counter reads for the copy (N MiB read, N MiB written), so `traffic_bytes` is HBM bytes per launch
in the copy kernel's units.
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
    a = ap.parse_args()

    fetch, write = read(a.fetch, "FETCH_SIZE"), read(a.write, "WRITE_SIZE")
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
    for rows, key in ((fetch, "fetch_kib"), (write, "write_kib")):
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
    with open(a.out_json, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")

    order = ["qkv", "attention", "o_proj", "gate_up", "down", "lm_head", "argmax"]
    lines = [
        "# HBM traffic per launch: batch-1 decode step, Qwen3-0.6B architecture",
        "",
        "Counters: `FETCH_SIZE` then `WRITE_SIZE` (KiB per dispatch), one rocprofv3 run each, over",
        "`qe_stage_pmc` (each decode-step kernel of the Qwen3-0.6B shapes on synthetic inputs, weights",
        "rotating over four copies; f32 KV). Scale: each counter divided into what it reads for the",
        f"{a.copy_mib} MiB copy kernel (read {a.copy_mib} MiB, write {a.copy_mib} MiB): FETCH_SIZE x {ff:.4f},",
        f"WRITE_SIZE x {fw:.4f}. Attention runs at position {a.attn_pos} ({a.attn_pos + 1} cached positions).",
        "Algorithmic bytes: weights + f32 input + f32 output per matvec; K/V history + q/k/v + output",
        "for attention (the figures `bench.py` divides by the launch time)." +
        ("" if a.no_prefetch else " The attention launch also streams the layer's gate/up and down weights into"
         " L2 (prefetch bytes, counted with those stages); its ratio is traffic over own + prefetch bytes."),
        "",
        "Commands (MI355X, one GPU; committed files only):",
        "",
        "```",
        a.command.strip(),
        "```",
        "",
        "| Stage | Kernel | Dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes/launch | Algorithmic bytes | Prefetch bytes | Ratio |",
        "|---|---|---|---|---|---|---|---|---|",
    ]
    for st in order:
        r = out["stages"].get(st)
        if r:
            lines.append(f"| {st} | `{r['kernel']}` | {r['dispatches']} | {r['fetch_kib']:.1f} | {r['write_kib']:.1f} | "
                         f"{r['traffic_bytes']:,} | {r['algorithmic_bytes']:,} | {r['prefetch_bytes']:,} | "
                         f"{r['traffic_over_algorithmic']:.3f} |")
    with open(a.out_md, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(json.dumps(out["stages"], indent=1))


if __name__ == "__main__":
    main()
