"""Markdown table of the kernels in a `rocprofv3 --kernel-trace --stats` database.

  python mac-gpu-compiler_amd/trace_summary.py RUN_results.db [--top N]

Reads the `top_kernels` view of the rocprofv3 SQLite output: name, calls, average and total
duration, share of GPU time. Kernel names are shortened (namespaces and parameter lists dropped).
"""
import argparse
import re
import sqlite3


def short(name: str) -> str:
    name = name.replace("void ", "").replace("qe::(anonymous namespace)::", "").replace("qe::", "")
    m = re.match(r"([\w:]+(<[^()]*>)?)", name)
    return m.group(1) if m else name[:60]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("db")
    ap.add_argument("--top", type=int, default=16)
    a = ap.parse_args()
    db = sqlite3.connect(a.db)
    rows = db.execute("select name, total_calls, average, total_duration, percentage from top_kernels "
                      f"order by total_duration desc limit {int(a.top)}").fetchall()
    print("| Kernel | Calls | Avg (us) | Total (ms) | % of GPU time |")
    print("|---|---|---|---|---|")
    for name, calls, avg, total, pct in rows:
        # the top_kernels view reports durations in microseconds
        print(f"| `{short(name)}` | {calls} | {avg:.3f} | {total / 1e3:.1f} | {pct:.1f} |")


if __name__ == "__main__":
    main()
