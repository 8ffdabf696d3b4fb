"""Markdown table of the kernels in a `rocprofv3 --kernel-trace --stats` database.

  python mac-gpu-compiler_amd/trace_summary.py RUN_results.db [--top N]
      [--window MARKER FIRST LAST] [--by-grid]

Reads the `top_kernels` view of the rocprofv3 SQLite output: name, calls, average and total
duration, share of GPU time. Kernel names are shortened (namespaces and parameter lists dropped).
With --window, only the dispatches from the FIRST-th to just before the LAST-th dispatch of a
kernel whose name contains MARKER (0-based, in start order) are counted, from the `kernels`
view: e.g. one multi-chunk prefill between two of its embedding launches. With --by-grid, the
dispatches of one kernel are also told apart by their grid (threads in x, y, z), e.g. one GEMM
kernel at two shapes.
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
    ap.add_argument("--window", nargs=3, metavar=("MARKER", "FIRST", "LAST"))
    ap.add_argument("--by-grid", action="store_true")
    a = ap.parse_args()
    db = sqlite3.connect(a.db)
    if a.window or a.by_grid:
        ks = db.execute("select name, start, duration, grid_x, grid_y, grid_z from kernels order by start").fetchall()
        if a.window:
            marker, first, last = a.window[0], int(a.window[1]), int(a.window[2])
            marks = [i for i, k in enumerate(ks) if marker in k[0]]
            sel = ks[marks[first]:marks[last]] if last < len(marks) else ks[marks[first]:]
        else:
            sel = ks
        agg = {}
        for name, _, dur, gx, gy, gz in sel:  # the kernels view reports nanoseconds
            key = short(name) + (f" grid ({gx}, {gy}, {gz})" if a.by_grid else "")
            c = agg.setdefault(key, [0, 0.0])
            c[0] += 1
            c[1] += dur / 1e3
        busy = sum(v[1] for v in agg.values())
        span = (sel[-1][1] + sel[-1][2] - sel[0][1]) / 1e3
        rows = sorted(((n, c, t / c, t, 100.0 * t / busy) for n, (c, t) in agg.items()), key=lambda r: -r[3])
        print(f"Window: {len(sel)} dispatches, {busy / 1e3:.3f} ms of kernel time in a {span / 1e3:.3f} ms span.")
        print()
        print("| Kernel | Calls | Avg (us) | Total (ms) | % of window |")
        print("|---|---|---|---|---|")
        for name, calls, avg, total, pct in rows[: a.top]:
            print(f"| `{name}` | {calls} | {avg:.3f} | {total / 1e3:.3f} | {pct:.1f} |")
        return
    rows = db.execute("select name, total_calls, average, total_duration, percentage from top_kernels "
                      f"order by total_duration desc limit {int(a.top)}").fetchall()
    print("| Kernel | Calls | Avg (us) | Total (ms) | % of GPU time |")
    print("|---|---|---|---|---|")
    for name, calls, avg, total, pct in rows:
        # the top_kernels view reports durations in microseconds
        print(f"| `{short(name)}` | {calls} | {avg:.3f} | {total / 1e3:.1f} | {pct:.1f} |")


if __name__ == "__main__":
    main()
