"""Per-kernel means of any rocprofv3 counters.

  python mac-gpu-compiler_amd/pmc_kernels.py RUN1.csv [RUN2.csv ...]

Each argument is the counter_collection CSV of one `rocprofv3 --pmc ...` run (one row per
dispatch and counter). Prints a markdown table: per kernel and grid size (threads), the dispatches
and the mean value of every counter per dispatch, over all runs given.
"""
import csv
import sys
from collections import defaultdict


def main(paths):
    vals = defaultdict(lambda: defaultdict(list))  # kernel -> counter -> values
    disp = defaultdict(set)
    for path in paths:
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                k = r["Kernel_Name"]
                k = (k if len(k) <= 60 else k[:57] + "...") + f" [grid {r.get('Grid_Size', '?')}]"
                vals[k][r["Counter_Name"]].append(float(r["Counter_Value"]))
                disp[k].add((path, r.get("Dispatch_Id", r.get("Correlation_Id", ""))))
    counters = sorted({c for k in vals for c in vals[k]})
    print("| Kernel | Dispatches | " + " | ".join(counters) + " |")
    print("|---|---|" + "---|" * len(counters))
    for k in sorted(vals, key=lambda k: -len(disp[k])):
        cells = []
        for c in counters:
            v = vals[k].get(c)
            cells.append(f"{sum(v) / len(v):,.0f}" if v else "")
        print(f"| `{k}` | {len(disp[k])} | " + " | ".join(cells) + " |")


if __name__ == "__main__":
    if len(sys.argv) < 2:
        sys.exit(__doc__)
    main(sys.argv[1:])
