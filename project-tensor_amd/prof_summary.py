"""Summarise rocprofv3 CSV output (``-f csv``) into the short text kept under profiles/.

    python project-tensor_amd/prof_summary.py stats <dir>     # kernel_stats.csv table
    python project-tensor_amd/prof_summary.py pmc <dir> ...   # per-kernel counter means

``stats`` prints, per kernel, calls, total and average duration.  ``pmc`` prints,
per kernel, the mean per dispatch of every counter in counter_collection.csv
(FETCH_SIZE and WRITE_SIZE are in KiB per dispatch).
"""
import collections
import csv
import glob
import os
import re
import sys


def _find(d, suffix):
    hits = sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True))
    if not hits:
        raise SystemExit(f"no *{suffix} under {d}")
    return hits


def _col(row, *names):
    low = {k.lower(): v for k, v in row.items()}
    for n in names:
        if n.lower() in low:
            return low[n.lower()]
    raise KeyError(f"none of {names} in {list(row)}")


def short(name, width=96):
    name = name.replace("(anonymous namespace)::", "")
    return re.sub(r"\(.*", "", name)[:width]


def stats(d):
    for path in _find(d, "kernel_stats.csv"):
        print(f"# {os.path.relpath(path, d)}")
        print(f"{'calls':>6} {'total_us':>11} {'avg_us':>10} {'min_us':>9} {'max_us':>9}  kernel")
        for r in csv.DictReader(open(path)):
            calls = int(_col(r, "Calls"))
            tot = float(_col(r, "TotalDurationNs")) / 1e3
            print(f"{calls:6d} {tot:11.1f} {tot / calls:10.2f} "
                  f"{float(_col(r, 'MinNs')) / 1e3:9.2f} {float(_col(r, 'MaxNs')) / 1e3:9.2f}  "
                  f"{short(_col(r, 'Name'))}")


def pmc(d):
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    disp = collections.defaultdict(set)
    for path in _find(d, "counter_collection.csv"):
        for r in csv.DictReader(open(path)):
            k = short(_col(r, "Kernel_Name"))
            did = _col(r, "Dispatch_Id")
            per[k][_col(r, "Counter_Name")] += float(_col(r, "Counter_Value"))
            disp[k].add(did)
    for k, c in per.items():
        n = len(disp[k])
        vals = "  ".join(f"{cn}={v / n:.1f}" for cn, v in sorted(c.items()))
        print(f"{n:5d} dispatches  {vals}  {k}")


if __name__ == "__main__":
    mode, dirs = sys.argv[1], sys.argv[2:]
    for d in dirs:
        {"stats": stats, "pmc": pmc}[mode](d)
