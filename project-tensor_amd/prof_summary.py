"""Summarise rocprofv3 CSV output (``-f csv``) into the short text kept under profiles/.

    python project-tensor_amd/prof_summary.py stats <dir>     # kernel_stats.csv table
    python project-tensor_amd/prof_summary.py pmc <dir> ...   # per-kernel counter means
    python project-tensor_amd/prof_summary.py traffic <fetch_dir> <write_dir> <calib_bytes>
    python project-tensor_amd/prof_summary.py mfma <dir> [n_xcd] [n_simd]
    python project-tensor_amd/prof_summary.py ranges <dir>   # kernels per roctx range

``stats`` prints, per kernel, calls, total and average duration.  ``pmc`` prints,
per kernel, the mean per dispatch of every counter in counter_collection.csv
(FETCH_SIZE and WRITE_SIZE are in KiB per dispatch).  ``mfma`` reads a run with
SQ_VALU_MFMA_BUSY_CYCLES, SQ_INSTS_VALU_MFMA_MOPS_F16 and GRBM_GUI_ACTIVE and prints,
per MFMA kernel, the fp16 flops executed per dispatch (MOPS x 512) and the MFMA
utilisation busy / (active cycles x SIMDs), where GRBM_GUI_ACTIVE is summed over the
n_xcd XCDs (default 8) and n_simd is the SIMD count (default 1024).  ``ranges``
reads a run with --kernel-trace --marker-trace and prints, per roctx push/pop range,
the kernels that started and ended inside it (count and total duration per kernel),
marking those that are not this library's (torch's at::native kernels and the like).
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


def _pmc_means(d, counter):
    tot = collections.defaultdict(float)
    disp = collections.defaultdict(set)
    for path in _find(d, "counter_collection.csv"):
        for r in csv.DictReader(open(path)):
            if _col(r, "Counter_Name") != counter:
                continue
            k = short(_col(r, "Kernel_Name"))
            tot[k] += float(_col(r, "Counter_Value"))
            disp[k].add(_col(r, "Dispatch_Id"))
    return {k: tot[k] / len(disp[k]) for k in tot}


def traffic(fetch_dir, write_dir, calib_bytes):
    """HBM bytes per dispatch from FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each
    scaled by what the counter reads for the calibration copy (a device copy of
    calib_bytes read + calib_bytes written): lines `traffic <kernel> <bytes>`."""
    calib_bytes = float(calib_bytes)
    f, w = _pmc_means(fetch_dir, "FETCH_SIZE"), _pmc_means(write_dir, "WRITE_SIZE")
    cal = [k for k in f if "copyBuffer" in k]
    if not cal or cal[0] not in w:
        raise SystemExit("calibration copy kernel not found in both runs")
    fs = calib_bytes / (f[cal[0]] * 1024.0)
    ws = calib_bytes / (w[cal[0]] * 1024.0)
    print(f"# calibration: {cal[0]} FETCH_SIZE {f[cal[0]]:.1f} KiB, WRITE_SIZE {w[cal[0]]:.1f} KiB "
          f"for {calib_bytes:.0f} B each way -> fetch scale {fs:.4f}, write scale {ws:.4f}")
    for k in sorted(f):
        name = k[5:] if k.startswith("void ") else k
        if k in w and (name.startswith("k_") or "_GLOBAL__N_" in name or k == cal[0]):
            fb, wb = f[k] * 1024.0 * fs, w[k] * 1024.0 * ws
            print(f"traffic {name.replace(' ', '')} {fb + wb:.0f} # fetch {fb:.0f} write {wb:.0f}")


def mfma(d, n_xcd=8, n_simd=1024):
    n_xcd, n_simd = int(n_xcd), int(n_simd)
    busy = _pmc_means(d, "SQ_VALU_MFMA_BUSY_CYCLES")
    mops = _pmc_means(d, "SQ_INSTS_VALU_MFMA_MOPS_F16")
    act = _pmc_means(d, "GRBM_GUI_ACTIVE")
    print(f"{'GFLOP/disp':>11} {'MFMA util':>9}  kernel   (GRBM_GUI_ACTIVE / {n_xcd} XCDs, {n_simd} SIMDs)")
    for k in sorted(busy):
        if not mops.get(k) or k not in act:
            continue
        util = busy[k] / (act[k] / n_xcd * n_simd)
        print(f"{mops[k] * 512 / 1e9:11.1f} {100 * util:8.1f}%  {k}")


def _ranges(d):
    """(name, start_ns, end_ns) of every roctx push/pop range in a marker trace."""
    out = []
    for path in _find(d, "marker_api_trace.csv"):
        for r in csv.DictReader(open(path)):
            name = r.get("Function") or r.get("Message") or r.get("Marker_Message") or ""
            if not name:
                continue
            out.append((name, int(_col(r, "Start_Timestamp")), int(_col(r, "End_Timestamp"))))
    return sorted(out, key=lambda x: x[1])


def ranges(d):
    kernels = []
    for path in _find(d, "kernel_trace.csv"):
        for r in csv.DictReader(open(path)):
            kernels.append((int(_col(r, "Start_Timestamp")), int(_col(r, "End_Timestamp")),
                            short(_col(r, "Kernel_Name"), 120)))
    for name, t0, t1 in _ranges(d):
        inside = [k for k in kernels if k[0] >= t0 and k[1] <= t1]
        per = collections.OrderedDict()
        for s0, s1, k in sorted(inside):
            c = per.setdefault(k, [0, 0.0])
            c[0] += 1
            c[1] += (s1 - s0) / 1e3
        foreign = [k for k in per if not _ours(k)]
        print(f"## {name}: {len(inside)} kernels, {sum(c[1] for c in per.values()):.1f} us of "
              f"kernel time, {len(foreign)} kernel names not from libtgbwd")
        for k, (n, us) in per.items():
            print(f"  {'  ' if _ours(k) else '**'} {n:4d} {us:10.1f} us  {k}")


def _ours(name):
    n = name[5:] if name.startswith("void ") else name
    return n.startswith("k_") or "_GLOBAL__N_" in n


if __name__ == "__main__":
    mode, args = sys.argv[1], sys.argv[2:]
    if mode == "traffic":
        traffic(*args)
    elif mode == "mfma":
        mfma(*args)
    else:
        for d in args:
            {"stats": stats, "pmc": pmc, "ranges": ranges}[mode](d)
