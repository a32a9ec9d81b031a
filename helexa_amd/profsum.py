"""Short text summaries of rocprofv3 CSV output for this library's kernels.

    python -m helexa_amd.profsum stats  <kernel_stats.csv> <out.txt> <title> <command>
    python -m helexa_amd.profsum pmc    <fetch_counter_collection.csv> <write_counter_collection.csv>
                                        <out.txt> <title> <command-fetch> <command-write> <copy_bytes>
                                        [<calibration fetch csv> <calibration write csv>]

`stats` keeps the library's kernels (names starting with "hx::" or "void hx::")
from a `--kernel-trace --stats` run: calls, average / min / max duration.

`pmc` reads two `--pmc FETCH_SIZE` / `--pmc WRITE_SIZE` runs (KiB per dispatch),
averages them per kernel, and calibrates both counters against the runtime's
device-to-device copy kernel of `copy_bytes` bytes run in the same program: the
HBM bytes of a kernel are counter * (copy_bytes / copy counter). The factor is
printed with the table. `bench.py` reads the calibrated per-launch bytes back
(`read_pmc`) for its roofline `traffic` field.
"""
from __future__ import annotations

import csv
import os
import sys
from collections import defaultdict

COPY_KERNEL = "__amd_rocclr_copyBuffer"


def _short(name: str) -> str:
    n = name.replace("void ", "")
    return n.split("(")[0] if "(" in n else n


def _is_hx(name: str) -> bool:
    return name.startswith("hx::") or name.startswith("void hx::")


def stats(csv_path: str, out_path: str, title: str, command: str) -> str:
    rows = []
    with open(csv_path, newline="") as f:
        for r in csv.DictReader(f):
            if _is_hx(r["Name"]):
                rows.append((_short(r["Name"]), int(r["Calls"]), float(r["AverageNs"]) / 1e3,
                             float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3, float(r["Percentage"])))
    rows.sort(key=lambda x: -x[1] * x[2])
    lines = [f"# {title}", "", f"command: {command}", "($REPO is the repository root)", "",
             f"{'kernel':58s} {'calls':>7s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'%time':>7s}"]
    for n, c, a, lo, hi, p in rows:
        lines.append(f"{n:58s} {c:7d} {a:9.3f} {lo:9.3f} {hi:9.3f} {p:7.2f}")
    text = "\n".join(lines) + "\n"
    with open(out_path, "w") as f:
        f.write(text)
    return text


def _counter_values(path: str, counter: str):
    vals = defaultdict(list)
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r.get("Counter_Name", counter) != counter:
                continue
            vals[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return vals


def _rel(path: str) -> str:
    return os.path.join(os.path.basename(os.path.dirname(path)), os.path.basename(path))


def _means(vals):
    return {k: (sum(v) / len(v), len(v)) for k, v in vals.items()}


def pmc(fetch_csv: str, write_csv: str, out_path: str, title: str, cmd_fetch: str, cmd_write: str,
        copy_bytes: int, calib_fetch_csv: str = None, calib_write_csv: str = None) -> str:
    """calib_*_csv: counter runs that hold the copy_bytes calibration copy when
    the measured runs do not (default: the measured runs themselves)"""
    fv = _counter_values(fetch_csv, "FETCH_SIZE")
    wv = _counter_values(write_csv, "WRITE_SIZE")
    fe, wr = _means(fv), _means(wv)
    cfv = _counter_values(calib_fetch_csv, "FETCH_SIZE") if calib_fetch_csv else fv
    cwv = _counter_values(calib_write_csv, "WRITE_SIZE") if calib_write_csv else wv
    # the calibration copies are the largest copy-kernel dispatches of the run
    cf = max((x for k, v in cfv.items() if COPY_KERNEL in k for x in v), default=None)
    cw = max((x for k, v in cwv.items() if COPY_KERNEL in k for x in v), default=None)
    if not cf or not cw:
        raise RuntimeError("no copy-kernel dispatch in the counter runs")
    kf = copy_bytes / (cf * 1024.0)
    kw = copy_bytes / (cw * 1024.0)
    lines = [f"# {title}", "", f"command (fetch): {cmd_fetch}", f"command (write): {cmd_write}",
             "($REPO is the repository root)", "",
             (f"calibration runs: {_rel(calib_fetch_csv)} and {_rel(calib_write_csv)} (the same two counters "
              "over bench.py --probe, which runs the copy)" if calib_fetch_csv else "calibration: the same runs"),
             f"calibration: {COPY_KERNEL} copying {copy_bytes} bytes reads FETCH_SIZE {cf:.1f} KiB and "
             f"WRITE_SIZE {cw:.1f} KiB per dispatch -> factors fetch {kf:.4f}, write {kw:.4f} "
             f"(HBM bytes = counter KiB * 1024 * factor)", "",
             f"{'kernel':58s} {'dispatches':>10s} {'fetch_KiB':>11s} {'write_KiB':>11s} {'hbm_bytes':>13s}"]
    for k in sorted(set(fe) | set(wr)):
        if not _is_hx(k):
            continue
        f_, n = fe.get(k, (0.0, 0))
        w_, _ = wr.get(k, (0.0, 0))
        hbm = f_ * 1024.0 * kf + w_ * 1024.0 * kw
        lines.append(f"{_short(k):58s} {n:10d} {f_:11.1f} {w_:11.1f} {hbm:13.0f}")
    text = "\n".join(lines) + "\n"
    with open(out_path, "w") as f:
        f.write(text)
    return text


def read_pmc(path: str, kernel_substr: str):
    """calibrated HBM bytes per dispatch of the first kernel whose name contains
    kernel_substr, from a file written by pmc(); None if absent"""
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.rsplit(None, 4)   # kernel name (may hold spaces), then four numbers
            if len(parts) == 5 and kernel_substr in parts[0]:
                try:
                    return float(parts[4])
                except ValueError:
                    continue
    return None


def read_stats_avg(path: str, kernel_substr: str):
    """average duration (us) of the first kernel whose name contains
    kernel_substr, from a file written by stats(); None if absent"""
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.rsplit(None, 5)   # kernel name (may hold spaces), then five numbers
            if len(parts) == 6 and kernel_substr in parts[0]:
                try:
                    return float(parts[2])
                except ValueError:
                    continue
    return None


if __name__ == "__main__":
    if sys.argv[1] == "stats":
        print(stats(*sys.argv[2:6]))
    elif sys.argv[1] == "pmc":
        print(pmc(*sys.argv[2:8], int(sys.argv[8]), *sys.argv[9:11]))
    else:
        raise SystemExit(__doc__)
