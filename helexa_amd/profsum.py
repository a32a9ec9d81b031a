"""Short text summaries of rocprofv3 CSV output for this library's kernels.

    python -m helexa_amd.profsum stats  <kernel_stats.csv> <out.txt> <title> <command> [<kernel_trace.csv>]
    python -m helexa_amd.profsum mfma   <counter_collection.csv> <out.txt> <title> <command>
    python -m helexa_amd.profsum pmc    <fetch_counter_collection.csv> <write_counter_collection.csv>
                                        <out.txt> <title> <command-fetch> <command-write> <copy_bytes>
                                        [<calibration fetch csv> <calibration write csv>]

`stats` keeps the library's kernels (names starting with "hx::" or "void hx::")
from a `--kernel-trace --stats` run: calls, average / min / max duration; given
the same run's kernel trace it adds the average over the dispatches bench.py
times with HIP events (those queued behind a sleep kernel).

`mfma` reads one `--pmc` run of MFMA_COUNTERS and reports per kernel the MFMA
flops and the share of cycles the matrix cores were busy.

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


SLEEP_KERNEL = "spin_kernel"   # torch.cuda._sleep


def timed_windows(trace_csv: str):
    """Per kernel, the durations (us) of the dispatches bench.py times with HIP
    events: the library's dispatches queued behind a sleep kernel. A window opens
    at the end of each sleep-kernel dispatch and closes at the first dispatch that
    is not one of the library's kernels (or at the next sleep)."""
    rows = []
    with open(trace_csv, newline="") as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    out = defaultdict(list)
    inside = False
    for t0, t1, name in rows:
        if SLEEP_KERNEL in name:
            inside = True
        elif not _is_hx(name):
            inside = False
        elif inside:
            out[_short(name)].append((t1 - t0) / 1e3)
    return out


def stats(csv_path: str, out_path: str, title: str, command: str, trace_csv: str = None) -> str:
    """kernel table from a --stats run; with trace_csv (the same run's
    --kernel-trace), also the average over the dispatches bench.py times
    (timed_windows), which is what its event-timed figures are compared with"""
    rows = []
    with open(csv_path, newline="") as f:
        for r in csv.DictReader(f):
            if _is_hx(r["Name"]):
                rows.append((_short(r["Name"]), int(r["Calls"]), float(r["AverageNs"]) / 1e3,
                             float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3, float(r["Percentage"])))
    rows.sort(key=lambda x: -x[1] * x[2])
    win = timed_windows(trace_csv) if trace_csv else {}
    lines = [f"# {title}", "", f"command: {command}", "($REPO is the repository root)", ""]
    if trace_csv:
        lines += ["timed_avg_us: average over the dispatches queued behind a sleep kernel (the launches bench.py",
                  "times with HIP events recorded by each kernel's own dispatch); avg_us: over every dispatch", ""]
    lines.append(f"{'kernel':58s} {'calls':>7s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'%time':>7s}"
                 + (f" {'timed_calls':>11s} {'timed_avg_us':>12s}" if trace_csv else ""))
    for n, c, a, lo, hi, p in rows:
        line = f"{n:58s} {c:7d} {a:9.3f} {lo:9.3f} {hi:9.3f} {p:7.2f}"
        if trace_csv:
            w = win.get(n, [])
            line += f" {len(w):11d} {sum(w) / len(w):12.3f}" if w else f" {0:11d} {'-':>12s}"
        lines.append(line)
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


def read_stats_avg(path: str, kernel_substr: str, timed: bool = True):
    """average duration (us) of the first kernel whose name contains
    kernel_substr, from a file written by stats(): the timed-window average when
    the file has one (and timed is set), else the all-dispatch average; None if
    absent"""
    if not os.path.exists(path):
        return None
    with open(path) as f:
        text = f.read()
    has_timed = "timed_avg_us" in text
    for line in text.splitlines():
        n = 7 if has_timed else 5
        parts = line.rsplit(None, n)   # kernel name (may hold spaces), then the numbers
        if len(parts) == n + 1 and kernel_substr in parts[0]:
            try:
                if has_timed and timed:
                    return float(parts[7])
                return float(parts[2])
            except ValueError:
                continue
    return None


MFMA_COUNTERS = ("MfmaFlopsF16", "MfmaUtil", "SQ_BUSY_CU_CYCLES", "GRBM_GUI_ACTIVE")


def mfma(counter_csv: str, out_path: str, title: str, command: str) -> str:
    """MFMA work and utilisation per kernel from one --pmc run of MFMA_COUNTERS
    (rocprofv3's gfx950 derived metrics and their inputs):
      MfmaFlopsF16 = SQ_INSTS_VALU_MFMA_MOPS_F16 * 512, the f16 MFMA flops issued
      MfmaUtil     = 100 * SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE * SIMD_NUM),
                     the percentage of the kernel's active cycles in which the
                     matrix cores of a SIMD were busy, over all 1024 SIMDs
      GRBM_GUI_ACTIVE, SQ_BUSY_CU_CYCLES as collected (per-dispatch values)"""
    vals = defaultdict(lambda: defaultdict(list))
    with open(counter_csv, newline="") as f:
        for r in csv.DictReader(f):
            if _is_hx(r["Kernel_Name"]) and r["Counter_Name"] in MFMA_COUNTERS:
                vals[_short(r["Kernel_Name"])][r["Counter_Name"]].append(float(r["Counter_Value"]))
    lines = [f"# {title}", "", f"command: {command}", "($REPO is the repository root)", "",
             "MfmaFlopsF16 = SQ_INSTS_VALU_MFMA_MOPS_F16 * 512; MfmaUtil = 100 * SQ_VALU_MFMA_BUSY_CYCLES / "
             "(GRBM_GUI_ACTIVE * SIMD_NUM) (rocprofv3 derived metrics; means per dispatch)", "",
             f"{'kernel':50s} {'dispatches':>10s} {'mfma_flops_f16':>15s} {'mfma_util_pct':>13s} "
             f"{'gui_active':>12s} {'busy_cu_cycles':>15s}"]
    for k in sorted(vals):
        v = vals[k]
        mean = {c: (sum(v[c]) / len(v[c]) if v[c] else float("nan")) for c in MFMA_COUNTERS}
        n = max(len(v[c]) for c in MFMA_COUNTERS)
        lines.append(f"{k:50s} {n:10d} {mean['MfmaFlopsF16']:15.4e} {mean['MfmaUtil']:13.2f} "
                     f"{mean['GRBM_GUI_ACTIVE']:12.0f} {mean['SQ_BUSY_CU_CYCLES']:15.0f}")
    text = "\n".join(lines) + "\n"
    with open(out_path, "w") as f:
        f.write(text)
    return text


def read_mfma(path: str, kernel_substr: str):
    """{mfma_flops_f16, mfma_util_pct} of the first kernel whose name contains
    kernel_substr, from a file written by mfma(); None if absent"""
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            parts = line.rsplit(None, 5)
            if len(parts) == 6 and kernel_substr in parts[0]:
                try:
                    return {"mfma_flops_f16": float(parts[2]), "mfma_util_pct": float(parts[3])}
                except ValueError:
                    continue
    return None


if __name__ == "__main__":
    if sys.argv[1] == "stats":
        print(stats(*sys.argv[2:7]))
    elif sys.argv[1] == "mfma":
        print(mfma(*sys.argv[2:6]))
    elif sys.argv[1] == "pmc":
        print(pmc(*sys.argv[2:8], int(sys.argv[8]), *sys.argv[9:11]))
    else:
        raise SystemExit(__doc__)
