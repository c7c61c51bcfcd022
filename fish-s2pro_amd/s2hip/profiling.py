"""Summaries of rocprofv3 CSV output for the decode kernels.

    python3 -m s2hip.profiling stats  <dir>/<run>_kernel_stats.csv [--top N]
    python3 -m s2hip.profiling counters <dir>/<run>_counter_collection.csv \
        --kernel REGEX --copy-kernel REGEX --copy-bytes BYTES

`stats` prints rocprofv3's per-kernel table (calls, average / min / max
duration) with demangled template arguments kept, so a kernel instance can be
matched against the engine's live timing.

`traffic` reads a FETCH_SIZE run and a WRITE_SIZE run of the same command
and prints, per --row 'LABEL|KERNEL_REGEX|GRID_SIZE|ALGORITHMIC_BYTES' (GRID_SIZE
in threads, or * for any launch), the calibrated fetched + written bytes per
launch against the algorithmic bytes.

`mfma` averages per-dispatch SQ / GRBM counters (an MFMA counter run) for the
kernels matching each --kernel and derives MFMA utilisation and f16 MFMA
flops (SQ_INSTS_VALU_MFMA_MOPS_F16 x 512) per dispatch.

`tail` averages the durations of the last --count dispatches of one kernel
in a kernel-trace CSV (e.g. bench.py's timing loop, which runs after the
decode generations).

`budget` splits the decode frames of a kernel-trace CSV (one stream, so
kernels do not overlap) into kernel time and launch gaps: the window runs
from the --begin kernel's first dispatch after the last --after dispatch
(the last prefill) up to its (--frames + 1)-th dispatch, i.e. --frames whole
frames that each start with --begin; it prints each kernel's dispatches and
microseconds per frame and the idle time between kernels per frame.

`counters` averages one HBM byte counter (FETCH_SIZE or WRITE_SIZE, reported
in KiB per dispatch) over every dispatch of the kernel matching --kernel, and
calibrates it against a plain copy kernel of known size: the copy reads and
writes exactly --copy-bytes / 2 bytes each way, so
    scale = (copy_bytes / 2) / (copy counter * 1024)
and the kernel's HBM bytes per launch = counter * 1024 * scale.
"""

import argparse
import csv
import re
import statistics
import sys


def _rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _col(row, *names):
    for n in names:
        if n in row:
            return row[n]
    raise KeyError(f"none of {names} in CSV columns {sorted(row)}")


def short_name(name):
    name = re.sub(r"^void ", "", name)
    name = name.replace("s2::(anonymous namespace)::", "")
    return name


def stats(path, top):
    rows = _rows(path)
    out = []
    for r in rows:
        out.append((short_name(_col(r, "Name", "KernelName")), int(_col(r, "Calls")),
                    float(_col(r, "TotalDurationNs")), float(_col(r, "AverageNs")),
                    float(_col(r, "MinNs")), float(_col(r, "MaxNs")), float(_col(r, "Percentage"))))
    out.sort(key=lambda t: -t[2])
    lines = [f"{'kernel':72s} {'calls':>7s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'total_ms':>9s} {'%':>6s}"]
    for name, calls, tot, avg, mn, mx, pct in out[:top]:
        lines.append(f"{name[:72]:72s} {calls:7d} {avg / 1e3:9.2f} {mn / 1e3:9.2f} {mx / 1e3:9.2f} "
                     f"{tot / 1e6:9.2f} {pct:6.2f}")
    return "\n".join(lines)


def counter_mean(rows, kernel_re, counter):
    pat = re.compile(kernel_re)
    vals = []
    for r in rows:
        if _col(r, "Counter_Name") != counter:
            continue
        if pat.search(_col(r, "Kernel_Name")):
            vals.append(float(_col(r, "Counter_Value")))
    if not vals:
        raise SystemExit(f"no {counter} samples for kernels matching {kernel_re!r}")
    return statistics.fmean(vals), len(vals)


def counters(path, kernel_re, copy_re, copy_bytes):
    rows = _rows(path)
    names = sorted({_col(r, "Counter_Name") for r in rows})
    lines = []
    for counter in names:
        k, nk = counter_mean(rows, kernel_re, counter)
        c, nc = counter_mean(rows, copy_re, counter)
        scale = (copy_bytes / 2) / (c * 1024.0)
        lines.append(f"{counter}: kernel {k:.1f} KiB/dispatch over {nk} dispatches; copy {c:.1f} KiB/dispatch "
                     f"over {nc} dispatches (copy moves {copy_bytes / 2 / 1024:.0f} KiB each way); "
                     f"scale {scale:.4f}; kernel bytes/launch {k * 1024 * scale:.0f}")
    return "\n".join(lines)


def _scale(rows, counter, copy_re, copy_bytes):
    c, _ = counter_mean(rows, copy_re, counter)
    return (copy_bytes / 2) / (c * 1024.0)


def _launch_bytes(rows, counter, kernel_re, grid, scale):
    pat = re.compile(kernel_re)
    vals = [float(_col(r, "Counter_Value")) for r in rows
            if _col(r, "Counter_Name") == counter and pat.search(_col(r, "Kernel_Name"))
            and (grid == "*" or _col(r, "Grid_Size") == grid)]
    if not vals:
        raise SystemExit(f"no {counter} samples for {kernel_re!r} at grid {grid}")
    return statistics.fmean(vals) * 1024.0 * scale, len(vals)


def traffic(fetch_csv, write_csv, copy_re, copy_bytes, specs):
    fr, wr = _rows(fetch_csv), _rows(write_csv)
    fs, ws = _scale(fr, "FETCH_SIZE", copy_re, copy_bytes), _scale(wr, "WRITE_SIZE", copy_re, copy_bytes)
    lines = [f"calibration: FETCH_SIZE x {fs:.4f}, WRITE_SIZE x {ws:.4f} (copy kernel moving "
             f"{copy_bytes / 2 / 2**20:.0f} MiB each way)",
             f"{'kernel':34s} {'launches':>8s} {'fetch MB':>10s} {'write MB':>9s} {'total MB':>10s} "
             f"{'algo MB':>9s} {'ratio':>6s}"]
    for spec in specs:
        label, kre, grid, algo = spec.split("|")
        f, n = _launch_bytes(fr, "FETCH_SIZE", kre, grid, fs)
        w, _ = _launch_bytes(wr, "WRITE_SIZE", kre, grid, ws)
        a = float(algo)
        lines.append(f"{label:34s} {n:8d} {f / 1e6:10.3f} {w / 1e6:9.3f} {(f + w) / 1e6:10.3f} {a / 1e6:9.3f} "
                     f"{(f + w) / a:6.3f}")
    return "\n".join(lines)


def mfma(path, kernel_res):
    rows = _rows(path)
    lines = []
    for kre in kernel_res:
        pat = re.compile(kre)
        per = {}
        for r in rows:
            if pat.search(_col(r, "Kernel_Name")):
                per.setdefault(_col(r, "Counter_Name"), []).append(float(_col(r, "Counter_Value")))
        if not per:
            raise SystemExit(f"no samples for {kre!r}")
        m = {k: statistics.fmean(v) for k, v in per.items()}
        n = max(len(v) for v in per.values())
        parts = [f"{k} {v:.0f}" for k, v in sorted(m.items())]
        if "SQ_VALU_MFMA_BUSY_CYCLES" in m and "GRBM_GUI_ACTIVE" in m:
            # busy cycles summed over the SIMDs (4 per CU, 256 CUs)
            parts.append(f"MFMA busy {100 * m['SQ_VALU_MFMA_BUSY_CYCLES'] / (m['GRBM_GUI_ACTIVE'] * 1024):.1f} %")
        if "SQ_INSTS_VALU_MFMA_MOPS_F16" in m:
            parts.append(f"f16 MFMA {m['SQ_INSTS_VALU_MFMA_MOPS_F16'] * 512 / 1e9:.2f} GFLOP/dispatch")
        lines.append(f"{short_name(kre)} ({n} dispatches): " + "; ".join(parts))
    return "\n".join(lines)


def tail(path, kernel_re, count):
    pat = re.compile(kernel_re)
    durs = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if pat.search(_col(r, "Kernel_Name")):
                durs.append((int(_col(r, "End_Timestamp")) - int(_col(r, "Start_Timestamp"))) / 1e3)
    if not durs:
        raise SystemExit(f"no dispatches of {kernel_re!r}")
    last = durs[-count:]
    return (f"{kernel_re}: {len(durs)} dispatches, mean {statistics.fmean(durs):.3f} us; "
            f"last {len(last)}: mean {statistics.fmean(last):.3f} us, min {min(last):.3f}, max {max(last):.3f}")


def budget(path, after_re, begin_re, frames, top):
    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            rows.append((int(_col(r, "Start_Timestamp")), int(_col(r, "End_Timestamp")),
                         short_name(_col(r, "Kernel_Name"))))
    rows.sort()
    after, begin = re.compile(after_re), re.compile(begin_re)
    last_after = max((i for i, r in enumerate(rows) if after.search(r[2])), default=-1)
    starts = [i for i in range(last_after + 1, len(rows)) if begin.search(rows[i][2])]
    if len(starts) < frames + 1:
        raise SystemExit(f"{len(starts)} {begin_re!r} dispatches after the last {after_re!r}; need {frames + 1}")
    win = rows[starts[0]:starts[frames]]
    span = (rows[starts[frames]][0] - win[0][0]) / 1e3
    busy = 0.0
    per = {}
    for s0, e0, name in win:
        d = (e0 - s0) / 1e3
        busy += d
        c, t = per.get(name, (0, 0.0))
        per[name] = (c + 1, t + d)
    lines = [f"window: {len(win)} dispatches, {frames} frames, {span / frames:.1f} us per frame; kernels "
             f"{busy / frames:.1f} us per frame, gaps {(span - busy) / frames:.1f} us per frame "
             f"({100 * (span - busy) / span:.1f} %)",
             f"{'kernel':72s} {'per frame':>9s} {'avg_us':>8s} {'us/frame':>9s} {'%':>6s}"]
    for name, (c, t) in sorted(per.items(), key=lambda kv: -kv[1][1])[:top]:
        lines.append(f"{name[:72]:72s} {c / frames:9.2f} {t / c:8.2f} {t / frames:9.1f} {100 * t / span:6.2f}")
    return "\n".join(lines)


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    a = sub.add_parser("stats")
    a.add_argument("csv")
    a.add_argument("--top", type=int, default=30)
    b = sub.add_parser("counters")
    b.add_argument("csv")
    b.add_argument("--kernel", required=True)
    b.add_argument("--copy-kernel", required=True)
    b.add_argument("--copy-bytes", type=float, required=True)
    t = sub.add_parser("traffic")
    t.add_argument("fetch_csv")
    t.add_argument("write_csv")
    t.add_argument("--copy-kernel", required=True)
    t.add_argument("--copy-bytes", type=float, required=True)
    t.add_argument("--row", action="append", required=True)
    tl = sub.add_parser("tail")
    tl.add_argument("csv")
    tl.add_argument("--kernel", required=True)
    tl.add_argument("--count", type=int, required=True)
    bu = sub.add_parser("budget")
    bu.add_argument("csv")
    bu.add_argument("--after", required=True)
    bu.add_argument("--begin", required=True)
    bu.add_argument("--frames", type=int, required=True)
    bu.add_argument("--top", type=int, default=40)
    m = sub.add_parser("mfma")
    m.add_argument("csv")
    m.add_argument("--kernel", action="append", required=True)
    args = ap.parse_args(argv)
    if args.cmd == "stats":
        print(stats(args.csv, args.top))
    elif args.cmd == "traffic":
        print(traffic(args.fetch_csv, args.write_csv, args.copy_kernel, args.copy_bytes, args.row))
    elif args.cmd == "tail":
        print(tail(args.csv, args.kernel, args.count))
    elif args.cmd == "budget":
        print(budget(args.csv, args.after, args.begin, args.frames, args.top))
    elif args.cmd == "mfma":
        print(mfma(args.csv, args.kernel))
    else:
        print(counters(args.csv, args.kernel, args.copy_kernel, args.copy_bytes))


if __name__ == "__main__":
    sys.exit(main())
