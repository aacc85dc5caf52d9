"""Text summaries of rocprofv3 CSV output (``--output-format csv``).

    python -m dli.rocprof_summary stats RUN_kernel_stats.csv [--top 20]
    python -m dli.rocprof_summary pmc --fetch FETCH_counter_collection.csv \
        --write WRITE_counter_collection.csv --kernel REGEX [--kernel REGEX ...] \
        --copy-kernel REGEX --copy-bytes N
    python -m dli.rocprof_summary mfma --counters MFMA_counter_collection.csv \
        --stats RUN_kernel_stats.csv --kernel REGEX [--kernel REGEX ...]

``pmc`` averages FETCH_SIZE and WRITE_SIZE (KiB per dispatch) over the dispatches of each
kernel and scales them by the factor that makes the same counters read the known size of a
plain copy kernel (``--copy-bytes`` read and written by the largest dispatches matching
``--copy-kernel``), giving HBM bytes per launch.
"""
from __future__ import annotations

import argparse
import csv
import re
import sys
from collections import OrderedDict


def _short(name: str, width: int = 48) -> str:
    return name if len(name) <= width else name[: width - 3] + "..."


def kernel_stats(path: str, top: int = 20) -> str:
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    out = [f"{'kernel':48s} {'calls':>7s} {'avg_us':>9s} {'min_us':>8s} {'max_us':>8s} "
           f"{'total_ms':>9s} {'%':>6s}"]
    for r in rows[:top]:
        out.append(f"{_short(r['Name']):48s} {int(r['Calls']):7d} {float(r['AverageNs']) / 1e3:9.2f} "
                   f"{float(r['MinNs']) / 1e3:8.2f} {float(r['MaxNs']) / 1e3:8.2f} "
                   f"{float(r['TotalDurationNs']) / 1e6:9.3f} "
                   f"{100 * float(r['TotalDurationNs']) / total:6.2f}")
    return "\n".join(out)


def counter_means(path: str, counter: str) -> "OrderedDict[str, tuple[int, float]]":
    """Kernel name -> (dispatches, mean counter value per dispatch)."""
    sums: OrderedDict[str, list] = OrderedDict()
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] != counter:
            continue
        s = sums.setdefault(r["Kernel_Name"], [0, 0.0])
        s[0] += 1
        s[1] += float(r["Counter_Value"])
    return OrderedDict((k, (n, v / n)) for k, (n, v) in sums.items())


COPY_LAST = 0  # > 0: calibrate on the last COPY_LAST copy dispatches (--copy-last)


def copy_mean(path: str, counter: str, pattern: str) -> float:
    """Mean counter value over the dispatches matching `pattern` that read within 2% of the
    largest value (the calibration copy is the largest copy in the run; copy kernels use a fixed
    grid, so the grid size does not tell copies of different sizes apart). With COPY_LAST set,
    the last COPY_LAST matching dispatches instead (for runs that also copy larger tensors
    before the calibration copies at their end)."""
    rx = re.compile(pattern)
    rows = [r for r in csv.DictReader(open(path))
            if r["Counter_Name"] == counter and rx.search(r["Kernel_Name"])]
    if not rows:
        raise SystemExit(f"no dispatch matches {pattern!r}")
    if COPY_LAST > 0:
        rows.sort(key=lambda r: int(r["Dispatch_Id"]))
        top = [float(r["Counter_Value"]) for r in rows[-COPY_LAST:]]
        return sum(top) / len(top)
    vals = [float(r["Counter_Value"]) for r in rows]
    top = [v for v in vals if v >= 0.98 * max(vals)]
    return sum(top) / len(top)


def _match(means, pattern: str):
    rx = re.compile(pattern)
    hits = [(k, v) for k, v in means.items() if rx.search(k)]
    if not hits:
        raise SystemExit(f"no dispatch matches {pattern!r}")
    n = sum(v[0] for _, v in hits)
    return n, sum(v[0] * v[1] for _, v in hits) / n


def pmc(fetch_csv: str, write_csv: str, kernels: list[str], copy_kernel: str,
        copy_bytes: int) -> str:
    fetch = counter_means(fetch_csv, "FETCH_SIZE")
    write = counter_means(write_csv, "WRITE_SIZE")
    copy_f = copy_mean(fetch_csv, "FETCH_SIZE", copy_kernel)
    copy_w = copy_mean(write_csv, "WRITE_SIZE", copy_kernel)
    f_scale = copy_bytes / (copy_f * 1024)
    w_scale = copy_bytes / (copy_w * 1024)
    out = [f"copy calibration ({copy_bytes} B read + written by /{copy_kernel}/): FETCH_SIZE "
           f"{copy_f:.1f} KiB -> x{f_scale:.3f}; WRITE_SIZE {copy_w:.1f} KiB -> x{w_scale:.3f}",
           f"{'kernel':48s} {'n':>5s} {'FETCH_KiB':>11s} {'WRITE_KiB':>11s} {'hbm_read_B':>12s} "
           f"{'hbm_write_B':>12s} {'traffic_B':>12s}"]
    for pattern in kernels:
        nf, f = _match(fetch, pattern)
        _, w = _match(write, pattern)
        rd, wr = f * 1024 * f_scale, w * 1024 * w_scale
        out.append(f"{_short(pattern):48s} {nf:5d} {f:11.1f} {w:11.1f} {rd:12.0f} {wr:12.0f} "
                   f"{rd + wr:12.0f}")
    return "\n".join(out)


def traffic_bytes(fetch_csv: str, write_csv: str, kernel: str, copy_kernel: str,
                  copy_bytes: int) -> float:
    """Calibrated HBM bytes (read + written) per dispatch of the kernels matching `kernel`."""
    fetch = counter_means(fetch_csv, "FETCH_SIZE")
    write = counter_means(write_csv, "WRITE_SIZE")
    copy_f = copy_mean(fetch_csv, "FETCH_SIZE", copy_kernel)
    copy_w = copy_mean(write_csv, "WRITE_SIZE", copy_kernel)
    _, f = _match(fetch, kernel)
    _, w = _match(write, kernel)
    return f * copy_bytes / copy_f + w * copy_bytes / copy_w


def mfma(counters_csv: str, stats_csv: str, kernels: list[str], simds: int, xcds: int) -> str:
    """MFMA evidence per kernel from one --pmc pass of SQ_INSTS_VALU_MFMA_MOPS_<type> (units of
    512 flop), SQ_VALU_MFMA_BUSY_CYCLES and GRBM_GUI_ACTIVE, plus the average durations of a
    --kernel-trace --stats run: MFMA flop per dispatch, the achieved MFMA rate over the traced
    average duration, and MFMA busy = busy cycles summed over SIMDs / (active cycles x SIMDs).
    rocprofv3 sums a counter over its hardware instances, so GRBM_GUI_ACTIVE arrives as the sum
    over the XCDs' GRBM blocks; the active cycles of the device are that sum / xcds."""
    busy = counter_means(counters_csv, "SQ_VALU_MFMA_BUSY_CYCLES")
    active = counter_means(counters_csv, "GRBM_GUI_ACTIVE")
    mops = OrderedDict()
    for kind in ("BF16", "F16", "F32", "F64"):
        for k, v in counter_means(counters_csv, f"SQ_INSTS_VALU_MFMA_MOPS_{kind}").items():
            n, prev = mops.get(k, (v[0], 0.0))
            mops[k] = (n, prev + v[1])
    stats = {r["Name"]: float(r["AverageNs"]) for r in csv.DictReader(open(stats_csv))}
    out = [f"{'kernel':48s} {'n':>5s} {'mfma_GFLOP':>11s} {'avg_us':>9s} {'TFLOP/s':>9s} "
           f"{'mfma_busy%':>10s}"]
    for pattern in kernels:
        n, m = _match(mops, pattern)
        _, b = _match(busy, pattern)
        _, a = _match(active, pattern)
        rx = re.compile(pattern)
        durs = [v for k, v in stats.items() if rx.search(k)]
        avg_us = sum(durs) / len(durs) / 1e3 if durs else float("nan")
        flop = m * 512
        out.append(f"{_short(pattern):48s} {n:5d} {flop / 1e9:11.2f} {avg_us:9.2f} "
                   f"{flop / (avg_us * 1e-6) / 1e12:9.1f} {100 * b / (a / xcds * simds):10.1f}")
    return "\n".join(out)


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m dli.rocprof_summary")
    sub = ap.add_subparsers(dest="cmd", required=True)
    st = sub.add_parser("stats")
    st.add_argument("csv")
    st.add_argument("--top", type=int, default=20)
    pm = sub.add_parser("pmc")
    pm.add_argument("--fetch", required=True)
    pm.add_argument("--write", required=True)
    pm.add_argument("--kernel", action="append", required=True)
    pm.add_argument("--copy-kernel", required=True)
    pm.add_argument("--copy-bytes", type=int, required=True)
    pm.add_argument("--copy-last", type=int, default=0,
                    help="calibrate on the last N copy dispatches (bench.py makes 3)")
    mf = sub.add_parser("mfma")
    mf.add_argument("--counters", required=True)
    mf.add_argument("--stats", required=True)
    mf.add_argument("--kernel", action="append", required=True)
    mf.add_argument("--simds", type=int, default=1024, help="SIMDs of the device (256 CUs x 4)")
    mf.add_argument("--xcds", type=int, default=8, help="GRBM instances GRBM_GUI_ACTIVE sums over")
    args = ap.parse_args(argv)
    if args.cmd == "stats":
        print(kernel_stats(args.csv, args.top))
    elif args.cmd == "mfma":
        print(mfma(args.counters, args.stats, args.kernel, args.simds, args.xcds))
    else:
        global COPY_LAST
        COPY_LAST = args.copy_last
        print(pmc(args.fetch, args.write, args.kernel, args.copy_kernel, args.copy_bytes))


if __name__ == "__main__":
    sys.exit(main())
