#!/usr/bin/env python3
"""Summaries of rocprofv3 CSV output for the measurement notes.

  rocprof_summary.py stats <prefix>_kernel_stats.csv [--top N]
      markdown table of the kernel-trace statistics (calls, total ms, average us)
  rocprof_summary.py traffic --fetch F.csv --write W.csv --cal-fetch CF.csv --cal-write CW.csv
                             --kernel SUBSTRING [--cal-kernel SUBSTRING] [--cal-bytes N] [--per-dispatch]
      HBM bytes per dispatch of the kernels whose name contains SUBSTRING (or one
      of its alternatives separated by '|'), from a
      FETCH_SIZE run and a WRITE_SIZE run (counter_collection.csv of each), each
      counter scaled by what it reads for a plain copy of known size (the
      calibration runs: --cal-kernel, default the elementwise add of
      `bench.py --workload copy`, which reads and writes --cal-bytes, default 1 GiB)
  rocprof_summary.py shapes <prefix>_kernel_trace.csv [--top N]
      markdown table per kernel and launch shape (grid size in work-items along
      x): launches and average duration, largest total first
  rocprof_summary.py counters C.csv --kernel SUBSTRING [--per-wave]
      one row per dispatch of those kernels: its duration in the counter run and
      every counter of the run (divided by SQ_WAVES with --per-wave)

Counters are in KiB per dispatch as rocprofv3 reports them.
"""
import argparse
import csv
import sys


def _rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def stats(path, top):
    rows = _rows(path)
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    print("| Kernel | Calls | Total ms | Avg us | % |")
    print("|---|---|---|---|---|")
    for r in rows[:top]:
        name = r["Name"] if len(r["Name"]) < 100 else r["Name"][:97] + "..."
        print(f"| `{name}` | {r['Calls']} | {float(r['TotalDurationNs']) / 1e6:.3f} | "
              f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")


def shapes(path, top):
    agg = {}
    for r in _rows(path):
        name = r["Kernel_Name"]
        name = name[5:] if name.startswith("void ") else name
        name = name.split("(")[0] if "mpcx::" in name else name[:60]
        key = (name.replace("mpcx::", ""), int(r["Grid_Size_X"]))
        n, t = agg.get(key, (0, 0.0))
        agg[key] = (n + 1, t + (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    print("| Kernel | grid x | launches | avg us |")
    print("|---|---|---|---|")
    for (name, gx), (n, t) in sorted(agg.items(), key=lambda kv: -kv[1][1])[:top]:
        print(f"| `{name}` | {gx} | {n} | {t / n:.1f} |")


def _match(name, sub):
    """name contains SUB, or one of the alternatives of SUB separated by '|'."""
    return any(s and s in name for s in sub.split("|"))


def _values(path, counter, sub):
    out = []
    for r in _rows(path):
        if r["Counter_Name"] == counter and _match(r["Kernel_Name"], sub):
            out.append((int(r["Dispatch_Id"]), float(r["Counter_Value"]), r["Kernel_Name"]))
    out.sort()
    return out


def _calibration(path, counter, sub):
    vals = _values(path, counter, sub)
    if not vals:
        sys.exit(f"{path}: no {counter} row for a kernel containing {sub!r}")
    return max(v for _, v, _ in vals)


def traffic(a):
    cf = _calibration(a.cal_fetch, "FETCH_SIZE", a.cal_kernel)
    cw = _calibration(a.cal_write, "WRITE_SIZE", a.cal_kernel)
    sf = a.cal_bytes / (cf * 1024.0)
    sw = a.cal_bytes / (cw * 1024.0)
    fetch = _values(a.fetch, "FETCH_SIZE", a.kernel)
    write = _values(a.write, "WRITE_SIZE", a.kernel)
    if not fetch or len(fetch) != len(write):
        sys.exit(f"dispatch counts differ or are empty: {len(fetch)} FETCH_SIZE, {len(write)} WRITE_SIZE rows")
    fb = [v * 1024.0 * sf for _, v, _ in fetch]
    wb = [v * 1024.0 * sw for _, v, _ in write]
    n = len(fb)
    print(f"calibration: {a.cal_kernel!r} FETCH_SIZE {cf:.1f} KiB, WRITE_SIZE {cw:.1f} KiB for "
          f"{a.cal_bytes} bytes: scale x{sf:.4f} (fetch), x{sw:.4f} (write)")
    print(f"{n} dispatches of kernels containing {a.kernel!r}")
    print(f"fetch total {sum(fb) / 1e9:.4f} GB, write total {sum(wb) / 1e9:.4f} GB")
    print(f"mean per dispatch: fetch {sum(fb) / n:.0f} B, write {sum(wb) / n:.0f} B, "
          f"traffic {(sum(fb) + sum(wb)) / n:.0f} B")
    if a.per_dispatch:
        print("| # | fetch MB | write MB |")
        print("|---|---|---|")
        for i, (f, w) in enumerate(zip(fb, wb)):
            print(f"| {i} | {f / 1e6:.2f} | {w / 1e6:.3f} |")


def counters(a):
    rows = [r for r in _rows(a.csv) if _match(r["Kernel_Name"], a.kernel)]
    if not rows:
        sys.exit(f"{a.csv}: no dispatch of a kernel containing {a.kernel!r}")
    names = sorted({r["Counter_Name"] for r in rows})
    by = {}
    for r in rows:
        d = by.setdefault(int(r["Dispatch_Id"]), {"us": (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3})
        d[r["Counter_Name"]] = float(r["Counter_Value"])
    shown = [n for n in names if not (a.per_wave and n == "SQ_WAVES")]
    unit = " / wave" if a.per_wave else ""
    print("| # | us | " + " | ".join(f"{n}{unit}" for n in shown) + " |")
    print("|---" * (len(shown) + 2) + "|")
    for i, k in enumerate(sorted(by)):
        d = by[k]
        w = d.get("SQ_WAVES", 1.0) if a.per_wave else 1.0
        vals = " | ".join(f"{d.get(n, 0.0) / w:.0f}" for n in shown)
        print(f"| {i} | {d['us']:.1f} | {vals} |")


def main():
    ap = argparse.ArgumentParser()
    sp = ap.add_subparsers(dest="cmd", required=True)
    s = sp.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--top", type=int, default=15)
    t = sp.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--cal-fetch", required=True)
    t.add_argument("--cal-write", required=True)
    t.add_argument("--kernel", required=True)
    t.add_argument("--cal-kernel", default="CUDAFunctorOnSelf_add")
    t.add_argument("--cal-bytes", type=float, default=float(1 << 30))
    t.add_argument("--per-dispatch", action="store_true")
    c = sp.add_parser("counters")
    c.add_argument("csv")
    c.add_argument("--kernel", required=True)
    c.add_argument("--per-wave", action="store_true")
    h = sp.add_parser("shapes")
    h.add_argument("csv")
    h.add_argument("--top", type=int, default=15)
    a = ap.parse_args()
    if a.cmd == "stats":
        stats(a.csv, a.top)
    elif a.cmd == "shapes":
        shapes(a.csv, a.top)
    elif a.cmd == "counters":
        counters(a)
    else:
        traffic(a)


if __name__ == "__main__":
    main()
