"""Summaries of rocprofv3 CSV output (`-f csv`) for profiles/.

  python -m measure.rocprof_summary stats <prefix>_kernel_stats.csv [--top N]
      per-kernel calls / average / min / max in microseconds, as a markdown table

  python -m measure.rocprof_summary traffic --fetch F.csv --write W.csv \\
          --kernel <symbol substring> --name <profile name> [--out traffic.json]
      HBM bytes per dispatch of one kernel from a FETCH_SIZE pass and a
      WRITE_SIZE pass (<prefix>_counter_collection.csv, values in KiB), each
      scaled by what the same counter reads for the calibration copy that
      `bench.py --calibrate-copy` runs first: ckv_copy_blocks of 1024 pages of
      32 KiB for keys and values, 64 MiB read and 64 MiB written.

  python -m measure.rocprof_summary counters <prefix>_counter_collection.csv \
          --kernel <symbol substring>
      every counter of a --pmc pass, mean per dispatch of one kernel (as the
      counters report it: summed over the XCDs), as a markdown table
"""
from __future__ import annotations

import argparse
import csv
import json
import re
import sys

CALIBRATION_KERNEL = "copy_blocks_kernel"
CALIBRATION_BYTES = 64 << 20  # read, and again written


def short_name(symbol: str) -> str:
    """A kernel symbol without its argument list, e.g. `decode_wg_kernel<2, false, ...>`."""
    name = symbol[5:] if symbol.startswith("void ") else symbol
    name = name.replace("(anonymous namespace)::", "")
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            name = name[:i]
            break
    return re.sub(r"^ckv::", "", name)


def kernel_stats(path: str) -> list[dict]:
    rows = []
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            rows.append({"name": short_name(r["Name"]), "calls": int(r["Calls"]),
                         "avg_us": float(r["AverageNs"]) / 1e3,
                         "min_us": float(r["MinNs"]) / 1e3, "max_us": float(r["MaxNs"]) / 1e3,
                         "percent": float(r["Percentage"])})
    return rows


def stats_markdown(rows: list[dict], top: int) -> str:
    out = ["| kernel | calls | avg | min | max | % time |", "|---|---:|---:|---:|---:|---:|"]
    for r in rows[:top]:
        name = r["name"] if len(r["name"]) < 90 else r["name"][:87] + "..."
        out.append(f"| `{name}` | {r['calls']} | {r['avg_us']:.2f} | {r['min_us']:.2f} | "
                   f"{r['max_us']:.2f} | {r['percent']:.2f} |")
    return "\n".join(out)


def counter_means(path: str, counter: str) -> dict[str, tuple[str, int, float]]:
    """Per kernel symbol: (symbol, dispatches, mean counter value per dispatch)."""
    sums: dict[str, list] = {}
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            if r["Counter_Name"] != counter:
                continue
            entry = sums.setdefault(r["Kernel_Name"], [set(), 0.0])
            entry[0].add(r["Dispatch_Id"])
            entry[1] += float(r["Counter_Value"])
    return {k: (k, len(v[0]), v[1] / len(v[0])) for k, v in sums.items()}


def pick(means: dict, fragment: str):
    hits = [v for k, v in means.items() if fragment in k]
    if len(hits) != 1:
        raise SystemExit(f"{len(hits)} kernels match {fragment!r}: "
                         + ", ".join(short_name(h[0]) for h in hits))
    return hits[0]


def traffic(fetch_csv: str, write_csv: str, kernel: str) -> dict:
    fetch = counter_means(fetch_csv, "FETCH_SIZE")
    write = counter_means(write_csv, "WRITE_SIZE")
    cal_f, cal_w = pick(fetch, CALIBRATION_KERNEL), pick(write, CALIBRATION_KERNEL)
    k_f, k_w = pick(fetch, kernel), pick(write, kernel)
    fetch_scale = CALIBRATION_BYTES / 1024 / cal_f[2]
    write_scale = CALIBRATION_BYTES / 1024 / cal_w[2]
    read_b = int(round(k_f[2] * 1024 * fetch_scale))
    write_b = int(round(k_w[2] * 1024 * write_scale))
    return {
        "kernel_symbol": k_f[0],
        "dispatches": k_f[1],
        "fetch_size_kib_raw": k_f[2],
        "write_size_kib_raw": k_w[2],
        "fetch_scale": round(fetch_scale, 4),
        "write_scale": round(write_scale, 4),
        "hbm_bytes_per_launch": read_b + write_b,
        "hbm_read_bytes_per_launch": read_b,
        "hbm_write_bytes_per_launch": write_b,
        "calibration": {"kernel_symbol": cal_f[0], "bytes_read": CALIBRATION_BYTES,
                        "bytes_written": CALIBRATION_BYTES,
                        "fetch_size_kib_raw": cal_f[2], "write_size_kib_raw": cal_w[2]},
    }


def counters_markdown(path: str, kernel: str) -> str:
    names = []
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            if r["Counter_Name"] not in names:
                names.append(r["Counter_Name"])
    out = ["| counter | per dispatch |", "|---|---:|"]
    symbol, dispatches = None, 0
    for name in names:
        symbol, dispatches, mean = pick(counter_means(path, name), kernel)
        out.append(f"| {name} | {mean:,.0f} |")
    out.insert(0, f"`{short_name(symbol)}`, mean over {dispatches} dispatches\n")
    return "\n".join(out)


def main(argv=None) -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--top", type=int, default=8)
    c = sub.add_parser("counters")
    c.add_argument("csv")
    c.add_argument("--kernel", required=True, help="substring of the kernel symbol")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--kernel", required=True, help="substring of the kernel symbol")
    t.add_argument("--name", required=True, help="the profile name bench.py looks up")
    t.add_argument("--out")
    t.add_argument("--command", action="append", default=[],
                   help="the rocprofv3 commands that made the CSVs, for the record")
    args = ap.parse_args(argv)
    if args.cmd == "stats":
        print(stats_markdown(kernel_stats(args.csv), args.top))
        return
    if args.cmd == "counters":
        print(counters_markdown(args.csv, args.kernel))
        return
    entry = traffic(args.fetch, args.write, args.kernel)
    doc = {"kernels": {args.name: entry}, "commands": args.command}
    text = json.dumps(doc, indent=1)
    if args.out:
        with open(args.out, "w") as fh:
            fh.write(text + "\n")
    print(text)


if __name__ == "__main__":
    main(sys.argv[1:])
