#!/usr/bin/env python3
"""Summaries of rocprofv3 CSV output for the decode path.

  profsum.py stats DIR
      per-kernel table of DIR/*_kernel_stats.csv (--kernel-trace --stats)
  profsum.py pmc DIR [DIR ...] [--kernels REGEX]
      per-kernel average of every counter of --pmc runs (one column per counter)
  profsum.py traffic FETCH_DIR WRITE_DIR --copy-bytes N [--json OUT]
      per-kernel HBM traffic from two --pmc runs (FETCH_SIZE, WRITE_SIZE; KiB
      per dispatch), each scaled so that the library's plain copy kernel
      (k_copy_v4, N bytes read and N bytes written) reads exactly N bytes

Output is markdown on stdout.
"""
import argparse
import collections
import csv
import glob
import json
import os
import re
import sys

COPY_KERNEL = "k_copy_v4"
# decode GEMV call sites at the 8B shape: template <MODE, KCH, R, PRO, NS>
# (PRO 2: the kernel normalizes its own input; PRO 1: it quantizes its input)
GEMV_SITES = {
    "k_gemv_dec<0, 4, 4, 2, 2>": "gemv_qkv",
    "k_gemv_dec<1, 4, 2, 1, 1>": "gemv_o",
    "k_gemv_dec<2, 4, 6, 2, 1>": "gemv_gate_up",
    "k_gemv_dec<1, 14, 2, 0, 2>": "gemv_down",
    "k_gemv_dec<3, 4, 2, 0, 1>": "gemv_head",
    # warp-specialized prologue GEMVs (k_gemv_ws<MODE, KCH, PRO, NS, PW, RWV>)
    "k_gemv_ws<0, 4, 2, 3, 8, 8>": "gemv_qkv",
    "k_gemv_ws<1, 4, 1, 2, 4, 8>": "gemv_o",
    "k_gemv_ws<2, 4, 2, 3, 4, 8>": "gemv_gate_up",
}


def short_name(s):
    s = s.replace("(anonymous namespace)::", "")
    s = re.sub(r"^void ", "", s)
    return s.split("(")[0]


def one(pattern):
    hits = glob.glob(pattern)
    if len(hits) != 1:
        sys.exit(f"profsum: expected one file matching {pattern}, found {len(hits)}")
    return hits[0]


def stats(d, top):
    rows = list(csv.DictReader(open(one(os.path.join(d, "*kernel_stats.csv")))))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    print("| kernel | calls | total ms | avg us | min us | max us | % |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for r in rows[:top]:
        print(f"| `{short_name(r['Name'])}` | {r['Calls']} | {float(r['TotalDurationNs']) / 1e6:.2f} | "
              f"{float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
              f"{float(r['MaxNs']) / 1e3:.2f} | {100 * float(r['TotalDurationNs']) / total:.2f} |")


def per_kernel(d, counter):
    agg = collections.defaultdict(list)
    for r in csv.DictReader(open(one(os.path.join(d, "*counter_collection.csv")))):
        if r["Counter_Name"] != counter:
            continue
        agg[short_name(r["Kernel_Name"])].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in agg.items()}, {k: len(v) for k, v in agg.items()}


def traffic(fd, wd, copy_bytes, out_json):
    fetch, nf = per_kernel(fd, "FETCH_SIZE")
    write, _ = per_kernel(wd, "WRITE_SIZE")
    if COPY_KERNEL not in fetch or COPY_KERNEL not in write:
        sys.exit(f"profsum: {COPY_KERNEL} missing from the counter runs")
    kib = copy_bytes / 1024.0
    f_scale, w_scale = kib / fetch[COPY_KERNEL], kib / write[COPY_KERNEL]
    print(f"Copy reference `{COPY_KERNEL}` of {copy_bytes} B: FETCH_SIZE {fetch[COPY_KERNEL]:.1f} KiB, "
          f"WRITE_SIZE {write[COPY_KERNEL]:.1f} KiB -> scale factors fetch x{f_scale:.4f}, write x{w_scale:.4f}\n")
    print("| kernel | site | dispatches | read MB | written MB | HBM MB per dispatch |")
    print("|---|---|---:|---:|---:|---:|")
    sites = {}
    for k in sorted(fetch, key=lambda k: -fetch[k]):
        if k == COPY_KERNEL:
            continue
        rd = fetch[k] * f_scale * 1024
        wr = write.get(k, 0.0) * w_scale * 1024
        site = GEMV_SITES.get(k, "")
        if site:
            sites[site] = rd + wr
        if rd + wr > 1e5 or site:
            print(f"| `{k}` | {site} | {nf[k]} | {rd / 1e6:.3f} | {wr / 1e6:.3f} | {(rd + wr) / 1e6:.3f} |")
    if out_json:
        with open(out_json, "w") as f:
            json.dump({"fetch_scale": f_scale, "write_scale": w_scale, "bytes_per_dispatch": sites}, f, indent=1)
            f.write("\n")


def pmc(dirs, kernels):
    """Per-kernel mean of each counter over its dispatches, across --pmc runs."""
    vals = collections.defaultdict(lambda: collections.defaultdict(list))
    order = []
    for d in dirs:
        for r in csv.DictReader(open(one(os.path.join(d, "*counter_collection.csv")))):
            k = short_name(r["Kernel_Name"])
            if kernels and not re.search(kernels, k):
                continue
            if k not in vals:
                order.append(k)
            vals[k][r["Counter_Name"]].append(float(r["Counter_Value"]))
    names = sorted({c for k in vals for c in vals[k]})
    print("| kernel | dispatches | " + " | ".join(names) + " |")
    print("|---|---:|" + "---:|" * len(names))
    for k in order:
        n = max(len(v) for v in vals[k].values())
        cells = [f"{sum(vals[k][c]) / len(vals[k][c]):.4g}" if vals[k][c] else "" for c in names]
        print(f"| `{k}` | {n} | " + " | ".join(cells) + " |")


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--top", type=int, default=20)
    t = sub.add_parser("traffic")
    t.add_argument("fetch_dir")
    t.add_argument("write_dir")
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--json")
    p = sub.add_parser("pmc")
    p.add_argument("dirs", nargs="+")
    p.add_argument("--kernels", default=None)
    a = ap.parse_args()
    if a.cmd == "stats":
        stats(a.dir, a.top)
    elif a.cmd == "pmc":
        pmc(a.dirs, a.kernels)
    else:
        traffic(a.fetch_dir, a.write_dir, a.copy_bytes, a.json)


if __name__ == "__main__":
    main()
