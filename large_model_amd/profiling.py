"""Summaries of rocprofv3 output for the layer's kernels (text for the profiles folder).

    python -m large_model_amd.profiling stats DIR [--command "..."]
        per-kernel launches / average / min / max duration from rocprofv3 --kernel-trace --stats
        CSV output under DIR (its *kernel_stats.csv), short names for the library's kernels.

    python -m large_model_amd.profiling counters DIR [DIR ...] [--command "..."]
        per kernel, the mean per dispatch of every counter in the rocprofv3 --pmc CSV output
        under the DIRs (a dispatch's rows summed over the device), one pass per DIR.

    python -m large_model_amd.profiling traffic --kernel gateup --fetch DIR --write DIR
        --copy-fetch DIR --copy-write DIR --copy-bytes N [--algorithmic-bytes B] [--command "..."]
        HBM bytes per dispatch of one kernel from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs
        (KiB per dispatch), each scaled by what the same counter reads for the plain copy kernel
        moving a known N bytes (N read, N written). Prints `hbm_bytes_per_launch = ...`.
"""
from __future__ import annotations

import argparse
import csv
import glob
import os
import statistics
import sys

SHORT = (
    ("route_small_kernel", "route"), ("route_big_kernel", "route"), ("select_kernel", "select"),
    ("dispatch_kernel", "dispatch"), ("gateup_kernel", "gateup"), ("down_exact_kernel", "down"),
    ("down_t1_kernel", "down"), ("down_small_kernel", "down"), ("act_quant_kernel", "actq"), ("swiglu_kernel", "swiglu"),
    ("route_exact_kernel", "route"), ("exact_rows_kernel", "rows_f32"),
    ("combine_kernel", "combine"), ("copy_kernel", "copy"), ("dense_kernel", "dense"),
    ("dense_oct_kernel", "dense"), ("dense_tok_kernel", "dense"), ("dense_quant_kernel", "dquant"),
    ("gateup_mfma_kernel", "gateup"), ("down_mfma_kernel", "down"), ("rmsnorm_kernel", "rmsnorm"),
    ("add_rows_kernel", "add"),
)


def short_name(kernel: str) -> str:
    if "tile_rows_kernel" in kernel:       # last template argument: 1 = gate/up rows, 0 = down rows
        return "gateup" if kernel.replace(" ", "").split(">")[0].endswith(",1") else "down"
    for key, name in SHORT:
        if key in kernel:
            return name
    return kernel.split("(")[0][:48]


def _find(d: str, suffix: str) -> str:
    hits = sorted(glob.glob(os.path.join(d, "**", "*" + suffix), recursive=True))
    if not hits:
        sys.exit(f"no *{suffix} under {d}")
    return hits[0]


def stats(d: str) -> list[str]:
    rows = list(csv.DictReader(open(_find(d, "kernel_stats.csv"))))
    out = [f"{'kernel':10s} {'launches':>9s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'share':>7s}  full name"]
    for r in rows:
        name = r["Name"]
        out.append(f"{short_name(name):10s} {int(r['Calls']):9d} {float(r['AverageNs']) / 1e3:9.3f} "
                   f"{float(r['MinNs']) / 1e3:9.3f} {float(r['MaxNs']) / 1e3:9.3f} {float(r['Percentage']):6.2f}%  "
                   f"{name[:90]}")
    return out


def counter_values(d: str, counter: str, kernel: str) -> list[float]:
    vals = []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] == counter and short_name(r["Kernel_Name"]) == kernel:
                vals.append(float(r["Counter_Value"]))
    if not vals:
        sys.exit(f"no {counter} values for {kernel} under {d}")
    return vals


def counters(dirs: list[str]) -> list[str]:
    per_kernel: dict[str, dict[str, list[float]]] = {}
    for d in dirs:
        files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if not files:
            sys.exit(f"no *counter_collection.csv under {d}")
        for f in files:
            per_dispatch: dict[tuple[str, str], dict[str, float]] = {}
            for r in csv.DictReader(open(f)):
                key = (r["Kernel_Name"], r["Dispatch_Id"])
                c = per_dispatch.setdefault(key, {})
                c[r["Counter_Name"]] = c.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            for (k, _), cs in per_dispatch.items():
                for c, v in cs.items():
                    per_kernel.setdefault(k, {}).setdefault(c, []).append(v)
    out = []
    for k in sorted(per_kernel):
        cs = per_kernel[k]
        out.append(f"{k.split('(')[0]}  [{max(len(v) for v in cs.values())} dispatches]")
        for c in sorted(cs):
            out.append(f"   {c:32s} {sum(cs[c]) / len(cs[c]):18.0f}")
    return out


def traffic(a) -> list[str]:
    f = counter_values(a.fetch, "FETCH_SIZE", a.kernel)
    w = counter_values(a.write, "WRITE_SIZE", a.kernel)
    cf = counter_values(a.copy_fetch, "FETCH_SIZE", "copy")
    cw = counter_values(a.copy_write, "WRITE_SIZE", "copy")
    kib = a.copy_bytes / 1024.0
    sf, sw = kib / statistics.median(cf), kib / statistics.median(cw)
    fb = statistics.median(f) * sf * 1024.0
    wb = statistics.median(w) * sw * 1024.0
    out = [
        f"kernel = {a.kernel}",
        f"dispatches_fetch = {len(f)}",
        f"dispatches_write = {len(w)}",
        f"fetch_kib_median_raw = {statistics.median(f):.1f}",
        f"write_kib_median_raw = {statistics.median(w):.1f}",
        f"copy_bytes = {a.copy_bytes}",
        f"copy_fetch_kib_raw = {statistics.median(cf):.1f}",
        f"copy_write_kib_raw = {statistics.median(cw):.1f}",
        f"fetch_scale = {sf:.4f}",
        f"write_scale = {sw:.4f}",
        f"hbm_fetch_bytes_per_launch = {fb:.0f}",
        f"hbm_write_bytes_per_launch = {wb:.0f}",
        f"hbm_bytes_per_launch = {fb + wb:.0f}",
    ]
    if a.algorithmic_bytes:
        out.append(f"algorithmic_bytes_per_launch = {a.algorithmic_bytes}")
        out.append(f"traffic_over_algorithmic = {(fb + wb) / a.algorithmic_bytes:.4f}")
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="mode", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--command", default="")
    c = sub.add_parser("counters")
    c.add_argument("dirs", nargs="+")
    c.add_argument("--command", default="")
    t = sub.add_parser("traffic")
    for k in ("fetch", "write", "copy_fetch", "copy_write"):
        t.add_argument("--" + k.replace("_", "-"), dest=k, required=True)
    t.add_argument("--kernel", default="gateup")
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--algorithmic-bytes", type=int, default=0)
    t.add_argument("--command", default="")
    a = ap.parse_args()
    if a.mode == "stats":
        lines = stats(a.dir)
    elif a.mode == "counters":
        lines = counters(a.dirs)
    else:
        lines = traffic(a)
    if a.command:
        print("# " + a.command.replace("\n", "\n# "))
    print("\n".join(lines))


if __name__ == "__main__":
    main()
