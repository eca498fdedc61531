#!/usr/bin/env python3
"""Summarise rocprofv3 CSV output of bench.py into a short markdown report.

Inputs (directories written by `rocprofv3 -f csv -d DIR -o NAME ...`, any NAME):
  --trace DIR   a --kernel-trace --stats run  (bench_kernel_stats.csv,
                bench_kernel_trace.csv)
  --fetch DIR   a --pmc FETCH_SIZE run         (bench_counter_collection.csv)
  --write DIR   a --pmc WRITE_SIZE run         (bench_counter_collection.csv)
  --copy-bytes N  bytes the calibration copy kernel (stream_copy_b128) read
                and wrote in those runs (bench.py --copy-calibration MIB)
  --split-after NAME  report a kernel's dispatches that directly follow a
                dispatch of NAME on the same queue as a row of their own
                ("kernel (after NAME)"), e.g. the launches of bench.py
                --scrub-only that follow its stream_read_b128 scrub

HBM traffic per dispatch = FETCH_SIZE * (N / FETCH_SIZE of the copy kernel)
+ WRITE_SIZE * (N / WRITE_SIZE of the copy kernel): each counter is scaled by
what it reads for a copy of known size.  Kernels are grouped by name and grid
size (one launch shape = one row).

Writes the markdown report to stdout and, with --json PATH, the per-kernel
traffic figures as JSON, each with the digest of the kernel's machine code in
the code objects of this tree (build.kernel_digest): a figure describes a
build whose kernel has that digest.
"""
from __future__ import annotations

import argparse
import csv
import json
import statistics
from collections import defaultdict
from pathlib import Path


def _one(d: Path, suffix: str) -> Path:
    """The one `<NAME>_<suffix>` file rocprofv3 wrote into d."""
    found = sorted(d.glob(f"*_{suffix}"))
    if len(found) != 1:
        raise SystemExit(f"expected one *_{suffix} in {d}, found {len(found)}")
    return found[0]


def _rows(path: Path):
    with open(path, newline="") as f:
        yield from csv.DictReader(f)


def kernel_durations(trace_dir: Path, split_after: str | None = None) -> dict:
    out = defaultdict(list)
    rows = sorted(_rows(_one(trace_dir, "kernel_trace.csv")),
                  key=lambda r: (r["Queue_Id"], int(r["Start_Timestamp"])))
    prev = {}
    for r in rows:
        name = r["Kernel_Name"]
        if split_after and prev.get(r["Queue_Id"]) == split_after and name != split_after:
            name = f"{name} (after {split_after})"
        prev[r["Queue_Id"]] = r["Kernel_Name"]
        key = (name, int(r["Grid_Size_X"]))
        out[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return out


def counter_values(pmc_dir: Path, counter: str) -> dict:
    out = defaultdict(list)
    for r in _rows(_one(pmc_dir, "counter_collection.csv")):
        if r["Counter_Name"] != counter:
            continue
        out[(r["Kernel_Name"], int(r["Grid_Size"]))].append(float(r["Counter_Value"]))
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--trace", type=Path, required=True)
    ap.add_argument("--fetch", type=Path)
    ap.add_argument("--write", type=Path)
    ap.add_argument("--copy-bytes", type=int, default=0)
    ap.add_argument("--kernels", nargs="*", default=None, help="only these kernel names")
    ap.add_argument("--split-after", default=None, metavar="NAME")
    ap.add_argument("--json", type=Path)
    args = ap.parse_args()

    durs = kernel_durations(args.trace, args.split_after)
    fetch = counter_values(args.fetch, "FETCH_SIZE") if args.fetch else {}
    write = counter_values(args.write, "WRITE_SIZE") if args.write else {}

    def scale(values: dict) -> float | None:
        # the calibration copy: the stream_copy_b128 launches of the largest grid
        # (bench.py also launches it empty, one workgroup, to time dispatches)
        grids = [g for (name, g) in values if name == "stream_copy_b128"]
        if not grids or not args.copy_bytes:
            return None
        copy = values[("stream_copy_b128", max(grids))]
        return args.copy_bytes / 1024.0 / statistics.mean(copy)

    fs, ws = scale(fetch), scale(write)
    import build as B  # the package directory is this script's

    digest = B.source_digest()

    def code_digest(name: str) -> str | None:
        for co in (B.CODE_OBJECT, B.DECODE_OBJECT, B.PREFILL_OBJECT):
            if co.exists() and (d := B.kernel_digest(name, co)) is not None:
                return d
        return None

    print("| kernel | grid (threads) | dispatches | mean us | median us | min us |"
          " FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes / dispatch |")
    print("|---|---|---|---|---|---|---|---|---|")
    report = {"source_digest": digest, "fetch_scale": fs, "write_scale": ws, "kernels": []}
    for key in sorted(durs, key=lambda k: -sum(durs[k])):
        name, grid = key
        if args.kernels and name.split(" (after ")[0] not in args.kernels:
            continue
        d = durs[key]
        f = statistics.mean(fetch[key]) if fetch.get(key) else None
        w = statistics.mean(write[key]) if write.get(key) else None
        traffic = None
        if f is not None and w is not None and fs and ws:
            traffic = round(f * 1024 * fs + w * 1024 * ws)
        print(f"| {name} | {grid} | {len(d)} | {statistics.mean(d):.3f} | {statistics.median(d):.3f} |"
              f" {min(d):.3f} | {'' if f is None else f'{f:.1f}'} | {'' if w is None else f'{w:.1f}'} |"
              f" {'' if traffic is None else traffic} |")
        report["kernels"].append({"name": name, "grid": grid, "dispatches": len(d),
                                  "mean_us": statistics.mean(d),
                                  "median_us": statistics.median(d), "fetch_kib": f,
                                  "write_kib": w, "hbm_bytes": traffic,
                                  "code_digest": code_digest(name.split(" (after ")[0])})
    print()
    print(f"FETCH_SIZE scale (copy kernel): {fs}; WRITE_SIZE scale: {ws}")
    print(f"Sources of the q8gemv code object (csrc/q8gemv_kernels.hip, csrc/q8_device.h) "
          f"sha256: {digest}")
    if args.json:
        args.json.write_text(json.dumps(report, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
