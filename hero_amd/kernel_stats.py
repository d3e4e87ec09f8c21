"""hero_amd.kernel_stats -- per-step kernel tables from a rocprofv3 kernel trace.

    rocprofv3 --kernel-trace --stats --output-format csv -d DIR -o run -- python3 bench.py ...
    python -m hero_amd.kernel_stats DIR [--marker advance_step_kernel] [--skip 10] [--take 20]
                                        [--title "..."] [--command "..."] [--out stats.txt]

The decode step ends with one launch of the marker kernel (the step-scalar
update), so the launches between its occurrence `skip` and `skip + take` are
`take` whole steps: the first table lists every kernel of those steps (launches
per step, mean duration, time per step) and the step's end-to-end time from the
marker's end timestamps. The second table is rocprofv3's own summary of the
whole run (prefill launches included). Kernel names lose their argument lists
and the hero:: namespace.
"""
from __future__ import annotations

import argparse
import csv
import glob
import gzip
import os
import re
import sys
from collections import defaultdict


def _name(n: str) -> str:
    return re.sub(r"\(.*$", "", n).replace("void ", "").replace("hero::", "").replace("(anonymous namespace)::", "")


def _open(path: str):
    return gzip.open(path, "rt") if path.endswith(".gz") else open(path)


def _find(root: str, suffix: str) -> str:
    hits = sorted(glob.glob(os.path.join(root, "**", "*" + suffix), recursive=True))
    hits += sorted(glob.glob(os.path.join(root, "**", "*" + suffix + ".gz"), recursive=True))
    if not hits:
        raise SystemExit(f"kernel_stats: no *{suffix} under {root}")
    return hits[0]


def step_table(trace_rows, marker: str, skip: int, take: int):
    rows = sorted(trace_rows, key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(rows) if marker in r["Kernel_Name"]]
    if len(marks) < skip + take + 1:
        raise SystemExit(f"kernel_stats: {len(marks)} launches of {marker}, need {skip + take + 1}")
    s, e = marks[skip], marks[skip + take]
    by = defaultdict(lambda: [0, 0.0])
    for r in rows[s + 1:e + 1]:
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        k = _name(r["Kernel_Name"])
        by[k][0] += 1
        by[k][1] += d
    step_us = (int(rows[e]["End_Timestamp"]) - int(rows[s]["End_Timestamp"])) / take / 1e3
    return by, step_us


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("dir")
    ap.add_argument("--marker", default="advance_step_kernel")
    ap.add_argument("--skip", type=int, default=10)
    ap.add_argument("--take", type=int, default=20)
    ap.add_argument("--title", default="Kernel statistics")
    ap.add_argument("--command", default="")
    ap.add_argument("--notes", default="", help="extra header lines, separated by '|'")
    ap.add_argument("--out", default=None)
    args = ap.parse_args(argv)
    trace = list(csv.DictReader(_open(_find(args.dir, "kernel_trace.csv"))))
    stats = list(csv.DictReader(_open(_find(args.dir, "kernel_stats.csv"))))
    by, step_us = step_table(trace, args.marker, args.skip, args.take)
    out = [f"# {args.title}", "#"]
    if args.command:
        out += ["# command (from the repository root, TMPDIR=/tmp):", f"#   {args.command}",
                f"#   python -m hero_amd.kernel_stats <dir> --skip {args.skip} --take {args.take}", "#"]
    for line in filter(None, args.notes.split("|")):
        out.append(f"# {line.strip()}")
    out += ["", f"## One step (steps {args.skip + 1}..{args.skip + args.take} of the trace)", ""]
    out.append("%-48s %9s %12s %12s" % ("kernel", "per step", "us / launch", "us / step"))
    for k, (c, d) in sorted(by.items(), key=lambda x: -x[1][1]):
        out.append("%-48s %9.1f %12.2f %12.1f" % (k[:48], c / args.take, d / c, d / args.take))
    out.append("%-48s %9s %12s %12.1f" % ("kernels, summed", "", "", sum(d for _, d in by.values()) / args.take))
    out.append("%-48s %9s %12s %12.1f" % ("step (end to end)", "", "", step_us))
    out += ["", "## Whole run (rocprofv3 --stats)", ""]
    out.append("%-64s %8s %9s %9s %9s %7s" % ("kernel", "calls", "avg us", "min us", "max us", "share"))
    for r in stats:
        out.append("%-64s %8s %9.2f %9.2f %9.2f %6.2f%%" % (_name(r["Name"])[:64], r["Calls"], float(r["AverageNs"]) / 1e3,
                                                            float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3, float(r["Percentage"])))
    text = "\n".join(out) + "\n"
    if args.out:
        with open(args.out, "w") as f:
            f.write(text)
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
