"""hero_amd.traffic -- HBM bytes per kernel launch from two rocprofv3 counter
collections of the same program, one with FETCH_SIZE and one with WRITE_SIZE
(KiB per dispatch).

The raw counters are scaled by what they read for a kernel of known traffic in
the same run: pack_q8_kernel, one thread per Q8_0 block, reads the 34-byte
GGUF block and writes 32 quant bytes + a 2-byte scale, so a dispatch of G
threads moves 34 G bytes each way (G is the block count rounded up to the
workgroup; only dispatches of at least 1M blocks are used).

    python -m hero_amd.traffic FETCH.csv[.gz] WRITE.csv[.gz] [--kernel gemv_q8_stream_kernel] [--json out.json]
"""
from __future__ import annotations

import argparse
import csv
import gzip
import json
import re
import sys
from collections import defaultdict


def _rows(path: str):
    opener = gzip.open if path.endswith(".gz") else open
    with opener(path, "rt") as f:
        return list(csv.DictReader(f))


def _short(name: str) -> str:
    return re.sub(r"\(.*$", "", name).replace("void ", "").replace("hero::", "")


def calibration(rows) -> float:
    """measured / known bytes of the large pack_q8_kernel dispatches"""
    measured = known = 0.0
    for r in rows:
        if "pack_q8_kernel" in r["Kernel_Name"] and int(r["Grid_Size"]) >= (1 << 20):
            measured += float(r["Counter_Value"]) * 1024.0
            known += 34.0 * int(r["Grid_Size"])
    if known == 0:
        raise SystemExit("traffic: no pack_q8_kernel dispatch of >= 1M blocks to calibrate with")
    return measured / known


def per_launch(rows, factor: float, pattern: str):
    by = defaultdict(list)
    for r in rows:
        if pattern in r["Kernel_Name"]:
            by[_short(r["Kernel_Name"])].append(float(r["Counter_Value"]) * 1024.0 / factor)
    return by


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("fetch")
    ap.add_argument("write")
    ap.add_argument("--kernel", default="gemv_q8_stream_kernel")
    ap.add_argument("--json", default=None)
    args = ap.parse_args(argv)
    fr, wr = _rows(args.fetch), _rows(args.write)
    ff, fw = calibration(fr), calibration(wr)
    fetch, write = per_launch(fr, ff, args.kernel), per_launch(wr, fw, args.kernel)
    out = {"calibration": {"FETCH_SIZE": ff, "WRITE_SIZE": fw}, "kernels": {}}
    total_bytes = total_launches = 0.0
    for name in sorted(fetch):
        f, w = fetch[name], write.get(name, [])
        n = min(len(f), len(w)) or len(f)
        mf, mw = sum(f) / len(f), (sum(w) / len(w) if w else 0.0)
        out["kernels"][name] = {"launches": n, "fetch_bytes": mf, "write_bytes": mw, "bytes": mf + mw}
        total_bytes += (mf + mw) * len(f)
        total_launches += len(f)
    out["bytes_per_launch"] = total_bytes / max(total_launches, 1)
    print(f"calibration (measured / known bytes of pack_q8_kernel): FETCH_SIZE {ff:.4f}, WRITE_SIZE {fw:.4f}")
    print(f"{'kernel':44s} {'launches':>8s} {'fetch MB':>10s} {'write MB':>10s}")
    for name, k in out["kernels"].items():
        print(f"{name:44s} {k['launches']:8d} {k['fetch_bytes'] / 1e6:10.2f} {k['write_bytes'] / 1e6:10.3f}")
    print(f"mean HBM bytes per launch over all of them: {out['bytes_per_launch'] / 1e6:.2f} MB")
    if args.json:
        with open(args.json, "w") as f:
            json.dump(out, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
