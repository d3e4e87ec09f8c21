"""hero_amd.traffic -- HBM bytes per kernel launch from two rocprofv3 counter
collections of the same program, one with FETCH_SIZE and one with WRITE_SIZE
(KiB per dispatch), and optionally MFMA utilisation from a third.

The raw counters are scaled by what they read for dispatches of known
traffic in the same run:
  * copy     the device-to-device copies of `python -m hero_amd.microbench
             --calibrate` (3 x 512 MiB, each byte read once and written once;
             rocclr's copyBuffer kernel), the preferred reference;
  * pack     pack_q8_kernel, one thread per Q8_0 block: reads the 34-byte GGUF
             block and writes 32 quant bytes + a 2-byte scale, so a dispatch of
             G threads moves 34 G bytes each way (dispatches of >= 1M blocks).
Both factors are printed when both kinds of dispatch are present; the copy's
is used.

    python -m hero_amd.traffic FETCH.csv[.gz] WRITE.csv[.gz] [--kernel PATTERN[,PATTERN]] [--mfma MFMA.csv] [--json out.json]
"""
from __future__ import annotations

import argparse
import csv
import gzip
import json
import re
import sys
from collections import defaultdict

COPY_BYTES = 512 << 20


def _rows(path: str):
    opener = gzip.open if path.endswith(".gz") else open
    with opener(path, "rt") as f:
        return list(csv.DictReader(f))


def _short(name: str) -> str:
    return re.sub(r"\(.*$", "", name).replace("void ", "").replace("hero::", "")


def calibration(rows) -> tuple[float, dict]:
    """measured / known bytes of the reference dispatches (copy preferred)"""
    factors = {}
    vals = [float(r["Counter_Value"]) * 1024.0 for r in rows if "copyBuffer" in r["Kernel_Name"]]
    vals = [v for v in vals if v > COPY_BYTES / 4]
    if vals:
        factors["copy"] = sum(vals) / (COPY_BYTES * len(vals))
    measured = known = 0.0
    for r in rows:
        if "pack_q8_kernel" in r["Kernel_Name"] and int(r["Grid_Size"]) >= (1 << 20):
            measured += float(r["Counter_Value"]) * 1024.0
            known += 34.0 * int(r["Grid_Size"])
    if known:
        factors["pack"] = measured / known
    if not factors:
        raise SystemExit("traffic: no known-size dispatch (a 512 MiB copy or pack_q8_kernel) to calibrate with")
    return factors.get("copy", factors.get("pack")), factors


def per_launch(rows, factor: float, pattern: str):
    by = defaultdict(list)
    pats = pattern.split(",")
    for r in rows:
        if any(p in r["Kernel_Name"] for p in pats):
            by[_short(r["Kernel_Name"])].append(float(r["Counter_Value"]) * 1024.0 / factor)
    return by


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("fetch")
    ap.add_argument("write")
    ap.add_argument("--kernel", default="gemv_q8_stream_kernel", help="comma-separated kernel name substrings")
    ap.add_argument("--mfma", default=None, help="a counter collection with SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE")
    ap.add_argument("--json", default=None)
    args = ap.parse_args(argv)
    fr, wr = _rows(args.fetch), _rows(args.write)
    (ff, ffs), (fw, fws) = calibration(fr), calibration(wr)
    fetch, write = per_launch(fr, ff, args.kernel), per_launch(wr, fw, args.kernel)
    out = {"calibration": {"FETCH_SIZE": ffs, "WRITE_SIZE": fws}, "kernels": {}}
    total_bytes = total_launches = 0.0
    for name in sorted(fetch):
        f, w = fetch[name], write.get(name, [])
        n = min(len(f), len(w)) or len(f)
        mf, mw = sum(f) / len(f), (sum(w) / len(w) if w else 0.0)
        out["kernels"][name] = {"launches": n, "fetch_bytes": mf, "write_bytes": mw, "bytes": mf + mw}
        total_bytes += (mf + mw) * len(f)
        total_launches += len(f)
    out["bytes_per_launch"] = total_bytes / max(total_launches, 1)
    cal = lambda d: ", ".join(f"{k} {v:.4f}" for k, v in d.items())  # noqa: E731
    print(f"calibration (measured / known bytes): FETCH_SIZE {cal(ffs)}; WRITE_SIZE {cal(fws)} (copy used when present)")
    print(f"{'kernel':60s} {'launches':>8s} {'fetch MB':>10s} {'write MB':>10s}")
    for name, k in out["kernels"].items():
        print(f"{name[:60]:60s} {k['launches']:8d} {k['fetch_bytes'] / 1e6:10.3f} {k['write_bytes'] / 1e6:10.3f}")
    print(f"mean HBM bytes per launch over all of them: {out['bytes_per_launch'] / 1e6:.2f} MB")
    if args.mfma:
        busy, active = defaultdict(list), defaultdict(list)
        simds = None
        for r in _rows(args.mfma):
            name = _short(r["Kernel_Name"])
            if not any(p in r["Kernel_Name"] for p in args.kernel.split(",")):
                continue
            if r["Counter_Name"] == "SQ_VALU_MFMA_BUSY_CYCLES":
                busy[name].append(float(r["Counter_Value"]))
            elif r["Counter_Name"] == "GRBM_GUI_ACTIVE":
                active[name].append(float(r["Counter_Value"]))
        out["mfma_busy_cycles"] = {k: sum(v) / len(v) for k, v in busy.items()}
        out["gui_active_cycles"] = {k: sum(v) / len(v) for k, v in active.items()}
        print(f"{'kernel':60s} {'MFMA busy cycles (sum over SIMDs)':>34s} {'GUI active cycles':>18s}")
        for name in sorted(busy):
            print(f"{name[:60]:60s} {out['mfma_busy_cycles'][name]:34.0f} {out['gui_active_cycles'].get(name, 0):18.0f}")
    if args.json:
        with open(args.json, "w") as f:
            json.dump(out, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
