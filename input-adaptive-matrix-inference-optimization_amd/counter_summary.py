#!/usr/bin/env python3
"""HBM traffic of the bucket walk from rocprofv3 counter runs.

usage: counter_summary.py --fetch FETCH.csv --write WRITE.csv --probe PROBE.json

FETCH.csv / WRITE.csv: the counter_collection CSV files of
`rocprofv3 --pmc FETCH_SIZE` and `rocprofv3 --pmc WRITE_SIZE` runs of
traffic_probe.py (--output-format csv).  PROBE.json: the JSON line that
traffic_probe.py printed.  Both counters are reported in KiB per dispatch;
each is scaled by what it reads for the probe's device-to-device copy of a
known size (the copy reads and writes copy_bytes), and the walk's average over
its last walk_launches_timed dispatches is compared with the algorithmic bytes
per launch.  Prints markdown.
"""
import argparse
import csv
import json


def per_dispatch(path, counter):
    """[(dispatch_id, kernel_name, value)] in dispatch order."""
    vals = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            if row.get("Counter_Name") != counter:
                continue
            d = int(row["Dispatch_Id"])
            name = row["Kernel_Name"]
            v = float(row["Counter_Value"])
            if d in vals:
                vals[d] = (name, vals[d][1] + v)   # one row per agent-level instance
            else:
                vals[d] = (name, v)
    return [(d, n, v) for d, (n, v) in sorted(vals.items())]


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--probe", required=True)
    args = ap.parse_args()
    probe = json.loads(open(args.probe).read().strip().splitlines()[-1])
    n_walk = int(probe["walk_launches_timed"])
    out = {}
    for key, path, counter in (("fetch", args.fetch, "FETCH_SIZE"), ("write", args.write, "WRITE_SIZE")):
        rows = per_dispatch(path, counter)
        copy = [v for d, n, v in rows if "copyBuffer" in n or "copy" in n.lower() and "walk" not in n]
        walk = [v for d, n, v in rows if "k_walk" in n][-n_walk:]
        copy_kib = max(copy) if copy else float("nan")
        factor = probe["copy_bytes"] / (copy_kib * 1024.0)
        out[key] = dict(copy_kib=copy_kib, factor=factor, walk_kib=sum(walk) / len(walk), n=len(walk))
    algo = probe["walk_bytes_per_launch"]
    fetch_b = out["fetch"]["walk_kib"] * 1024.0 * out["fetch"]["factor"]
    write_b = out["write"]["walk_kib"] * 1024.0 * out["write"]["factor"]
    print("| quantity | value |")
    print("|---|---:|")
    print(f"| copy calibration: bytes copied | {probe['copy_bytes']} |")
    print(f"| copy FETCH_SIZE (KiB) / factor | {out['fetch']['copy_kib']:.0f} / {out['fetch']['factor']:.4f} |")
    print(f"| copy WRITE_SIZE (KiB) / factor | {out['write']['copy_kib']:.0f} / {out['write']['factor']:.4f} |")
    print(f"| walk dispatches averaged | {out['fetch']['n']} |")
    print(f"| walk FETCH_SIZE per dispatch (KiB, raw) | {out['fetch']['walk_kib']:.1f} |")
    print(f"| walk WRITE_SIZE per dispatch (KiB, raw) | {out['write']['walk_kib']:.1f} |")
    print(f"| walk HBM bytes read per launch (calibrated) | {fetch_b:.0f} |")
    print(f"| walk HBM bytes written per launch (calibrated) | {write_b:.0f} |")
    print(f"| traffic_bytes_per_launch | {fetch_b + write_b:.0f} |")
    print(f"| algorithmic bytes per launch | {algo:.0f} |")
    print(f"| traffic / algorithmic | {(fetch_b + write_b) / algo:.3f} |")


if __name__ == "__main__":
    main()
