#!/usr/bin/env python3
"""Summarise a rocprofv3 kernel trace (results .db written by
`rocprofv3 --kernel-trace --stats -d DIR -o NAME -- ...`) as markdown:
per-kernel totals, and per-launch-shape averages of the bucket walk,
cutoff and reduce kernels (the grid size tells the matrix groups apart).

usage: profile_summary.py RESULTS.db [--steps N]
  --steps N   divide totals by N decode steps to report per-token time
"""
import argparse
import sqlite3


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("db")
    ap.add_argument("--steps", type=int, default=0)
    args = ap.parse_args()
    c = sqlite3.connect(args.db)
    rows = list(c.execute(
        "select name, count(*), sum(duration), avg(duration), min(duration), max(duration) "
        "from kernels group by name order by sum(duration) desc"))
    total = sum(r[2] for r in rows)
    print("| kernel | calls | total ms | avg us | min us | max us | % |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for name, n, tot, avg, mn, mx in rows:
        print(f"| `{name[:70]}` | {n} | {tot / 1e6:.3f} | {avg / 1e3:.2f} | {mn / 1e3:.2f} | {mx / 1e3:.2f} "
              f"| {100.0 * tot / total:.1f} |")
    print()
    print("Per launch shape (workgroups = grid / workgroup size):")
    print()
    print("| kernel | workgroups | calls | avg us | min us | max us |")
    print("|---|---:|---:|---:|---:|---:|")
    for name, wgs, n, avg, mn, mx in c.execute(
            "select name, grid_x / workgroup_x, count(*), avg(duration), min(duration), max(duration) "
            "from kernels where name like '%k_walk%' or name like '%k_cutoff%' or name like '%k_reduce%' "
            "or name like '%attn%' or name like '%rmsnorm%' "
            "group by name, grid_x order by name, grid_x"):
        print(f"| `{name[:60]}` | {wgs} | {n} | {avg / 1e3:.2f} | {mn / 1e3:.2f} | {mx / 1e3:.2f} |")


if __name__ == "__main__":
    main()
