"""Summarise rocprofv3 SQLite output (the `*_results.db` a run writes) as short text.

    python -m vib3_amd.profile_summary trace <db>   per-kernel dispatch count and durations
    python -m vib3_amd.profile_summary pmc <db>     per-kernel average of each PMC counter

Only kernels of this library and the runtime copy kernels are listed (the synthetic-weight
generator kernels are skipped).
"""
from __future__ import annotations

import sqlite3
import statistics
import sys


def _keep(name: str) -> bool:
    return ("vib3::" in name and "synth" not in name) or "copy" in name.lower()


def trace(db: str) -> None:
    con = sqlite3.connect(db)
    rows = con.execute("select name, start, end from kernels order by start").fetchall()
    by = {}
    for name, s, e in rows:
        if _keep(name):
            by.setdefault(name, []).append((e - s) / 1000.0)
    print(f"{'dispatches':>10} {'avg_us':>9} {'median_us':>9} {'min_us':>8} {'max_us':>8}  kernel")
    for name, d in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        print(f"{len(d):10d} {statistics.mean(d):9.2f} {statistics.median(d):9.2f} "
              f"{min(d):8.2f} {max(d):8.2f}  {name[:110]}")


def pmc(db: str) -> None:
    con = sqlite3.connect(db)
    q = ("select kernel_name, counter_name, count(*), avg(value), avg(duration), max(value) "
         "from counters_collection group by kernel_name, counter_name order by kernel_name")
    print(f"{'counter':20s} {'dispatches':>10} {'avg_value':>14} {'max_value':>14} {'avg_dur_us':>10}"
          "  kernel")
    for k, c, n, v, d, mx in con.execute(q):
        if _keep(k):
            print(f"{c:20s} {n:10d} {v:14.1f} {mx:14.1f} {d / 1000:10.2f}  {k[:100]}")
    # copy kernels: the long dispatches are the bench's 1 GiB device-to-device copies, the
    # calibration of the byte counters (value per GiB moved)
    q = ("select counter_name, count(*), avg(value), avg(duration) from counters_collection "
         "where kernel_name like '%copy%' and duration > 200000 group by counter_name")
    for c, n, v, d in con.execute(q):
        print(f"calibration: {c} over {n} copy dispatches longer than 200 us: avg {v:.1f} "
              f"(avg {d / 1000:.1f} us)")


if __name__ == "__main__":
    if len(sys.argv) != 3 or sys.argv[1] not in ("trace", "pmc"):
        print(__doc__, file=sys.stderr)
        sys.exit(2)
    (trace if sys.argv[1] == "trace" else pmc)(sys.argv[2])
