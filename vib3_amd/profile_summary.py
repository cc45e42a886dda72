"""Summarise rocprofv3 SQLite output (the `*_results.db` a run writes) as short text.

    python -m vib3_amd.profile_summary trace <db>   per-kernel dispatch count and durations
    python -m vib3_amd.profile_summary pmc <db>     per-kernel average of each PMC counter
    python -m vib3_amd.profile_summary traffic <fetch_db> <write_db> <out.json> <source>
                                               [<cal_fetch_db> <cal_write_db>]
        HBM bytes per dispatch of each kernel: FETCH_SIZE and WRITE_SIZE (KiB) scaled by what
        the same counter reads for the bench's 1 GiB device copies (the calibration; taken from
        the optional databases when the runs themselves hold no copy, as bench --config c4)

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


def _kernel_key(name: str) -> str:
    """`void vib3::k_mx_gemm<true, 4>(vib3::MxArgs)` -> `k_mx_gemm<true, 4>`."""
    short = name.replace("(anonymous namespace)::", "").split("vib3::", 1)[-1]
    depth = 0
    for i, ch in enumerate(short):
        depth += ch == "<"
        depth -= ch == ">"
        if ch == "(" and depth == 0:
            return short[:i]
    return short


def _counter(db: str, counter: str):
    con = sqlite3.connect(db)
    per = {}
    for k, v in con.execute("select kernel_name, avg(value) from counters_collection "
                            "where counter_name = ? group by kernel_name", (counter,)):
        if "vib3::" in k and "synth" not in k:
            per[_kernel_key(k)] = float(v)
    cal = con.execute("select avg(value) from counters_collection where counter_name = ? and "
                      "kernel_name like '%copy%' and duration > 200000", (counter,)).fetchone()[0]
    return per, cal


def traffic(fetch_db: str, write_db: str, out: str, source: str, cal_fetch_db: str = "",
            cal_write_db: str = "") -> None:
    import json
    fetch, fcal = _counter(fetch_db, "FETCH_SIZE")
    write, wcal = _counter(write_db, "WRITE_SIZE")
    if fcal is None and cal_fetch_db:
        fcal = _counter(cal_fetch_db, "FETCH_SIZE")[1]
    if wcal is None and cal_write_db:
        wcal = _counter(cal_write_db, "WRITE_SIZE")[1]
    gib_kib = float(1 << 20)
    ff, wf = gib_kib / fcal, gib_kib / wcal  # counter KiB -> bytes moved, per the copy kernels
    res = {"source": source,
           "calibration": {"copy_bytes_each_way": 1 << 30, "FETCH_SIZE_KiB": round(fcal, 1),
                           "WRITE_SIZE_KiB": round(wcal, 1), "fetch_factor": round(ff, 4),
                           "write_factor": round(wf, 4)},
           "kernels": {}}
    for k in sorted(set(fetch) | set(write)):
        f, w = fetch.get(k, 0.0), write.get(k, 0.0)
        res["kernels"][k] = {"FETCH_SIZE_KiB": round(f, 1), "WRITE_SIZE_KiB": round(w, 1),
                             "hbm_bytes": round((f * ff + w * wf) * 1024)}
    with open(out, "w") as fh:
        json.dump(res, fh, indent=1)
        fh.write("\n")
    print(json.dumps(res, indent=1))


if __name__ == "__main__":
    if len(sys.argv) in (6, 8) and sys.argv[1] == "traffic":
        traffic(*sys.argv[2:])
    elif len(sys.argv) == 3 and sys.argv[1] in ("trace", "pmc"):
        (trace if sys.argv[1] == "trace" else pmc)(sys.argv[2])
    else:
        print(__doc__, file=sys.stderr)
        sys.exit(2)
