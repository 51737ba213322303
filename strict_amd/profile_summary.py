"""Summaries of rocprofv3 output for the libstrict_hip kernels.

    python -m strict_amd.profile_summary trace <run_kernel_trace.csv | run_results.db> [--last N]
    python -m strict_amd.profile_summary counters <run_counter_collection.csv | run_results.db> [--last N]

Either rocprofv3's CSV files or its default rocpd SQLite database
(``run_results.db``) are read; the database survives a profiler that
crashes while writing its CSV files at exit.

``trace``: per-kernel dispatch count, average and total duration of the last N
dispatches (all by default), plus their span from first start to last end;
with a decode step's dispatch count as N this is the per-step breakdown.
``counters``: per-kernel average of each PMC counter per dispatch (for
FETCH_SIZE / WRITE_SIZE: KiB per dispatch as the hardware counts them).
"""
from __future__ import annotations

import argparse
import collections
import csv
import sys


def _rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _demangle(names: dict) -> dict:
    """Demangled kernel names through c++filt when it is installed."""
    import shutil
    import subprocess

    if not names or not shutil.which("c++filt"):
        return names
    keys = list(names)
    res = subprocess.run(["c++filt"], input="\n".join(names[k] for k in keys), text=True,
                         capture_output=True)
    out = res.stdout.splitlines()
    return dict(zip(keys, out)) if res.returncode == 0 and len(out) == len(keys) else names


def _db_dispatches(path):
    """Kernel dispatches of a rocpd database as CSV-like rows."""
    import sqlite3

    con = sqlite3.connect(path)
    names = _demangle({k: v.removesuffix(".kd") for k, v in
                       con.execute("select id, kernel_name from rocpd_info_kernel_symbol")})
    rows = []
    for kid, ev, start, end, did in con.execute(
            "select kernel_id, event_id, start, end, dispatch_id from rocpd_kernel_dispatch"):
        rows.append({"Kernel_Name": names.get(kid, str(kid)),
                     "Start_Timestamp": start, "End_Timestamp": end, "Dispatch_Id": did,
                     "_event": ev})
    return con, rows


def _db_counter_rows(path):
    """(dispatch row, counter name, value summed over instances) of a rocpd database."""
    con, disp = _db_dispatches(path)
    by_event = {r["_event"]: r for r in disp}
    pmc = dict(con.execute("select id, name from rocpd_info_pmc"))
    sums = collections.defaultdict(float)
    for ev, pid, val in con.execute("select event_id, pmc_id, value from rocpd_pmc_event"):
        sums[(ev, pmc.get(pid, str(pid)))] += float(val)
    out = []
    for (ev, name), val in sums.items():
        if ev in by_event:
            r = dict(by_event[ev])
            r["Counter_Name"] = name
            r["Counter_Value"] = val
            out.append(r)
    return out


def trace(path: str, last: int | None) -> str:
    rows = _db_dispatches(path)[1] if path.endswith(".db") else _rows(path)
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    if last:
        rows = rows[-last:]
    agg = collections.defaultdict(list)
    for r in rows:
        agg[r["Kernel_Name"]].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    span = int(rows[-1]["End_Timestamp"]) - int(rows[0]["Start_Timestamp"])
    busy = sum(sum(v) for v in agg.values())
    out = [f"{len(rows)} dispatches: span {span / 1e3:.1f} us, summed kernel time {busy / 1e3:.1f} us",
           f"{'calls':>7} {'avg_us':>9} {'total_us':>10}  kernel"]
    for k, v in sorted(agg.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"{len(v):7d} {sum(v) / len(v) / 1e3:9.2f} {sum(v) / 1e3:10.1f}  {k[:120]}")
    return "\n".join(out)


def counters(path: str, last: int | None) -> str:
    rows = _db_counter_rows(path) if path.endswith(".db") else _rows(path)
    key = "Dispatch_Id" if "Dispatch_Id" in rows[0] else "Correlation_Id"
    rows.sort(key=lambda r: int(r[key]))
    if last:
        ids = sorted({int(r[key]) for r in rows})[-last:]
        keep = set(ids)
        rows = [r for r in rows if int(r[key]) in keep]
    agg = collections.defaultdict(lambda: collections.defaultdict(float))
    calls = collections.defaultdict(set)
    for r in rows:
        agg[r["Kernel_Name"]][r["Counter_Name"]] += float(r["Counter_Value"])
        calls[r["Kernel_Name"]].add(int(r[key]))
    out = [f"{'calls':>7}  counter averages per dispatch  kernel"]
    for k in sorted(agg, key=lambda k: -len(calls[k])):
        n = len(calls[k])
        vals = ", ".join(f"{c}={v / n:.1f}" for c, v in sorted(agg[k].items()))
        out.append(f"{n:7d}  {vals}  {k[:120]}")
    return "\n".join(out)


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("kind", choices=["trace", "counters"])
    p.add_argument("csv")
    p.add_argument("--last", type=int, default=None)
    a = p.parse_args(argv)
    print(trace(a.csv, a.last) if a.kind == "trace" else counters(a.csv, a.last))
    return 0


if __name__ == "__main__":
    sys.exit(main())
