"""Summarises a rocprofv3 output directory (rocpd SQLite database) as text:
per-kernel dispatch count and average / min / max duration from a
--kernel-trace run, one row per kernel and launch shape (workgroups), so that
the same kernel launched by two operations (e.g. the column-sum finalize of
the LayerNorm backward, 48 workgroups, and of the GELU backward, 96) gets two
rows; or per-kernel average counter values from a --pmc run.

  python3 cme213-final-project_amd/cme213_amd/rocpd_summary.py DIR [DIR ...]
"""
import collections
import glob
import re
import sqlite3
import sys


def short(name):
    n = name.replace("mi::(anonymous namespace)::", "").replace("(anonymous namespace)::", "")
    m = re.match(r"(?:void )?([A-Za-z_0-9]+(?:<[^()]*?>)?)", n)
    s = m.group(1) if m else n[:60]
    op = re.search(r"(\w+Op)<", n)
    if op and op.group(1) not in s:
        s += " [" + op.group(1) + "]"
    return s[:90]


def summarise(d):
    dbs = glob.glob(d + "/**/*.db", recursive=True)
    if not dbs:
        print(f"{d}: no rocpd database")
        return
    c = sqlite3.connect(dbs[0])
    tables = {r[0] for r in c.execute("select name from sqlite_master")}
    if "counters_collection" in tables and c.execute(
            "select count(*) from counters_collection").fetchone()[0]:
        rows = collections.defaultdict(list)
        for name, cn, val in c.execute(
                "select kernel_name, counter_name, value from counters_collection "
                "order by dispatch_id"):
            rows[(short(name), cn)].append(val)
        print(f"{'counter':12s} {'n':>3s} {'avg (KiB)':>14s}  kernel")
        for (k, cn), v in sorted(rows.items()):
            print(f"{cn:12s} {len(v):3d} {sum(v) / len(v):14.1f}  {k}")
    else:
        print(f"{'n':>5s} {'avg us':>9s} {'min us':>9s} {'max us':>9s} {'wgs':>7s}  kernel")
        q = ("select name, grid_x / max(workgroup_x, 1), count(*), avg(end-start)/1000.0, "
             "min(end-start)/1000.0, max(end-start)/1000.0 from kernels "
             "group by name, grid_x, workgroup_x order by sum(end-start) desc")
        for name, wgs, n, avg, mn, mx in c.execute(q):
            print(f"{n:5d} {avg:9.2f} {mn:9.2f} {mx:9.2f} {wgs:7d}  {short(name)}")


if __name__ == "__main__":
    for d in sys.argv[1:]:
        summarise(d)
