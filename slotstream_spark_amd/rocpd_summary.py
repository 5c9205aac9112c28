"""Summaries of rocprofv3 result databases (rocpd SQLite), as committed under profiles/.

  python -m slotstream_spark_amd.rocpd_summary kernels RUN_results.db        per-kernel calls / avg / min / max (us)
  python -m slotstream_spark_amd.rocpd_summary counters RUN_results.db [pat]  per-kernel average of each counter
  python -m slotstream_spark_amd.rocpd_summary grids RUN_results.db [pat]     per kernel and launch shape (workgroups
                                                                              x threads), names like pat
  python -m slotstream_spark_amd.rocpd_summary sequence RUN_results.db pat n1,n2,...
                                                 the dispatches of kernels named like pat in launch order, split into
                                                 consecutive groups of n1, n2, ... dispatches (one group per phase of
                                                 the program, e.g. per bench configuration), median / min / max each
"""
from __future__ import annotations

import sqlite3
import sys


def kernels(db: str) -> str:
    c = sqlite3.connect(db)
    rows = list(c.execute("""select name, count(*), avg(end - start), min(end - start), max(end - start),
                                    sum(end - start) from kernels group by name order by sum(end - start) desc"""))
    tot = sum(r[5] for r in rows) or 1
    out = [f"{'kernel':70s} {'calls':>6s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'pct':>6s}"]
    for n, cnt, avg, mn, mx, s in rows:
        out.append(f"{n[:70]:70s} {cnt:6d} {avg / 1e3:9.2f} {mn / 1e3:9.2f} {mx / 1e3:9.2f} {100 * s / tot:6.1f}")
    return "\n".join(out)


def grids(db: str, pattern: str = "%") -> str:
    """One line per (kernel, workgroups, threads per workgroup): a kernel launched at several shapes (the draft head's
    GEMV instantiations) splits into its launch kinds."""
    c = sqlite3.connect(db)
    rows = c.execute("""select name, grid_x, workgroup_x, count(*), avg(end - start), min(end - start),
                               max(end - start) from kernels where name like ? group by name, grid_x, workgroup_x
                        order by sum(end - start) desc""", (pattern,))
    out = [f"{'kernel':72s} {'wgs':>6s} {'thr':>4s} {'calls':>6s} {'avg_us':>8s} {'min_us':>8s} {'max_us':>8s}"]
    for n, gx, wx, cnt, avg, mn, mx in rows:
        n = n.replace("(anonymous namespace)::", "").replace("ss::", "")
        out.append(f"{n[:72]:72s} {gx // max(wx, 1):6d} {wx:4d} {cnt:6d} {avg / 1e3:8.2f} {mn / 1e3:8.2f} {mx / 1e3:8.2f}")
    return "\n".join(out)


def counters(db: str, pattern: str = "%") -> str:
    c = sqlite3.connect(db)
    rows = c.execute("""select kernel_name, counter_name, avg(value), min(value), max(value), count(*)
                        from counters_collection where kernel_name like ? group by kernel_name, counter_name
                        order by kernel_name""", (pattern,))
    return "\n".join(f"{k[:60]:60s} {n:14s} avg {v:14.2f} min {lo:14.2f} max {hi:14.2f} ({cnt} dispatches)"
                     for k, n, v, lo, hi, cnt in rows)


def sequence(db: str, pattern: str, sizes: list[int]) -> str:
    c = sqlite3.connect(db)
    d = [r[0] for r in c.execute("select end - start from kernels where name like ? order by start", (pattern,))]
    if sum(sizes) != len(d):
        raise SystemExit(f"{len(d)} dispatches named like {pattern!r}, groups cover {sum(sizes)}")
    out = [f"{'group':>5s} {'calls':>6s} {'median_us':>10s} {'min_us':>9s} {'max_us':>9s}"]
    i = 0
    for g, n in enumerate(sizes):
        v = sorted(d[i:i + n])
        i += n
        med = v[n // 2] if n % 2 else (v[n // 2 - 1] + v[n // 2]) / 2
        out.append(f"{g:5d} {n:6d} {med / 1e3:10.2f} {v[0] / 1e3:9.2f} {v[-1] / 1e3:9.2f}")
    return "\n".join(out)


if __name__ == "__main__":
    what, db = sys.argv[1], sys.argv[2]
    pat = sys.argv[3] if len(sys.argv) > 3 else "%"
    if what == "sequence":
        print(sequence(db, pat, [int(x) for x in sys.argv[4].split(",")]))
    else:
        print(kernels(db) if what == "kernels" else grids(db, pat) if what == "grids" else counters(db, pat))
