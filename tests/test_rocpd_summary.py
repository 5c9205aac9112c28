"""The profile summaries (slotstream_spark_amd/rocpd_summary.py) on a small synthetic database with rocpd's kernels
view layout (name, start, end in ns)."""
import sqlite3

import pytest

from slotstream_spark_amd import rocpd_summary as rs


@pytest.fixture
def db(tmp_path):
    p = tmp_path / "run_results.db"
    c = sqlite3.connect(p)
    c.execute("create table kernels(name text, start int, end int, grid_x int, workgroup_x int)")
    # kernel "k": three 10 us dispatches, then four of 50, 52, 54, 90 us; "z" one 4 us dispatch in between
    durs = [10_000] * 3 + [50_000, 52_000, 54_000, 90_000]
    rows = [("k", 1_000_000 * i, 1_000_000 * i + d, 65536, 256) for i, d in enumerate(durs)]
    rows.append(("z", 1_500_000, 1_504_000, 256, 256))
    c.executemany("insert into kernels values (?, ?, ?, ?, ?)", rows)
    c.commit()
    return str(p)


def test_kernels_totals(db):
    lines = rs.kernels(db).splitlines()
    assert lines[1].split()[:5] == ["k", "7", "39.43", "10.00", "90.00"]
    assert lines[2].split()[:2] == ["z", "1"]


def test_sequence_groups_in_launch_order(db):
    lines = rs.sequence(db, "k", [3, 4]).splitlines()
    assert lines[1].split() == ["0", "3", "10.00", "10.00", "10.00"]
    assert lines[2].split() == ["1", "4", "53.00", "50.00", "90.00"]  # even count: mean of the middle two


def test_sequence_rejects_groups_that_do_not_cover(db):
    with pytest.raises(SystemExit, match="7 dispatches"):
        rs.sequence(db, "k", [3, 3])
