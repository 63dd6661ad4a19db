"""bench.py's counter summaries on small rocpd-shaped databases (no GPU): the
calibration takes the last three copyBuffer dispatches, GRBM counters take the max
over instances and the others the sum, and the per-kernel table's arithmetic."""

import json
import os
import sqlite3
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402

MIB = 1 << 20


def _pmc_db(path, dispatches):
    """dispatches: (id, kernel name, {counter: [per-instance values]})."""
    db = sqlite3.connect(path)
    db.execute("create table pmc_events (name text, dispatch_id int, counter_name text, counter_value real)")
    for did, name, counters in dispatches:
        for c, vals in counters.items():
            for v in vals:
                db.execute("insert into pmc_events values (?, ?, ?, ?)", (name, did, c, v))
    db.commit()
    db.close()


def _trace_db(path, kernels):
    db = sqlite3.connect(path)
    db.execute("create table kernels (name text, duration int)")
    db.executemany("insert into kernels values (?, ?)", kernels)
    db.commit()
    db.close()


def _copy(did, fetch_kib=None, write_kib=None):
    c = {}
    if fetch_kib is not None:
        c["FETCH_SIZE"] = [fetch_kib / 2, fetch_kib / 2]  # two instances
    if write_kib is not None:
        c["WRITE_SIZE"] = [write_kib]
    return (did, "__amd_rocclr_copyBuffer", c)


def test_calibration_uses_the_last_three_copies(tmp_path):
    f, w = tmp_path / "f", tmp_path / "w"
    f.mkdir()
    w.mkdir()
    calib = 512 * MIB  # 256 MiB read + 256 MiB written
    # an earlier, larger setup copy must not be taken for the calibration
    _pmc_db(f / "a.db", [_copy(1, fetch_kib=900000),
                         (2, "void mk2::k_k2_layer<1>(mk2::K2Dev)", {"FETCH_SIZE": [60000, 60000]}),
                         _copy(3, fetch_kib=131072), _copy(4, fetch_kib=131072), _copy(5, fetch_kib=131072)])
    _pmc_db(w / "a.db", [_copy(1, write_kib=10),
                         (2, "void mk2::k_k2_layer<1>(mk2::K2Dev)", {"WRITE_SIZE": [15000]}),
                         _copy(3, write_kib=262144), _copy(4, write_kib=262144), _copy(5, write_kib=262144)])
    rec = bench.pmc_summary([str(f), str(w)], calib)
    assert rec["scale"]["FETCH_SIZE"] == pytest.approx(2.0)
    assert rec["scale"]["WRITE_SIZE"] == pytest.approx(1.0)
    assert rec["traffic_bytes_per_launch"] == int(120000 * 1024 * 2.0 + 15000 * 1024 * 1.0)


def test_calibration_rejects_disagreeing_copies(tmp_path):
    _pmc_db(tmp_path / "a.db", [_copy(1, fetch_kib=131072), _copy(2, fetch_kib=131072), _copy(3, fetch_kib=150000)])
    with pytest.raises(SystemExit):
        bench.pmc_summary([str(tmp_path)], 512 * MIB)


def test_per_kernel_table(tmp_path):
    (tmp_path / "kt").mkdir()
    (tmp_path / "p").mkdir()
    name = "void mk2::k_idx_score(mk2::IdxDev)"
    _trace_db(tmp_path / "kt" / "kt.db", [(name, 10000), (name, 14000), ("void other(int)", 5)])
    _pmc_db(tmp_path / "p" / "p.db", [
        (1, name, {"FETCH_SIZE": [10000, 10000], "WRITE_SIZE": [2000],
                   "TCC_EA0_RDREQ_DRAM_32B": [600000, 650000],
                   "SQ_VALU_MFMA_BUSY_CYCLES": [1024 * 100], "GRBM_GUI_ACTIVE": [1000, 1000, 1000],
                   "SQ_INSTS_VALU_MFMA_MOPS_BF16": [1000000], "SQ_LDS_BANK_CONFLICT": [7, 8]}),
        _copy(2, fetch_kib=131072, write_kib=262144), _copy(3, fetch_kib=131072, write_kib=262144),
        _copy(4, fetch_kib=131072, write_kib=262144),
    ])
    out = bench.pmc_kernels([str(tmp_path)], 512 * MIB)
    json.dumps(out)
    (row,) = out["kernels"]
    assert row["calls"] == 2 and row["avg_us"] == 12.0
    assert row["read_mb"] == round(20000 * 1024 * 2.0 / 1e6, 2)
    assert row["write_mb"] == round(2000 * 1024 / 1e6, 2)
    assert row["dram32_read_mb"] == round(1250000 * 32 / 1e6, 2)
    assert row["hbm_gbs"] == round((20000 * 1024 * 2.0 + 2000 * 1024) / 12e-6 / 1e9, 1)
    # GRBM: max over instances (1000), not their sum
    assert row["mfma_busy_pct"] == 10.0
    assert row["mfma_tflops"]["BF16"] == round(1000000 * 512 / 12e-6 / 1e12, 2)
    assert row["lds_bank_conflict_cycles"] == 15


def test_timeline_markdown_records_a_command_that_parses_back():
    """The recorded command quotes its arguments: an empty --extra-rows survives, so the
    command in a committed profile runs as written."""
    import shlex

    stage = {"first_in": 0.0, "ready_median": 1.0, "ready_last": None, "last_out": 2.5}
    tl = {name: stage for name in bench.TIMELINE_STAGES + bench.ROUTE_MARKS}
    argv = ["bench.py", "--rows", "32", "--extra-rows", "", "--timeline", "profiles/x.md"]
    md = bench.timeline_markdown(tl, argv, 32, 24)
    cmd = next(l for l in md.splitlines() if l.startswith("    python3 "))
    assert shlex.split(cmd.strip())[1:] == argv
    assert "| 2.50 |" in md and "| - |" in md
