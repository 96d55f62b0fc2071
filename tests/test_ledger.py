"""Solution ledger (reference ILedger, include/unikern/components.hpp:83-125): both stores, the
reference's row formats and schema, all-or-nothing commits (the crash-transaction test of
tests/smoke.cpp:49-76), violation events kept apart from solutions, and calibration
(src/solver.cpp:194-244)."""
from __future__ import annotations

import json
import sqlite3
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
GEMM = '{"op": "gemm", "dtype": "fp16", "dims": [4096, 4096, 4096], "layout": "TN"}'
ROWS = '{"op": "rmsnorm", "dtype": "fp32", "dims": [4096, 4096]}'


@pytest.fixture(params=["ledger.jsonl", "ledger.sqlite3"])
def ledger_path(tmp_path, request):
    return tmp_path / request.param


def test_miss_commit_hit_replace(uk, ledger_path):
    with uk.Ledger(ledger_path) as L:
        assert L.lookup(GEMM) is None
        sol = uk.solve(uk.kml_import(GEMM))
        L.commit(GEMM, sol.plan)  # solve-only row
        hit = L.lookup(GEMM)
        assert hit is not None
        assert hit.plan.key == sol.plan.key and (hit.plan.family, hit.plan.variant) == (sol.plan.family,
                                                                                         sol.plan.variant)
        assert hit.c_ms == pytest.approx(sol.predicted_us * 1e-3, rel=0, abs=0)  # exact round trip
        assert hit.measured_ms == 0.0
        L.commit(GEMM, sol.plan, measured_ms=0.5, kernel_ms=0.15)  # run replaces it
        hit = L.lookup(GEMM)
        assert (hit.measured_ms, hit.kernel_ms) == (0.5, 0.15)
        assert L.lookup(ROWS) is None
        n, v = L.size()
        assert v == 0 and n == (1 if ledger_path.suffix == ".sqlite3" else 2)  # text store appends


def test_violations_are_not_solutions(uk, ledger_path):
    with uk.Ledger(ledger_path) as L:
        L.record_violation(ROWS, 0.5, 0.0, 1, 2, 1 << 30)
        L.record_violation(ROWS, 1.0, 0.0, 2, 2, 1 << 30)
        assert L.size() == (0, 2)
        assert L.lookup(ROWS) is None


def test_key_is_signature_fingerprint_tree_hash(uk):
    key = uk.Ledger.key(GEMM)
    sig, fp, th = key.split("|")
    assert sig == "gemm:fp16:4096x4096x4096:TN"
    assert fp == uk.hcs_fingerprint()
    assert th == uk.tree_hash(GEMM)
    other = uk.Ledger.key(GEMM, (ROOT / "samples" / "hcs_mi355x.json").read_text().replace('"clock_mhz": 2400',
                                                                                           '"clock_mhz": 2100'))
    assert other.split("|")[1] != fp  # another HCS files elsewhere


def test_reads_reference_text_rows(uk, tmp_path):
    # The reference's 4-, 6- and 7-field lines (src/runtime.cpp:36-83) with a plan placement.
    key = uk.Ledger.key(ROWS)
    p = tmp_path / "ref.jsonl"
    place = "plan=rows:tpr=512,nv=2,nt family=1 variant=17 | from the reference layout"
    p.write_text(f"{key}\t0.03\t0.04\t{place}\n")
    with uk.Ledger(p) as L:
        hit = L.lookup(ROWS)
        assert hit.plan.variant == 17 and hit.c_ms == 0.03 and hit.measured_ms == 0.04
    p.write_text(f"{key}\t0.03\t0.04\t64\t128\t{place}\n")
    with uk.Ledger(p) as L:
        hit = L.lookup(ROWS)
        assert (hit.plan.tile_m, hit.plan.tile_n) == (64, 128)
    p.write_text(f"{key}\tnot-a-number\t0.04\t{place}\n{key}\t0.03\t0.05\t0.02\t1\t2\t{place}\n")
    with uk.Ledger(p) as L:
        hit = L.lookup(ROWS)  # the corrupt line is skipped
        assert (hit.measured_ms, hit.kernel_ms) == (0.05, 0.02)


def test_opens_reference_sqlite_schema_and_migrates(uk, tmp_path):
    # A database in the reference's pre-calibration schema (no kernel_ms column,
    # src/sqlite_ledger.cpp:44-62) gains the column on open and keeps its rows.
    db = tmp_path / "old.sqlite3"
    con = sqlite3.connect(db)
    con.execute("CREATE TABLE solutions(key TEXT PRIMARY KEY, op_sig TEXT, hcs_fp TEXT, tree_hash TEXT, "
                "c_ms REAL, measured_ms REAL, tm INTEGER, tn INTEGER, placement TEXT)")
    key = uk.Ledger.key(ROWS)
    sig, fp, th = key.split("|")
    con.execute("INSERT INTO solutions VALUES(?,?,?,?,?,?,?,?,?)",
                (key, sig, fp, th, 0.03, 0.04, 0, 0, "plan=rows:tpr=512,nv=2,nt family=1 variant=17 | x"))
    con.commit()
    con.close()
    with uk.Ledger(db) as L:
        hit = L.lookup(ROWS)
        assert hit.plan.key == b"rows:tpr=512,nv=2,nt" and hit.kernel_ms == 0.0
        assert L.size() == (1, 0)
    cols = [r[1] for r in sqlite3.connect(db).execute("PRAGMA table_info(solutions)")]
    assert "kernel_ms" in cols


CRASH_CHILD = r"""
import os, sqlite3, sys
con = sqlite3.connect(sys.argv[1], isolation_level=None)
con.execute("PRAGMA cache_size=1")
con.execute("CREATE TABLE IF NOT EXISTS solutions(key TEXT PRIMARY KEY, op_sig TEXT, hcs_fp TEXT, tree_hash TEXT, "
            "c_ms REAL, measured_ms REAL, tm INTEGER, tn INTEGER, placement TEXT)")
con.execute("BEGIN IMMEDIATE")
for i in range(2000):
    con.execute("INSERT INTO solutions(key, op_sig, hcs_fp, tree_hash, c_ms, measured_ms, tm, tn, placement) "
                "VALUES(?, 'op', 'fp', 'th', 1.0, 1.0, 0, 0, 'half-row')", (f"crash-{i}",))
open(sys.argv[1] + ".marker", "w").write("reached-uncommitted-tx")
os._exit(9)
"""


def test_interrupted_transaction_leaves_no_row(uk, tmp_path):
    # tests/smoke.cpp:49-76: a process dies inside BEGIN IMMEDIATE .. (no COMMIT); the hot journal
    # is rolled back on the next open, so the ledger holds no half record.
    db = tmp_path / "crash.sqlite3"
    r = subprocess.run([sys.executable, "-c", CRASH_CHILD, str(db)])
    assert r.returncode == 9
    assert (tmp_path / "crash.sqlite3.marker").read_text() == "reached-uncommitted-tx"
    with uk.Ledger(db) as L:
        assert L.size() == (0, 0)
        sol = uk.solve(uk.kml_import(ROWS))
        L.commit(ROWS, sol.plan, measured_ms=0.1, kernel_ms=0.02)
        assert L.size() == (1, 0)


def test_calibrate_link_bandwidth(uk, ledger_path):
    hcs = (ROOT / "samples" / "hcs_mi355x.json").read_text()
    with uk.Ledger(ledger_path) as L:
        with pytest.raises(uk.UnikernError) as e:
            L.calibrate(hcs)
        assert e.value.code == uk.UK_INFEASIBLE
        # bytes / (measured - kernel): rmsnorm moves 134,234,112 B; 10 ms of copies -> 13.42 GB/s;
        # gemm f16 4096^3 moves 100,663,296 B in 5 ms -> 20.13 GB/s; median of two = mean
        for kml, copy_ms in ((ROWS, 10.0), (GEMM, 5.0)):
            sol = uk.solve(uk.kml_import(kml), hcs)
            L.commit(kml, sol.plan, measured_ms=copy_ms + 0.1, kernel_ms=0.1, hcs_json=hcs)
        out, detail = L.calibrate(hcs)
        cal = json.loads(out)
        want = 0.5 * (134_234_112 / 10e6 + 100_663_296 / 5e6)
        assert cal["link_bw_gbps"] == pytest.approx(want, rel=1e-9)
        assert cal["constants_version"] == 2 and "usable_rows=2" in detail
        assert uk.hcs_fingerprint(out) != uk.hcs_fingerprint(hcs)


def test_hcs_with_capacity(uk):
    t = uk.hcs_with_capacity(None, 12345678)
    assert json.loads(t)["tiers"][0]["bytes"] == 12345678
    d = uk.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN")
    with pytest.raises(uk.UnikernError):
        uk.solve(d, t)  # 100 MB working set no longer fits
