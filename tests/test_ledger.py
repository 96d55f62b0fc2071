"""Solution ledger (reference ILedger, include/unikern/components.hpp:83-125): both stores, the
reference's row formats and schema, all-or-nothing commits (the crash-transaction test of
tests/smoke.cpp:49-76), violation events kept apart from solutions, and the calibration closure
that replaces the reference's (src/main.cpp:579-652)."""
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


SOFTMAX = '{"op": "softmax", "dtype": "fp32", "dims": [4096, 4096]}'
ROWSUM = '{"op": "reduce", "dtype": "fp32", "dims": [4096, 4096]}'


def _commit_ratio(uk, L, kml, hcs, ratio, copy_ms=0.0):
    """Commit a row whose kernel-only time is the prediction / ratio, plus copy_ms of host copies."""
    sol = uk.solve(uk.kml_import(kml), hcs)
    kernel_ms = sol.predicted_us * 1e-3 / ratio
    L.commit(kml, sol.plan, measured_ms=kernel_ms + copy_ms, kernel_ms=kernel_ms, hcs_json=hcs)
    return sol


def test_calibrate_rate_constants(uk, ledger_path):
    hcs = (ROOT / "samples" / "hcs_mi355x.json").read_text()
    base = json.loads(hcs)
    with uk.Ledger(ledger_path) as L:
        with pytest.raises(uk.UnikernError) as e:
            L.calibrate(hcs)
        assert e.value.code == uk.UK_INFEASIBLE
        # Streaming rows 2x too slow and 2x too fast cancel: a geometric mean, not an arithmetic one
        # (which would raise the bandwidth by 1.25x).
        _commit_ratio(uk, L, ROWS, hcs, 2.0)
        _commit_ratio(uk, L, SOFTMAX, hcs, 0.5)
        cal = json.loads(L.calibrate(hcs)[0])
        assert cal["hbm_bw_gbps"] == pytest.approx(base["hbm_bw_gbps"], rel=1e-12)
        assert cal["clock_mhz"] == base["clock_mhz"] and cal["constants_version"] == 2
        # A third streaming row 8x too pessimistic: (2 * 0.5 * 8)^(1/3) = 2.
        _commit_ratio(uk, L, ROWSUM, hcs, 8.0)
        # One MFMA-bound row that ran 1.25x faster than predicted: the clock it is priced at rises.
        g_before = _commit_ratio(uk, L, GEMM, hcs, 1.25)
        out, detail = L.calibrate(hcs)
        cal = json.loads(out)
        assert cal["hbm_bw_gbps"] == pytest.approx(2.0 * base["hbm_bw_gbps"], rel=1e-9)
        assert cal["clock_mhz"] == pytest.approx(1.25 * base["clock_mhz"], rel=1e-9)
        assert cal["link_bw_gbps"] == base["link_bw_gbps"]  # no row carries host copy time
        assert "streaming: 3 row(s)" in detail and "matrix: 1 row(s)" in detail and "link" not in detail
        assert uk.hcs_fingerprint(out) != uk.hcs_fingerprint(hcs)
        # The calibrated description moves the solver's predictions toward what was measured.
        g_after = uk.solve(uk.kml_import(GEMM), out)
        measured_us = g_before.predicted_us / 1.25
        assert abs(g_after.predicted_us - measured_us) < 0.5 * abs(g_before.predicted_us - measured_us)
        r_before = uk.solve(uk.kml_import(ROWSUM), hcs).predicted_us
        r_after = uk.solve(uk.kml_import(ROWSUM), out).predicted_us
        assert r_after < 0.6 * r_before


def test_calibrate_link_line(uk, ledger_path):
    # copy_ms = 0.05 + bytes / 20 GB/s on three rows of different sizes: the least-squares line
    # recovers both the per-call latency and the link rate exactly (a per-row ratio would not).
    hcs = (ROOT / "samples" / "hcs_mi355x.json").read_text()
    nbytes = {ROWS: 134_234_112, GEMM: 100_663_296, ROWSUM: 67_125_248}
    with uk.Ledger(ledger_path) as L:
        for kml, b in nbytes.items():
            assert uk.workload_of(uk.kml_import(kml))["bytes"] == b
            _commit_ratio(uk, L, kml, hcs, 1.0, copy_ms=0.05 + b / 20e6)
        out, detail = L.calibrate(hcs)
        cal = json.loads(out)
        assert cal["link_bw_gbps"] == pytest.approx(20.0, rel=1e-6)
        assert "copy_ms = 0.05 +" in detail
        # ratio 1 everywhere: the rate constants stay where they were
        assert cal["hbm_bw_gbps"] == pytest.approx(8000.0, rel=1e-12)
        assert cal["clock_mhz"] == pytest.approx(2400.0, rel=1e-12)
    # A unified-memory description has no host copy: its link constant is left alone.
    uni = json.loads(hcs)
    uni["unified_memory"] = True
    uni["tiers"] = [{"name": "unified", "bytes": 1 << 40, "bw_gbps": 8000, "confidence": "official"}]
    uni = json.dumps(uni)
    upath = ledger_path.with_name("u" + ledger_path.name)
    with uk.Ledger(upath) as L:
        _commit_ratio(uk, L, ROWS, uni, 1.0, copy_ms=3.0)
        out, detail = L.calibrate(uni)
        assert json.loads(out)["link_bw_gbps"] == json.loads(uni)["link_bw_gbps"]
        assert "unified memory has no host copy" in detail


def test_calibrate_from_probe(uk, ledger_path):
    # No measured MFMA-bound row: the matrix-core probe's sustained clock, relative to the clock
    # under which the variant efficiencies were fitted (2.02 GHz), scales the priced clock.
    hcs = (ROOT / "samples" / "hcs_mi355x.json").read_text()
    with uk.Ledger(ledger_path) as L:
        out, detail = L.calibrate(hcs, probe={"clock_ghz": 2.02 * 0.9})
        cal = json.loads(out)
        assert cal["clock_mhz"] == pytest.approx(2400 * 0.9, rel=1e-9)
        assert cal["hbm_bw_gbps"] == 8000 and cal["constants_version"] == 2
        assert "probe sustains" in detail
        g0 = uk.solve(uk.kml_import(GEMM), hcs).predicted_us
        g1 = uk.solve(uk.kml_import(GEMM), out).predicted_us
        assert g1 > g0
        # A measured MFMA-bound row outranks the probe.
        _commit_ratio(uk, L, GEMM, hcs, 0.8)
        cal = json.loads(L.calibrate(hcs, probe={"clock_ghz": 2.02 * 0.9})[0])
        assert cal["clock_mhz"] == pytest.approx(2400 * 0.8, rel=1e-9)


def test_calibrate_leaves_out_streamed_and_replayed_rows(uk, ledger_path):
    # A streamed (scenario-B) GEMM row is priced as a pass of host copies overlapping shard
    # kernels while its kernel_ms covers the shard kernels only: its c_ms / kernel_ms measures copy
    # against kernel (here 15x), not the clock. Beside a resident streaming row (2x) the fit
    # takes only the resident one; a row replayed from a recorded output is left out as well.
    h = json.loads((ROOT / "samples" / "hcs_mi355x.json").read_text())
    h["tiers"][0]["bytes"] = 96 << 20
    hcs = json.dumps(h)
    streamed = uk.solve(uk.kml_import(GEMM), hcs)
    assert streamed.plan.shard_rows > 0
    with uk.Ledger(ledger_path) as L:
        _commit_ratio(uk, L, ROWSUM, hcs, 2.0)
        k_ms = streamed.predicted_us * 1e-3 / 15.0
        L.commit(GEMM, streamed.plan, measured_ms=20 * k_ms, kernel_ms=k_ms, hcs_json=hcs)
        sm = uk.solve(uk.kml_import(SOFTMAX))  # a plan from the full tier; the small one cannot hold it
        L.commit(SOFTMAX, sm.plan, measured_ms=sm.predicted_us * 1e-3 / 7.0, kernel_ms=sm.predicted_us * 1e-3 / 7.0,
                 hcs_json=hcs, replayed=True)
        assert L.lookup(SOFTMAX, hcs).measured_ms > 0  # the replayed row is kept for lookups
        out, detail = L.calibrate(hcs)
        cal = json.loads(out)
        assert cal["hbm_bw_gbps"] == pytest.approx(2.0 * h["hbm_bw_gbps"], rel=1e-9)
        assert cal["clock_mhz"] == h["clock_mhz"]  # no resident MFMA-bound row: the clock is kept
        assert cal["link_bw_gbps"] == h["link_bw_gbps"]  # the streamed pass is not one host copy
        assert "streaming: 1 row(s)" in detail and "matrix:" not in detail
        assert "left out: 1 replayed row(s)" in detail and "left out: 1 streamed row(s)" in detail
        # A resident GEMM row beside them is fitted as usual.
        _commit_ratio(uk, L, '{"op": "gemm", "dtype": "fp16", "dims": [1024, 1024, 1024], "layout": "TN"}', hcs, 1.25)
        cal = json.loads(L.calibrate(hcs)[0])
        assert cal["clock_mhz"] == pytest.approx(1.25 * h["clock_mhz"], rel=1e-9)


def test_streamed_plan_round_trips(uk, ledger_path):
    # A scenario-B plan's shard height is part of the recorded plan (placement text), so a ledger
    # hit runs the same streamed pass; rows written without it read back as resident.
    h = json.loads((ROOT / "samples" / "hcs_mi355x.json").read_text())
    h["tiers"][0]["bytes"] = 96 << 20
    hcs = json.dumps(h)
    sol = uk.solve(uk.kml_import(GEMM), hcs)
    assert sol.plan.shard_rows > 0
    with uk.Ledger(ledger_path) as L:
        L.commit(GEMM, sol.plan, measured_ms=5.0, kernel_ms=0.2, hcs_json=hcs)
        hit = L.lookup(GEMM, hcs)
        assert hit.plan.shard_rows == sol.plan.shard_rows and hit.plan.key == sol.plan.key
        assert hit.plan.stream_path == 1
        L.commit(ROWS, uk.solve(uk.kml_import(ROWS)).plan)
        assert L.lookup(ROWS).plan.shard_rows == 0 and L.lookup(ROWS).plan.stream_path == 0
        # The mapped path is recorded through its plan key ("+stream_mmap"), so a hit runs it again.
        mapped = sol.plan
        mapped.stream_path = 2
        mapped.key = sol.plan.key + b"_mmap"
        L.commit(GEMM, mapped, measured_ms=9.0, kernel_ms=0.3, hcs_json=hcs)
        hit = L.lookup(GEMM, hcs)
        assert hit.plan.stream_path == 2 and hit.plan.key.endswith(b"+stream_mmap")


def test_hcs_with_capacity(uk):
    t = uk.hcs_with_capacity(None, 12345678)
    assert json.loads(t)["tiers"][0]["bytes"] == 12345678
    d = uk.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN")
    with pytest.raises(uk.UnikernError):
        uk.solve(d, t)  # not even B and two shard pairs fit
