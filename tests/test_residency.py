"""Residency, refusal and alarm paths of one run (reference src/codegen_hip.cpp:205-293,
src/runner.cpp:195-255, src/main.cpp:441-539), all on the CPU: the alarm criterion's boundary
table, the residency probe's exit classes, the payload refusals of uk_run (which return before any
input is generated or the device is touched), the parse of a program's result and refusal lines,
and the CLI's violation -> record -> re-solve -> retry flow over recorded program outputs.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest

from test_cli import cli

ROOT = Path(__file__).resolve().parent.parent
SAMPLES = ROOT / "samples"

# hipMemoryType (hip_runtime_api.h) and hipError_t values the probe can return.
MEM_UNREGISTERED, MEM_HOST, MEM_DEVICE, MEM_MANAGED, MEM_ARRAY, MEM_UNIFIED = 0, 1, 2, 3, 10, 11
HIP_SUCCESS, HIP_ERROR_INVALID_VALUE = 0, 1


# The boundary table of the reference's alarm criterion (tests/acceptance.cpp:2497-2513): each
# row pins one boundary, so a flipped comparison turns exactly one of them red.
@pytest.mark.parametrize("migrations,checks,threshold,violation", [
    (0, 6, 0.0, False),   # the clean device case
    (1, 6, 0.0, True),    # the default threshold alarms on one migration
    (1, 6, 0.2, False),   # 1/6 <= 0.2: relaxing is explicit
    (2, 6, 0.2, True),    # 2/6 > 0.2
    (1, 0, 0.9, True),    # a refusal has no denominator: worst rate 1.0
    (-1, 6, 0.0, False),  # a backend that never reports: unknown, not a zero
])
def test_migration_alarm_boundaries(uk, migrations, checks, threshold, violation):
    v, rate = uk.migration_alarm(migrations, checks, threshold)
    assert v == violation
    if migrations <= 0:
        assert rate == 0.0
    if migrations > 0 and checks == 0:
        assert rate == 1.0
    if migrations > 0 and checks > 0:
        assert rate == pytest.approx(migrations / checks) and 0.0 < rate <= 1.0


def test_migration_alarm_rate_equal_to_threshold_does_not_fire(uk):
    # strictly above the threshold: 2/8 == 0.25 stays quiet, 3/8 fires
    assert uk.migration_alarm(2, 8, 0.25) == (False, 0.25)
    assert uk.migration_alarm(3, 8, 0.25)[0]


@pytest.mark.parametrize("probe,mem,want", [
    (HIP_SUCCESS, MEM_DEVICE, 0),
    (HIP_SUCCESS, MEM_MANAGED, 5),       # managed memory is oversubscription
    (HIP_SUCCESS, MEM_HOST, 5),          # host-resident memory too
    (HIP_SUCCESS, MEM_UNREGISTERED, 5),
    (HIP_SUCCESS, MEM_UNIFIED, 5),
    (HIP_SUCCESS, MEM_ARRAY, 5),
    (HIP_ERROR_INVALID_VALUE, MEM_DEVICE, 4),  # a failed probe is a HIP failure, not residency
])
def test_residency_class(uk, probe, mem, want):
    assert uk.residency_class(probe, mem) == want


def _tiny_hcs(nbytes: int) -> str:
    h = json.loads((SAMPLES / "hcs_mi355x.json").read_text())
    h["tiers"][0]["bytes"] = nbytes
    return json.dumps(h)


def test_payload_refused_before_inputs_or_device(uk):
    # rmsnorm 4096 x 4096 moves 134,234,112 B. With a 150 MB device tier the solver finds it
    # feasible (it fits), but a run may occupy only 0.85 of the tier: uk_run refuses with exit
    # class 4 before generating inputs (so an oversized op cannot exhaust host memory) and before
    # touching the device (this runs on a machine without one).
    d = uk.make_desc("rmsnorm", [4096, 4096])
    hcs = _tiny_hcs(150_000_000)
    assert uk.solve(d, hcs).feasible >= 1
    r = uk.run(d, hcs_json=hcs)
    assert r.exit_code == uk.UK_HIP_FAILURE and r.built and not r.ran
    assert "UNIKERN_ERROR what=stream_refused payload_bytes=134234112 vram_bytes=150000000" in r.log
    assert r.checks == -1 and r.migrations == -1  # no allocation was probed
    # 0.85 boundary: 134,234,112 B fits a tier of ceil(134,234,112 / 0.85) B and is refused just below it.
    edge = math.ceil(134_234_112 / 0.85)
    assert "stream_refused" in uk.run(d, hcs_json=_tiny_hcs(edge - 2)).log
    assert "stream_refused" not in uk.run(d, hcs_json=_tiny_hcs(edge)).log  # stops later, at the device check
    # A caller-supplied resident GEMM plan bypasses the solver's streaming choice and is refused
    # the same way; the solver's own plan for that tier streams instead.
    g = uk.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN")
    r = uk.run(g, plan=uk.solve(g).plan, hcs_json=_tiny_hcs(100_000_000))
    assert "UNIKERN_ERROR what=stream_refused payload_bytes=100663296 vram_bytes=100000000" in r.log
    streamed = uk.solve(g, _tiny_hcs(100_000_000)).plan
    assert streamed.shard_rows > 0
    r = uk.run(g, plan=streamed, hcs_json=_tiny_hcs(100_000_000))
    assert "stream_refused" not in r.log  # B + two shard pairs fit; stops at the device check


def test_vram_unknown_refused_before_inputs_or_device(uk):
    # An HCS without a vram tier cannot decide residency (src/codegen_hip.cpp:209-215, the tier
    # read at :309): the run is refused with exit class 4 before any input is generated or the
    # device touched. The import accepts such a description only as unified memory (a "unified"
    # tier and no "vram" one, src/hcs.cpp:83-89); a caller-supplied plan gets past the solver.
    h = json.loads((SAMPLES / "hcs_mi355x.json").read_text())
    h["unified_memory"] = True
    h["tiers"] = [{"name": "unified", "bytes": 309237645312, "bw_gbps": 8000, "confidence": "official"}]
    d = uk.make_desc("rmsnorm", [4096, 4096])
    r = uk.run(d, plan=uk.solve(d).plan, hcs_json=json.dumps(h))
    assert r.exit_code == uk.UK_HIP_FAILURE and r.built and not r.ran
    assert "UNIKERN_ERROR what=vram_unknown" in r.log
    assert (r.checks, r.migrations, r.cpu_ms) == (-1, -1, -1.0)  # nothing probed, no CPU pass


def test_streamed_plan_refused_when_shards_do_not_fit(uk):
    g = uk.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN")
    p = uk.solve(g, _tiny_hcs(100_000_000)).plan
    r = uk.run(g, plan=p, hcs_json=_tiny_hcs(40_000_000))
    assert r.exit_code == uk.UK_HIP_FAILURE and "UNIKERN_ERROR what=stream_refused device_bytes=" in r.log
    # Only the MFMA GEMMs stream.
    q = uk.make_desc("rmsnorm", [4096, 4096])
    qp = uk.solve(q).plan
    qp.shard_rows = 256
    assert uk.run(q, plan=qp).exit_code == uk.UK_BAD_INVOCATION


def test_parse_result_line(uk):
    line = ("UNIKERN_RESULT backend=amd verify=PASS max_rel=1.5e-06 measured_ms=2.5 kernel_ms=0.024 mode=resident "
            "payload_mb=128.0 perf=4096x4096 dtype=fp32 migrations=0 checks=20 vram_free=305000000000 "
            "vram_total=309237645312 gate=max_rel err=1.5e-06 tol=1e-05 achieved=5600.0 unit=GB/s peak=8000.0 "
            "frac=0.7000 plan=rows:tpr=256,nv=4,nt,rpb=2")
    r = uk.parse_result("offload noise\n" + line + "\ntrailing\n", 0)
    assert r.verified and r.ran and r.built and r.exit_code == 0
    assert (r.max_rel, r.measured_ms, r.kernel_ms) == (1.5e-06, 2.5, 0.024)
    assert (r.migrations, r.checks, r.vram_free, r.vram_total) == (0, 20, 305000000000, 309237645312)
    assert r.plan_key == "rows:tpr=256,nv=4,nt,rpb=2" and r.frac == 0.7 and r.bound == "hbm"
    # A library result line round-trips through its own formatter.
    again = uk.parse_result(r.line, 0)
    assert (again.verified, again.kernel_ms, again.checks, again.plan_key) == (True, 0.024, 20, r.plan_key)
    assert (again.cpu_ms, again.cpu_cores, again.cpu_outputs) == (-1.0, -1, -1)
    # Absent residency and CPU tokens keep the -1 sentinels; a FAIL verdict is not verified.
    r = uk.parse_result("UNIKERN_RESULT backend=amd verify=FAIL max_rel=0.5 measured_ms=1 kernel_ms=0.5", 1)
    assert not r.verified and (r.migrations, r.checks) == (-1, -1) and r.exit_code == 1
    assert (r.cpu_ms, r.cpu_cores, r.cpu_outputs) == (-1.0, -1, -1)


def test_result_line_carries_cpu_tokens(uk):
    # The CPU reference pass beside the device time: cpu_ms= and cpu_cores= (plus how many
    # outputs that pass computed) are formatted and parsed back.
    line = ("UNIKERN_RESULT backend=amd verify=PASS max_rel=1e-07 measured_ms=3.0 kernel_ms=0.1 mode=resident "
            "payload_mb=96.0 perf=4096x4096x4096 dtype=fp16 migrations=0 checks=3 vram_free=1 vram_total=2 "
            "gate=frobenius err=2e-04 tol=1e-02 achieved=1356.000 unit=TFLOP/s peak=2516.6 frac=0.5389 "
            "plan=gemm_f16:256x256x64 cpu_ms=812.500 cpu_cores=16 cpu_outputs=131072")
    r = uk.parse_result(line, 0)
    assert (r.cpu_ms, r.cpu_cores, r.cpu_outputs) == (812.5, 16, 131072)
    again = uk.parse_result(r.line, 0)
    assert (again.cpu_ms, again.cpu_cores, again.cpu_outputs) == (812.5, 16, 131072)
    assert " cpu_ms=812.500 cpu_cores=16 cpu_outputs=131072" in r.line


def test_result_line_carries_the_stream_path(uk):
    # A streamed run names its data path after mode= (the reference's stream_path= token,
    # src/codegen_hip.cpp:1716); a resident line has none and parses to "".
    line = ("UNIKERN_RESULT backend=amd verify=PASS max_rel=0 measured_ms=90.0 kernel_ms=0.3 mode=streamed "
            "stream_path=mmap payload_mb=96.0 perf=4096x4096x4096 dtype=fp16 migrations=0 checks=5")
    r = uk.parse_result(line, 0)
    assert r.stream_path == "mmap" and " mode=streamed stream_path=mmap payload_mb=" in r.line
    assert uk.parse_result(r.line, 0).stream_path == "mmap"
    r = uk.parse_result(line.replace("mode=streamed stream_path=mmap", "mode=resident"), 0)
    assert r.stream_path == "" and "stream_path=" not in r.line


def test_stream_path_pin_is_validated_before_the_device(uk, monkeypatch):
    # UK_GEMM_STREAM_PATH pins scenario B's data path for A/B runs (pinned | mmap | auto); any
    # other value is refused with class 2 before inputs or the device are touched, as the
    # reference's program refuses it (src/codegen_hip.cpp:1344-1356).
    g = uk.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN")
    small = _tiny_hcs(96 << 20)
    monkeypatch.setenv("UK_GEMM_STREAM_PATH", "zero-copy")
    r = uk.run(g, hcs_json=small)
    assert r.exit_code == uk.UK_BAD_INVOCATION and "UNIKERN_ERROR what=stream_path_pin_unfit val=zero-copy" in r.log
    assert r.cpu_ms == -1.0  # refused before the inputs and their CPU pass
    # A resident run does not stream, so the knob is not consulted.
    assert "stream_path_pin_unfit" not in uk.run(uk.make_desc("gemm", [256, 256, 256], dtype="fp16", layout="TN"),
                                                 hcs_json=small).log
    for ok in ("pinned", "mmap", "auto"):
        monkeypatch.setenv("UK_GEMM_STREAM_PATH", ok)
        assert "stream_path_pin_unfit" not in uk.run(g, hcs_json=small).log


def test_stream_gemm_file_refuses_a_short_or_missing_file(uk, tmp_path):
    d = uk.make_desc("gemm", [64, 64, 64], dtype="fp16", layout="TN")
    B = np.zeros((64, 64), np.uint16)
    with pytest.raises(uk.UnikernError) as e:
        uk.stream_gemm_file(d, tmp_path / "absent.bin", B)
    assert e.value.code == uk.UK_BAD_INVOCATION and "mmap_open" in str(e.value)
    short = tmp_path / "short.bin"
    short.write_bytes(b"\0" * (64 * 64 * 2 - 2))
    with pytest.raises(uk.UnikernError) as e:
        uk.stream_gemm_file(d, short, B)
    assert e.value.code == uk.UK_BAD_INVOCATION and "mmap_short_file need=8192 have=8190" in str(e.value)
    with pytest.raises(uk.UnikernError) as e:
        uk.stream_gemm_file(d, short, np.zeros((64, 64), np.float32))
    assert e.value.code == uk.UK_BAD_INVOCATION and "stream_gemm_file:" in str(e.value)


def test_parse_refusal_line(uk):
    # No result line: the oversubscription refusal still carries the rate's numerator and
    # denominator and the measured headroom (src/runner.cpp:199-214).
    out = ("UNIKERN_ERROR what=oversubscription ptr=in type=3 migrations=1 checks=4 vram_free=8407547904 "
           "vram_total=17163091968\n")
    r = uk.parse_result(out, 5)
    assert (r.migrations, r.checks, r.vram_free, r.vram_total, r.exit_code) == (1, 4, 8407547904, 17163091968, 5)
    assert not r.verified
    with pytest.raises(uk.UnikernError):
        uk.parse_result("compile failed\n", 4)


# ---------------------------------------------------------------------------------------------
# The CLI's residency flow (src/main.cpp:441-569) over recorded program outputs.

OK_LINE = ("UNIKERN_RESULT backend=amd verify=PASS max_rel=0 measured_ms=0.9 kernel_ms=0.12 mode=resident "
           "migrations=0 checks=20 vram_free=300000000000 vram_total=309237645312 plan=x")


def _outcomes(tmp_path, *blocks):
    f = tmp_path / "outcomes.txt"
    f.write_text("".join(f"#exit {code}\n{text}\n" for code, text in blocks))
    return f


def _run(uk, tmp_path, outcomes, *extra, ledger="l.jsonl"):
    return cli(uk, "run", "--hcs", "builtin", "--kml", SAMPLES / "kml_gemm_f16_4096.json", "--ledger", ledger,
               "--outcomes", outcomes, *extra, cwd=tmp_path)


@pytest.mark.parametrize("ledger", ["l.jsonl", "l.sqlite3"])
def test_cli_violation_resolve_commit(uk, tmp_path, ledger):
    # First run: one managed allocation of six probed (rate 1/6 > threshold 0) -> violation
    # recorded, re-solve on the measured free capacity, retry clean -> commit under the
    # tightened HCS, exit 0.
    viol = OK_LINE.replace("migrations=0 checks=20 vram_free=300000000000", "migrations=1 checks=6 vram_free=8407547904")
    f = _outcomes(tmp_path, (0, viol), (0, OK_LINE))
    rc, out, err = _run(uk, tmp_path, f, ledger=ledger)
    assert rc == 0, out + err
    assert "UNIKERN_VIOLATION what=migration_rate rate=0.166667 threshold=0 migrations=1 checks=6 exit=0" in out
    assert "RESOLVE re-solve device_capacity -> 8407547904" in out
    assert "LEDGER COMMIT" in out
    tight = uk.hcs_with_capacity(None, 8407547904)
    kml = (SAMPLES / "kml_gemm_f16_4096.json").read_text()
    with uk.Ledger(tmp_path / ledger) as L:
        assert L.size() == (1, 1)  # one solution (under the tightened HCS), one violation event
        assert L.lookup(kml) is None and L.lookup(kml, tight) is not None


def test_cli_pinned_arm_is_not_committed(uk, tmp_path):
    # A run whose executed data path is not the plan's (UK_GEMM_STREAM_PATH pinned an experiment
    # arm) verifies but lands in no ledger row (reference src/main.cpp:544-556): the plan here
    # takes the pinned path, the recorded run says it ran the mapped one.
    arm = OK_LINE.replace("mode=resident", "mode=streamed stream_path=mmap")
    rc, out, err = _run(uk, tmp_path, _outcomes(tmp_path, (0, arm)))
    assert rc == 0, out + err
    assert "LEDGER SKIP reason=env_path_pin executed=mmap planned=pinned" in out and "LEDGER COMMIT" not in out
    with uk.Ledger(tmp_path / "l.jsonl") as L:
        assert L.size() == (0, 0)
    # The plan's own path commits.
    same = OK_LINE.replace("mode=resident", "mode=streamed stream_path=pinned")
    rc, out, err = _run(uk, tmp_path, _outcomes(tmp_path, (0, same)))
    assert rc == 0 and "LEDGER COMMIT" in out and "LEDGER SKIP" not in out, out + err


def test_cli_refusal_without_denominator(uk, tmp_path):
    # The guard's own refusal (exit 5, no result line): rate 1.0, re-solve, retry clean.
    refusal = ("UNIKERN_ERROR what=oversubscription ptr=in type=3 migrations=1 checks=0 vram_free=8407547904 "
               "vram_total=17163091968")
    f = _outcomes(tmp_path, (5, refusal), (0, OK_LINE))
    rc, out, err = _run(uk, tmp_path, f, "--migration-threshold", "0.9")
    assert rc == 0, out + err
    assert "UNIKERN_VIOLATION what=migration_rate rate=1 threshold=0.9 migrations=1 checks=0 exit=5" in out


def test_cli_retry_still_violates(uk, tmp_path):
    viol = OK_LINE.replace("migrations=0 checks=20", "migrations=2 checks=6")
    f = _outcomes(tmp_path, (0, viol), (0, viol))
    rc, out, err = _run(uk, tmp_path, f, "--migration-threshold", "0.2")
    assert rc == 5
    assert "UNIKERN_VIOLATION stage=retry" in out and "one retry is the bound" in err
    with uk.Ledger(tmp_path / "l.jsonl") as L:
        assert L.size() == (0, 2)  # two violation events, no solution row


def test_cli_no_measured_capacity_stops(uk, tmp_path):
    viol = OK_LINE.replace("migrations=0 checks=20 vram_free=300000000000", "migrations=1 checks=6 vram_free=0")
    f = _outcomes(tmp_path, (0, viol))
    rc, out, err = _run(uk, tmp_path, f)
    assert rc == 5 and "RESOLVE STOP: no measured device capacity" in err
    with uk.Ledger(tmp_path / "l.jsonl") as L:
        assert L.size() == (0, 1)


def test_cli_relaxed_threshold_commits_without_resolve(uk, tmp_path):
    viol = OK_LINE.replace("migrations=0 checks=20", "migrations=1 checks=6")
    f = _outcomes(tmp_path, (0, viol))
    rc, out, err = _run(uk, tmp_path, f, "--migration-threshold", "0.2")
    assert rc == 0 and "UNIKERN_VIOLATION" not in out and "LEDGER COMMIT" in out


def test_cli_verify_failure_not_committed(uk, tmp_path):
    f = _outcomes(tmp_path, (1, OK_LINE.replace("verify=PASS", "verify=FAIL")))
    rc, out, err = _run(uk, tmp_path, f)
    assert rc == 1 and "RUN FAILED; solution NOT committed" in err
    with uk.Ledger(tmp_path / "l.jsonl") as L:
        assert L.size() == (0, 0)


@pytest.mark.parametrize("bad", ["nan", "-1", "abc"])
def test_cli_threshold_validated_at_parse(uk, tmp_path, bad):
    f = _outcomes(tmp_path, (0, OK_LINE))
    rc, _, err = _run(uk, tmp_path, f, "--migration-threshold", bad)
    assert rc == 2 and "--migration-threshold must be a number >= 0" in err
    assert not (tmp_path / "l.jsonl").exists()


def test_stream_gemm_checks_operands_before_the_call(uk):
    # uk_stream_gemm copies rows straight out of the host arrays, so a short or mistyped array is
    # refused on the Python side before the library (or the device) is reached.
    d = uk.make_desc("gemm", [256, 128, 64], dtype="fp16", layout="TN")
    A = np.zeros((256, 64), np.uint16)
    B = np.zeros((128, 64), np.uint16)
    for a, b in ((A[:255], B), (A, B[:, :63]), (A.astype(np.float32), B), (A, np.zeros((64, 128), np.uint16))):
        with pytest.raises(uk.UnikernError) as e:
            uk.stream_gemm(d, a, b)
        assert e.value.code == uk.UK_BAD_INVOCATION and "stream_gemm:" in str(e.value)
    with pytest.raises(uk.UnikernError):
        uk.stream_gemm(uk.make_desc("softmax", [16, 16]), A, B)
