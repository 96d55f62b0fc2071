"""The `unikern` command line (reference src/main.cpp:276-736): its lines and exit codes.

CPU tests cover kml/hcs/solve/calibrate and the refusal paths; the GPU tests run and verify the
BASELINE configurations through the binary and the ledger.
"""
from __future__ import annotations

import json
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SAMPLES = ROOT / "samples"


def cli(uk, *args, cwd=None, timeout=300):
    assert uk.CLI.exists(), "the CLI is built with the library (python3 unikern_amd/build.py)"
    p = subprocess.run([str(uk.CLI), *map(str, args)], capture_output=True, text=True, cwd=cwd, timeout=timeout)
    return p.returncode, p.stdout, p.stderr


def test_usage_and_unknown_commands(uk):
    rc, out, err = cli(uk)
    assert rc == 2 and "usage: unikern" in err
    rc, _, err = cli(uk, "solve", "--kml", SAMPLES / "kml_softmax_4096.json")
    assert rc == 2 and "usage: unikern solve" in err  # --hcs is required, as in the reference


def test_kml_and_hcs(uk, tmp_path):
    rc, out, _ = cli(uk, "kml", SAMPLES / "kml_conv_nchw.json")
    assert rc == 0
    assert out.startswith("VALID  conv:fp32:56x56x64x3x3x64:NCHW:n8:p1:s1:cs")
    assert "ops=1849688064" in out and "COVER amd:hip primitive=covered" in out
    bad = tmp_path / "bad.json"
    bad.write_text('{"op": "gemm", "dtype": "fp32", "dims": [4, -4, 4]}')
    rc, _, err = cli(uk, "kml", bad)
    assert rc == 2 and "dims[1]=-4 must be positive" in err
    rc, out, _ = cli(uk, "hcs", SAMPLES / "hcs_mi355x.json")
    assert rc == 0 and f"hcs_fp={uk.hcs_fingerprint()}" in out
    rc, out2, _ = cli(uk, "hcs", "builtin")
    assert rc == 0 and out2 == out


@pytest.mark.parametrize("ledger", ["l.jsonl", "l.sqlite3"])
def test_solve_ledger_hit_and_selfcheck(uk, tmp_path, ledger):
    kml = SAMPLES / "kml_gemm_f16_4096.json"
    rc, out, _ = cli(uk, "solve", "--hcs", "builtin", "--kml", kml, "--ledger", ledger, "--selfcheck", cwd=tmp_path)
    assert rc == 0
    m = re.search(r"SOLVED  x\* tile=(\d+)x(\d+)  c_ms=(\S+)  \|X\|=(\d+)  hcs_fp=(\w{8})", out)
    assert m and m.group(5) == uk.hcs_fingerprint()[:8]
    assert "SELFCHECK OK (deterministic)" in out and "COVER amd:hip primitive=covered" in out
    rc, out2, _ = cli(uk, "solve", "--hcs", "builtin", "--kml", kml, "--ledger", ledger, cwd=tmp_path)
    assert rc == 0 and out2.startswith("LEDGER HIT  c_cached_ms=" + m.group(3))
    with uk.Ledger(tmp_path / ledger) as L:
        assert L.size()[0] == 1
        assert L.lookup(kml.read_text()).plan.key == uk.solve(uk.kml_load(kml)).plan.key


def test_solve_shorthand_matches_reference_surface(uk, tmp_path):
    rc, out, _ = cli(uk, "solve", "--hcs", "builtin", "--op", "reduce", "--dims", "1048576", "--ledger", "x.jsonl",
                     cwd=tmp_path)
    assert rc == 0 and "key=reduce1d" in out


def test_refusals(uk, tmp_path):
    unsupported = tmp_path / "u.json"
    unsupported.write_text('{"op": "softmax", "dtype": "fp16", "dims": [16, 16]}')
    rc, _, err = cli(uk, "solve", "--hcs", "builtin", "--kml", unsupported, "--ledger", "x.jsonl", cwd=tmp_path)
    assert rc == 2 and err.startswith("UNSUPPORTED:")
    rc, _, err = cli(uk, "run", "--hcs", "builtin", "--kml", unsupported, "--ledger", "x.jsonl", cwd=tmp_path)
    assert rc == 2 and err.startswith("UNSUPPORTED:")
    tiny = tmp_path / "tiny.json"
    h = json.loads((SAMPLES / "hcs_mi355x.json").read_text())
    h["tiers"][0]["bytes"] = 1 << 20
    tiny.write_text(json.dumps(h))
    rc, _, err = cli(uk, "solve", "--hcs", tiny, "--kml", SAMPLES / "kml_rmsnorm_4096.json", "--ledger", "x.jsonl",
                     cwd=tmp_path)
    assert rc == 3 and "INFEASIBLE" in err and "working_set<=device_capacity" in err
    rejected = tmp_path / "r.json"
    rejected.write_text('{"vendor": "amd"}')
    rc, _, err = cli(uk, "solve", "--hcs", rejected, "--kml", SAMPLES / "kml_gemm_f16_4096.json", cwd=tmp_path)
    assert rc == 2 and "HCS rejected" in err
    assert not (tmp_path / "x.jsonl").exists() or (tmp_path / "x.jsonl").read_text() == ""


def test_calibrate_without_rows(uk, tmp_path):
    rc, _, err = cli(uk, "calibrate", "--hcs", "builtin", "--ledger", "c.jsonl", cwd=tmp_path)
    assert rc == 3 and "CALIBRATE SKIP" in err


# ---------------------------------------------------------------------------------------------
# On the device


@pytest.mark.gpu
@pytest.mark.parametrize("sample", ["kml_rmsnorm_4096.json", "kml_gemm_f16_4096.json", "kml_conv_nchw.json",
                                    "kml_q8_0_m1_n4096.json"])
def test_run_commits_then_hits(gpu, tmp_path, sample):
    kml = SAMPLES / sample
    rc, out, err = cli(gpu, "run", "--hcs", "builtin", "--kml", kml, "--ledger", "l.sqlite3", "--iters", "10",
                       cwd=tmp_path)
    assert rc == 0, out + err
    assert "RUN amd:hip built=yes ran=yes verified=PASS" in out
    assert "UNIKERN_RESULT backend=amd verify=PASS" in out and "migrations=0" in out
    assert "LEDGER COMMIT predicted_ms=" in out
    rc, out2, err2 = cli(gpu, "verify", "--hcs", "builtin", "--kml", kml, "--ledger", "l.sqlite3", "--iters", "5",
                         cwd=tmp_path)
    assert rc == 0, out2 + err2
    assert "LEDGER HIT" in out2 and "(from ledger)" in out2 and "VERIFY PASS (no ledger write)" in out2
    with gpu.Ledger(tmp_path / "l.sqlite3") as L:
        hit = L.lookup(kml.read_text())
        assert hit.measured_ms > 0 and hit.kernel_ms > 0 and L.size() == (1, 0)


@pytest.mark.gpu
@pytest.mark.parametrize("sample", ["kml_q8_0_m1_n4096.json", "kml_q8_0_m16_n11008.json"])
def test_run_exact_mode_q8_0_is_bit_exact(gpu, tmp_path, sample):
    rc, out, err = cli(gpu, "run", "--hcs", "builtin", "--kml", SAMPLES / sample, "--iters", "5", "--exact",
                       cwd=tmp_path)
    assert rc == 0, out + err
    assert "verify=PASS" in out and " gate=bit_exact_mismatches err=0.000000e+00 " in out, out


@pytest.mark.gpu
def test_run_exact_mode_and_calibrate(gpu, tmp_path):
    kml = SAMPLES / "kml_softmax_4096.json"
    rc, out, err = cli(gpu, "run", "--hcs", SAMPLES / "hcs_mi355x.json", "--kml", kml, "--ledger", "c.jsonl",
                       "--iters", "10", cwd=tmp_path)
    assert rc == 0, out + err
    rc, out, err = cli(gpu, "run", "--hcs", SAMPLES / "hcs_mi355x.json", "--kml", SAMPLES / "kml_gemm_f16_4096.json",
                       "--ledger", "c.jsonl", "--iters", "5", "--exact", cwd=tmp_path)
    assert rc == 0 and "mode=resident" in out, out + err
    rc, out, err = cli(gpu, "calibrate", "--hcs", SAMPLES / "hcs_mi355x.json", "--ledger", "c.jsonl", "--out",
                       "cal.json", cwd=tmp_path)
    assert rc == 0, out + err
    cal = json.loads((tmp_path / "cal.json").read_text())
    assert cal["constants_version"] == 2 and cal["link_bw_gbps"] > 0
