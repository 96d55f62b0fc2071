"""Scenario B on the device: the GEMM streamed in M-shards through pinned host memory (reference
src/codegen_hip.cpp:1143-1238 uk_stream_pass, :1480-1708), with B resident, and its mapped path (A
read from a file into host-mapped staging that the kernel reads, :1239-1326).

On an MI355X (288 GB) no BASELINE GEMM exceeds the device tier, so these tests give the solver an
HCS with a small device tier; the pass then really shards. Every output row is computed by the same
kernel variant over the same k order as in a resident launch, so a streamed result must equal the
resident one bit for bit; it is also checked against the oracle (Frobenius 1e-3 for f16 with f32
accumulation, binary32-exact on sawtooth inputs).
"""
import json
from pathlib import Path

import numpy as np
import pytest

import _oracle as O

from test_cli import cli

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
SAMPLES = ROOT / "samples"


def tier(nbytes: int) -> str:
    h = json.loads((SAMPLES / "hcs_mi355x.json").read_text())
    h["tiers"][0]["bytes"] = nbytes
    return json.dumps(h)


def resident_gemm(uk, d, A, B, out_dtype):
    ab, bb = uk.DeviceBuffer.from_array(A), uk.DeviceBuffer.from_array(B)
    M, N = int(d.dims[0]), int(d.dims[1])
    cb = uk.DeviceBuffer(M * N * np.dtype(out_dtype).itemsize)
    uk.launch(d, [ab, bb], cb, plan=uk.solve(d).plan)
    return cb.download(out_dtype, (M, N))


@pytest.mark.parametrize("M,N,K,cap", [(4096, 4096, 4096, 96 << 20), (3328, 2048, 1024, 24 << 20)])
def test_stream_f16_matches_resident_bitwise(gpu, M, N, K, cap):
    d = gpu.make_desc("gemm", [M, N, K], dtype="fp16", layout="TN")
    plan = gpu.solve(d, tier(cap)).plan
    assert 0 < plan.shard_rows < M  # at least two shards; (3328, ...) ends on a shorter one
    A = O.f16_bits(O.uniform(M * K, 500 + M, -1.0, 1.0)).reshape(M, K)
    B = O.f16_bits(O.uniform(N * K, 501 + N, -1.0, 1.0)).reshape(N, K)
    Cs, ms = gpu.stream_gemm(d, A, B, plan=plan)
    assert ms > 0
    Cr = resident_gemm(gpu, d, A, B, np.uint16)
    assert np.array_equal(Cs, Cr)
    rows = np.array([0, 1, plan.shard_rows - 1, plan.shard_rows, M // 2, M - 1])
    R = O.gemm_f16q(A[rows], B, True)
    g, r = O.f16_to_f32(Cs[rows]).astype(np.float64), R.astype(np.float64)
    assert np.linalg.norm(g - r) / np.linalg.norm(r) <= 1e-3


def test_stream_f32_nt_matches_resident_and_oracle(gpu):
    M = N = K = 1024
    d = gpu.make_desc("gemm", [M, N, K])
    plan = gpu.solve(d, tier(12 << 20)).plan
    assert plan.shard_rows > 0 and plan.shard_rows % 64 == 0 and M // plan.shard_rows >= 2
    A = O.uniform(M * K, 20261201, -1.0, 1.0).reshape(M, K)
    B = O.uniform(K * N, 20261202, -1.0, 1.0).reshape(K, N)
    Cs, _ = gpu.stream_gemm(d, A, B, plan=plan)
    assert np.array_equal(Cs.view(np.uint32), resident_gemm(gpu, d, A, B, np.float32).view(np.uint32))
    R = O.gemm_f32(A, B, False)
    assert np.linalg.norm(Cs.astype(np.float64) - R) / np.linalg.norm(R.astype(np.float64)) <= 1e-5


def test_stream_without_plan_is_one_shard(gpu):
    # No plan and the built-in description: everything fits, one shard (upload, run, download).
    M, N, K = 512, 768, 256
    d = gpu.make_desc("gemm", [M, N, K], dtype="fp16", layout="TN")
    A = O.f16_bits(O.uniform(M * K, 7, -1.0, 1.0)).reshape(M, K)
    B = O.f16_bits(O.uniform(N * K, 8, -1.0, 1.0)).reshape(N, K)
    Cs, _ = gpu.stream_gemm(d, A, B)
    assert np.array_equal(Cs, resident_gemm(gpu, d, A, B, np.uint16))


def test_run_streamed_mode_verifies(gpu):
    # uk_run under a 96 MiB device tier: the solver's plan streams; the verified pass is streamed,
    # measured_ms is a whole pass and kernel_ms the shards' kernels.
    d = gpu.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN")
    hcs = tier(96 << 20)
    r = gpu.run(d, hcs_json=hcs, iters=5)
    assert r.exit_code == 0 and r.verified, r.log
    assert "mode=streamed" in r.line and "UNIKERN_INFO mode=streamed shards=" in r.log
    assert r.raw.plan.shard_rows > 0 and r.err_metric <= 1e-2
    assert r.measured_ms > r.kernel_ms > 0
    r = gpu.run(gpu.make_desc("gemm", [1024, 1024, 1024], dtype="fp16", layout="TN"), hcs_json=tier(6 << 20),
                exact=True, iters=3)
    assert r.exit_code == 0 and r.verified and r.err_metric == 0 and "mode=streamed" in r.line, r.log


def test_stream_file_f32_matches_resident_and_pinned(gpu, tmp_path):
    # The mapped path (reference src/codegen_hip.cpp:1239-1326): A's shards are read from a file
    # into host-mapped staging and the kernel reads them there. Same kernel, same k order: the
    # result equals the resident launch's and the pinned stream's bit for bit.
    M = N = K = 1024
    d = gpu.make_desc("gemm", [M, N, K])
    plan = gpu.solve(d, tier(12 << 20)).plan
    assert plan.shard_rows > 0 and M // plan.shard_rows >= 2
    A = O.uniform(M * K, 20261203, -1.0, 1.0).reshape(M, K)
    B = O.uniform(K * N, 20261204, -1.0, 1.0).reshape(K, N)
    path = tmp_path / "a_f32.bin"
    A.tofile(path)
    Cm, ms = gpu.stream_gemm_file(d, path, B, plan=plan)
    assert ms > 0
    Cp, _ = gpu.stream_gemm(d, A, B, plan=plan)
    assert np.array_equal(Cm.view(np.uint32), Cp.view(np.uint32))
    assert np.array_equal(Cm.view(np.uint32), resident_gemm(gpu, d, A, B, np.float32).view(np.uint32))


@pytest.mark.parametrize("M,N,K,cap", [(3328, 2048, 1024, 24 << 20), (512, 768, 256, 1 << 30)])
def test_stream_file_f16_matches_resident_bitwise(gpu, tmp_path, M, N, K, cap):
    # (3328, ...) ends on a shorter shard; (512, ...) fits and runs as one shard. The file holds
    # more than M K elements (a trailing row): only the first M K are read.
    d = gpu.make_desc("gemm", [M, N, K], dtype="fp16", layout="TN")
    plan = gpu.solve(d, tier(cap)).plan
    A = O.f16_bits(O.uniform(M * K, 600 + M, -1.0, 1.0)).reshape(M, K)
    B = O.f16_bits(O.uniform(N * K, 601 + N, -1.0, 1.0)).reshape(N, K)
    path = tmp_path / "a_f16.bin"
    np.concatenate([A, np.full((1, K), 0x7C00, np.uint16)]).tofile(path)
    Cm, _ = gpu.stream_gemm_file(d, path, B, plan=plan if plan.shard_rows > 0 else None)
    assert np.array_equal(Cm, resident_gemm(gpu, d, A, B, np.uint16))


def test_run_streamed_mapped_path_verifies(gpu, monkeypatch):
    # uk_run takes the plan's path unless UK_GEMM_STREAM_PATH pins one; the result line and the
    # log say which ran and where the choice came from.
    d = gpu.make_desc("gemm", [2048, 2048, 2048], dtype="fp16", layout="TN")
    hcs = tier(24 << 20)
    r = gpu.run(d, hcs_json=hcs, iters=3)
    assert r.exit_code == 0 and r.verified and r.stream_path == "pinned", r.log
    assert "stream_path=pinned source=plan plan=pinned" in r.log
    monkeypatch.setenv("UK_GEMM_STREAM_PATH", "mmap")
    r = gpu.run(d, hcs_json=hcs, iters=3)
    assert r.exit_code == 0 and r.verified and r.stream_path == "mmap", r.log
    assert "mode=streamed stream_path=mmap" in r.line and "stream_path=mmap source=env plan=pinned" in r.log
    assert r.err_metric <= 1e-2 and r.measured_ms > 0 and r.kernel_ms > 0
    r = gpu.run(gpu.make_desc("gemm", [1024, 1024, 1024]), hcs_json=tier(12 << 20), exact=True, iters=3)
    assert r.exit_code == 0 and r.verified and r.err_metric == 0 and r.stream_path == "mmap", r.log


def test_cli_streamed_run_commits_and_hits(gpu, tmp_path):
    hcs = tmp_path / "small.json"
    hcs.write_text(tier(96 << 20))
    kml = SAMPLES / "kml_gemm_f16_4096.json"
    rc, out, err = cli(gpu, "run", "--hcs", hcs, "--kml", kml, "--ledger", "s.jsonl", "--iters", "3", cwd=tmp_path)
    assert rc == 0, out + err
    assert "mode=streamed" in out and "LEDGER COMMIT" in out
    rc, out, err = cli(gpu, "verify", "--hcs", hcs, "--kml", kml, "--ledger", "s.jsonl", "--iters", "3", cwd=tmp_path)
    assert rc == 0 and "LEDGER HIT" in out and "+stream" in out and "mode=streamed" in out, out + err
