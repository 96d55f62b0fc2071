"""uk_run end to end (the emitted-program contract: seeded inputs, verified launch, timing,
UNIKERN_RESULT line) on the BASELINE configurations, through the C ABI."""
import pytest



def _ok(r):
    assert r.exit_code == 0, r.log
    assert r.built and r.ran and r.verified, r.log
    assert r.migrations == 0 and r.checks > 0
    assert r.kernel_ms > 0 and r.measured_ms >= r.kernel_ms
    assert r.line.startswith("UNIKERN_RESULT backend=amd verify=PASS")
    # the run's own CPU reference pass is reported beside the device time (cpu_ms=, cpu_cores=)
    assert r.cpu_ms >= 0 and r.cpu_cores >= 1 and r.cpu_outputs > 0
    assert f" cpu_cores={r.cpu_cores} " in r.line and " cpu_ms=" in r.line


def _tracks_prediction(r):
    # Reported here; bounded in test_cost_model_tracks_measured_time (perf marker): a slower or
    # faster box moves the ratio without any result changing.
    ratio = r.kernel_ms * 1e3 / r.raw.plan.predicted_us
    print(f"{r.plan_key}: measured {r.kernel_ms * 1e3:.2f} us, predicted {r.raw.plan.predicted_us:.2f} us ({ratio:.2f}x)")
    return ratio


@pytest.mark.gpu
@pytest.mark.parametrize("op", ["reduce", "rmsnorm", "softmax"])
def test_run_reduction_family_config(gpu, op):
    r = gpu.run(gpu.make_desc(op, [4096, 4096]), iters=20)
    _ok(r)
    assert r.bound == "hbm" and r.peak == 8000.0
    _tracks_prediction(r)
    print(r.line)


@pytest.mark.gpu
@pytest.mark.parametrize("op", ["reduce", "rmsnorm", "softmax", "channelscale"])
def test_run_reference_sample_shapes_exact_mode(gpu, op):
    # samples/kml_{softmax,rmsnorm,channelscale}.json shape, the reference's sawtooth inputs.
    r = gpu.run(gpu.make_desc(op, [65536, 256]), exact=True, iters=10)
    _ok(r)


@pytest.mark.gpu
def test_run_gemm_f16_config(gpu):
    r = gpu.run(gpu.make_desc("gemm", [4096, 4096, 4096], dtype="fp16", layout="TN"), iters=10)
    _ok(r)
    assert r.bound == "mfma" and r.err_metric <= 1e-2
    _tracks_prediction(r)
    print(r.line)


@pytest.mark.gpu
def test_run_gemm_f16_exact_mode_bit_exact(gpu):
    r = gpu.run(gpu.make_desc("gemm", [1024, 1024, 1024], dtype="fp16", layout="TN"), exact=True, iters=5)
    _ok(r)
    assert r.err_metric == 0  # bit-exact mismatches


@pytest.mark.gpu
def test_run_reference_gemm_samples(gpu):
    # samples/kml_gemm.json (fp32 512^3 NT) and kml_gemm_f16.json (fp16 512^3 NT), exact mode.
    for dt in ("fp32", "fp16"):
        r = gpu.run(gpu.make_desc("gemm", [512, 512, 512], dtype=dt), exact=True, iters=5)
        _ok(r)
        assert r.err_metric == 0


@pytest.mark.gpu
def test_run_reduce1d_sample(gpu):
    r = gpu.run(gpu.make_desc("reduce", [4194304]), iters=20)
    _ok(r)


@pytest.mark.gpu
def test_run_refuses_unsupported(gpu):
    r = gpu.run(gpu.make_desc("softmax", [16, 16], dtype="fp16"))
    assert r.exit_code == 2 and not r.ran
    assert "op_unsupported" in r.log


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 8, 16])
@pytest.mark.parametrize("N", [4096, 11008])
def test_run_q8_0_configs(gpu, M, N):
    r = gpu.run(gpu.make_desc("gemm", [M, N, 4096], dtype="q8_0", layout="TN"), iters=50)
    _ok(r)
    assert r.bound == "hbm" and r.raw.weight_bytes == N * 128 * 34
    _tracks_prediction(r)
    print(r.line)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 16])
def test_run_q8_0_exact_mode_bit_exact(gpu, M):
    # Small-integer activations and power-of-two scales keep every partial sum exact in f32,
    # so the MFMA tile kernel (M = 16) and the one-row kernel (M = 1) must match bit for bit.
    r = gpu.run(gpu.make_desc("gemm", [M, 4096, 4096], dtype="q8_0", layout="TN"), exact=True, iters=5)
    _ok(r)
    assert r.err_metric == 0 and "bit_exact" in r.line


@pytest.mark.gpu
def test_run_conv_config(gpu):
    d = gpu.make_desc("conv", [56, 56, 64, 3, 3, 64], layout="NCHW", batch=8, pad=1, epilogue="channelscale")
    r = gpu.run(d, iters=20)
    _ok(r)
    assert r.bound == "mfma" and r.err_metric <= 1e-5
    _tracks_prediction(r)
    print(r.line)
    r = gpu.run(d, exact=True, iters=5)
    _ok(r)
    assert r.err_metric == 0


@pytest.mark.gpu
def test_run_reference_conv_sample(gpu):
    r = gpu.run(gpu.make_desc("conv", [64, 64, 32, 3, 3, 64]), exact=True, iters=5)
    _ok(r)
    assert r.err_metric == 0


# The solver's cost model against measured time at the BASELINE shapes (it is fitted there; the
# box-to-box range is 0.82-1.19x). The window is loose on purpose, so a broken price or
# calibration constant fails while box-to-box variation does not.
COST_SHAPES = [
    ("rmsnorm", [4096, 4096], {}),
    ("softmax", [4096, 4096], {}),
    ("reduce", [4096, 4096], {}),
    ("gemm", [4096, 4096, 4096], dict(dtype="fp16", layout="TN")),
    ("gemm", [1, 4096, 4096], dict(dtype="q8_0", layout="TN")),
    ("gemm", [16, 11008, 4096], dict(dtype="q8_0", layout="TN")),
    ("conv", [56, 56, 64, 3, 3, 64], dict(layout="NCHW", batch=8, pad=1, epilogue="channelscale")),
]


@pytest.mark.perf
@pytest.mark.parametrize("op,dims,kw", COST_SHAPES, ids=[f"{o}-{'x'.join(map(str, d))}" for o, d, _ in COST_SHAPES])
def test_cost_model_tracks_measured_time(gpu, op, dims, kw):
    r = gpu.run(gpu.make_desc(op, dims, **kw), iters=20)
    _ok(r)
    assert 0.5 <= _tracks_prediction(r) <= 2.0
