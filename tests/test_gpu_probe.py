"""The matrix-core ceiling probe (uk_probe_mfma) through the C ABI: the sustained f16 MFMA rate,
the shader clock under that load and the issue interval of both MFMA forms. The gpu test checks
what holds on any box (the rate follows from the launch time, never above the dense peak); the
perf test checks the clock and issue windows against the part's published limits (2516.6 dense
f16 TFLOP/s at 2.4 GHz; on one SIMD 16 cycles per v_mfma_f32_16x16x32_f16 and 32 per
v_mfma_f32_32x32x16_f16), which a throttled box could leave."""
import pytest


@pytest.fixture(scope="module")
def probe(gpu):
    r = gpu.probe_mfma()
    print(r)
    return r


@pytest.mark.gpu
def test_mfma_probe(gpu, probe):
    r = probe
    cus = gpu.device_props()["compute_units"]
    assert r["workgroups"] == cus and r["mfmas_per_wave"] == 8 * 16384
    # the rate follows from the launch time (2^17 flops per wavefront per loop iteration)
    flops = r["workgroups"] * 4 * 16384 * 131072
    assert r["tflops"] == pytest.approx(flops / (r["ms_per_launch"] * 1e-3) / 1e12, rel=1e-9)
    for sfx in ("", "_32x32"):
        # positive, and never above the dense peak
        assert 0 < r["tflops" + sfx] <= 2516.6 * 1.001
        assert r["clock_ghz" + sfx] > 0 and r["cycles_per_mfma" + sfx] > 0


@pytest.mark.perf
def test_mfma_probe_windows(gpu, probe):
    r = probe
    cus = gpu.device_props()["compute_units"]
    for sfx, flop_per_mfma, cyc in (("", 16384, 16), ("_32x32", 32768, 32)):
        tflops, clock, cpm = r["tflops" + sfx], r["clock_ghz" + sfx], r["cycles_per_mfma" + sfx]
        assert 300 < tflops
        assert 0.5 < clock <= 2.45
        # one wavefront per SIMD issues back to back
        assert cyc - 0.5 < cpm < 1.5 * cyc
        # rate = CUs x 4 SIMDs x flops per MFMA x clock / cycles per MFMA (within the loop's
        # share of the launch)
        implied = cus * 4 * flop_per_mfma * clock * 1e9 / cpm / 1e12
        assert 0.8 * implied < tflops <= 1.02 * implied
