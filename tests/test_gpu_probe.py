"""The matrix-core ceiling probe (uk_probe_mfma) through the C ABI: the sustained f16 MFMA rate,
the shader clock under that load and the issue interval, checked for internal consistency and
against the part's published limits (2516.6 dense f16 TFLOP/s at 2.4 GHz, 32 cycles per
v_mfma_f32_32x32x16_f16 on one SIMD)."""
import pytest

pytestmark = pytest.mark.gpu


def test_mfma_probe(gpu):
    r = gpu.probe_mfma()
    print(r)
    cus = gpu.device_props()["compute_units"]
    assert r["workgroups"] == cus and r["mfmas_per_wave"] == 4 * 16384
    # the rate follows from the launch time
    flops = r["workgroups"] * 4 * r["mfmas_per_wave"] * 32768
    assert r["tflops"] == pytest.approx(flops / (r["ms_per_launch"] * 1e-3) / 1e12, rel=1e-9)
    # never above the dense peak; one wavefront per SIMD issues back to back at 32 cycles
    assert 300 < r["tflops"] <= 2516.6 * 1.001
    assert 0.5 < r["clock_ghz"] <= 2.45
    assert 31.5 < r["cycles_per_mfma"] < 40
    # rate = CUs x 4 SIMDs x 16384 flop per MFMA x clock / cycles per MFMA (within the loop's
    # share of the launch)
    implied = cus * 4 * 32768 * r["clock_ghz"] * 1e9 / r["cycles_per_mfma"] / 1e12
    assert 0.8 * implied < r["tflops"] <= 1.02 * implied
