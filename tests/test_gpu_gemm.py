"""Parity of the MFMA GEMMs against the CPU oracle, through the C ABI.

Gates: f16 GEMM ||C - R||_F / ||R||_F <= 1e-2 (north star) where R is the reference's f16
program loop (f32 accumulate over the f16-rounded inputs, src/codegen_hip.cpp:1814-1822); in
exact mode (the reference's sawtooth inputs, every partial sum exact) the f16 output must equal
the round-to-nearest-even of R bit for bit. f32 GEMM: Frobenius <= 1e-5, exact mode bit-exact.
"""
import numpy as np
import pytest

import _oracle as O

pytestmark = pytest.mark.gpu

# (BM, BN, BK) of every compiled f16 TN variant, in table order; 10-11 and 14-15 are the ping-pong
# kernel (two LDS swizzles), 12-13 the four-wavefront 128x128-wave-tile kernel (four and five
# ring stages), 16 its v_mfma_f32_16x16x32_f16 form, 17 its 64-deep form and 18 that on
# v_mfma_f32_16x16x32_f16.
F16_VARIANTS = [(256, 256, 32), (256, 256, 32), (256, 256, 32), (256, 256, 32), (256, 128, 32), (256, 128, 64),
                (128, 128, 64), (128, 128, 32), (256, 256, 32), (256, 256, 32), (256, 256, 32), (256, 256, 32),
                (256, 256, 32), (256, 256, 32), (256, 256, 32), (256, 256, 32), (256, 256, 32), (256, 256, 64), (256, 256, 64),
                (256, 256, 64)]


def gemm_gpu(uk, A, B, dtype, layout, plan=None):
    M, K = A.shape
    N = B.shape[0] if layout == "TN" else B.shape[1]
    d = uk.make_desc("gemm", [M, N, K], dtype=dtype, layout=layout)
    ab = uk.DeviceBuffer.from_array(A)
    bb = uk.DeviceBuffer.from_array(B)
    es = 2 if dtype == "fp16" else 4
    cb = uk.DeviceBuffer(M * N * es)
    cb.fill(0xFF)
    uk.launch(d, [ab, bb], cb, plan=plan)
    return cb.download(np.uint16 if dtype == "fp16" else np.float32, (M, N))


def frob(got, ref):
    g = got.astype(np.float64)
    r = ref.astype(np.float64)
    return float(np.linalg.norm(g - r) / np.linalg.norm(r))


def f16_inputs(M, N, K, seed, tn=True):
    A = O.f16_bits(O.uniform(M * K, seed, -1.0, 1.0)).reshape(M, K)
    shape = (N, K) if tn else (K, N)
    B = O.f16_bits(O.uniform(M * 0 + N * K, seed + 1, -1.0, 1.0)).reshape(shape)
    return A, B


@pytest.mark.parametrize("vi", range(len(F16_VARIANTS)))
@pytest.mark.parametrize("kt", [1, 2, 3, 5, 9])
def test_f16_tn_fast_variants(gpu, vi, kt):
    # kt k-tiles: 1 and 2 exercise the prologue/tail paths of the DMA ring (fewer tiles than stages).
    bm, bn, bk = F16_VARIANTS[vi]
    M, N, K = 2 * bm, 3 * bn, kt * bk
    A, B = f16_inputs(M, N, K, 100 + vi + kt)
    p = gpu.Plan()
    p.family, p.variant = 5, vi
    C = gemm_gpu(gpu, A, B, "fp16", "TN", plan=p)
    R = O.gemm_f16q(A, B, True)
    assert frob(O.f16_to_f32(C), R) <= 1e-2
    # Both sides accumulate in f32; the only extra error is the final rounding to half.
    assert frob(O.f16_to_f32(C), R) <= 1e-3


@pytest.mark.parametrize("vi", range(len(F16_VARIANTS)))
def test_f16_tn_exact_mode_bit_exact(gpu, vi):
    bm, bn, bk = F16_VARIANTS[vi]
    M, N, K = bm, 2 * bn, 8 * bk
    A = O.f16_bits(O.sawtooth(M * K, 17, 8)).reshape(M, K)
    Bl = O.sawtooth(K * N, 13, 6).reshape(K, N)  # the reference's initB over B[K][N]
    B = O.f16_bits(np.ascontiguousarray(Bl.T))
    p = gpu.Plan()
    p.family, p.variant = 5, vi
    C = gemm_gpu(gpu, A, B, "fp16", "TN", plan=p)
    R = O.gemm_f16q(A, B, True)
    assert np.array_equal(C, O.f16_bits(R))


def test_f16_tn_4096_cubed_full(gpu):
    # The config-3 shape through the solver's plan, every one of its 16.8 M outputs against the
    # oracle (f32 accumulation over the same half inputs, k ascending; about 2 s on 16 host
    # threads): the Frobenius gate over the whole matrix, and each 256 x 256 tile on its own, so a
    # single wrong tile cannot hide in the whole-matrix norm.
    M = N = K = 4096
    A, B = f16_inputs(M, N, K, 20261201 + 20)
    sol = gpu.solve(gpu.make_desc("gemm", [M, N, K], dtype="fp16", layout="TN"))
    assert sol.family == "gemm_f16_mfma"
    C = O.f16_to_f32(gemm_gpu(gpu, A, B, "fp16", "TN"))
    R = O.gemm_f16q(A, B, True, threads=16)
    assert frob(C, R) <= 1e-2
    # Both sides accumulate in f32; the only extra error is the final rounding to half.
    assert frob(C, R) <= 1e-3
    t = 256
    per_tile = np.sqrt(((C.astype(np.float64) - R) ** 2).reshape(M // t, t, N // t, t).sum(axis=(1, 3)) /
                       (R.astype(np.float64) ** 2).reshape(M // t, t, N // t, t).sum(axis=(1, 3)))
    print(f"frobenius {frob(C, R):.3e}, worst tile {per_tile.max():.3e}")
    assert per_tile.max() <= 1e-3


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (33, 47, 129), (100, 70, 5), (64, 64, 16), (257, 129, 300)])
@pytest.mark.parametrize("layout", ["NT", "TN"])
def test_f16_generic(gpu, M, N, K, layout):
    A, B = f16_inputs(M, N, K, M * 7 + N, tn=(layout == "TN"))
    C = gemm_gpu(gpu, A, B, "fp16", layout)
    R = O.gemm_f16q(A, B, layout == "TN")
    assert frob(O.f16_to_f32(C), R) <= 1e-3


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (33, 47, 129), (128, 96, 64), (512, 512, 512)])
@pytest.mark.parametrize("layout", ["NT", "TN"])
def test_f32_generic(gpu, M, N, K, layout):
    A = O.uniform(M * K, 3 + M, -1.0, 1.0).reshape(M, K)
    B = O.uniform(N * K, 4 + N, -1.0, 1.0).reshape((N, K) if layout == "TN" else (K, N))
    C = gemm_gpu(gpu, A, B, "fp32", layout)
    R = O.gemm_f32(A, B, layout == "TN")
    assert frob(C, R) <= 1e-5


@pytest.mark.parametrize("vi", [0, 1])
@pytest.mark.parametrize("M,N,K", [(64, 64, 64), (128, 192, 320), (256, 128, 512), (1024, 1536, 704)])
@pytest.mark.parametrize("layout", ["NT", "TN"])
def test_f32_variants(gpu, vi, M, N, K, layout):
    # variant 0: bounds-checked generic kernel; 1: the LDS-tiled kernel (one and several tiles,
    # one and an odd number of k-tiles, more tiles than CUs); tolerance and exact mode
    p = gpu.Plan()
    p.family, p.variant = 6, vi
    A = O.uniform(M * K, 5 + M + vi, -1.0, 1.0).reshape(M, K)
    B = O.uniform(N * K, 6 + N + vi, -1.0, 1.0).reshape((N, K) if layout == "TN" else (K, N))
    C = gemm_gpu(gpu, A, B, "fp32", layout, plan=p)
    assert frob(C, O.gemm_f32(A, B, layout == "TN")) <= 1e-5
    A = O.sawtooth(M * K, 17, 8).reshape(M, K)
    B = O.sawtooth(N * K, 13, 6).reshape((N, K) if layout == "TN" else (K, N))
    C = gemm_gpu(gpu, A, B, "fp32", layout, plan=p)
    assert np.array_equal(C.view(np.uint32), O.gemm_f32(A, B, layout == "TN").view(np.uint32))


def test_f32_tiled_refuses_other_shapes(gpu):
    p = gpu.Plan()
    p.family, p.variant = 6, 1
    A = O.uniform(64 * 96, 1, -1.0, 1.0).reshape(64, 96)  # K = 96 is not a multiple of 64
    B = O.uniform(96 * 64, 2, -1.0, 1.0).reshape(96, 64)
    with pytest.raises(gpu.UnikernError):
        gemm_gpu(gpu, A, B, "fp32", "NT", plan=p)
    assert gpu.solve(gpu.make_desc("gemm", [1024, 1024, 1024], dtype="fp32", layout="NT")).key == "gemm_f32:64x64x64,w8"
    assert gpu.solve(gpu.make_desc("gemm", [64, 64, 96], dtype="fp32", layout="NT")).key == "gemm_generic:64x64x16"


def test_f32_exact_mode_reference_sample_shape(gpu):
    # samples/kml_gemm.json (512^3, NT) on the reference's sawtooth: bit-exact.
    M = N = K = 512
    A = O.sawtooth(M * K, 17, 8).reshape(M, K)
    B = O.sawtooth(K * N, 13, 6).reshape(K, N)
    C = gemm_gpu(gpu, A, B, "fp32", "NT")
    assert np.array_equal(C.view(np.uint32), O.gemm_f32(A, B, False).view(np.uint32))
