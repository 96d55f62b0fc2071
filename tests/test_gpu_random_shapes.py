"""Parity at seeded random shapes, through the solver's own plan and the C ABI.

Each family draws shapes from a fixed-seed generator (ragged sizes, primes, sizes one off a
tile) and lets the solver pick the kernel, so the predicates that route a shape to a fast tile
or to a bounds-checked fallback are exercised together with the kernels. Gates are those of
the family's own tests: f16 GEMM Frobenius <= 1e-2 (and <= 1e-3: only the final rounding to
half differs), f32 GEMM and conv Frobenius <= 1e-5, Q8_0 Frobenius <= 1e-5 against the binary64
dot of the exactly dequantised weights, row family max_rel <= 1e-5 against binary64.
"""
import numpy as np
import pytest

import _oracle as O
from test_gpu_conv import conv_nchw_gpu, rand_conv
from test_gpu_gemm import f16_inputs, gemm_gpu
from test_gpu_q8_0 import make_weights, q8_gpu
from test_gpu_rows import check_rowsum, max_rel, rmsnorm64, run_op, softmax64

pytestmark = pytest.mark.gpu


def frob(got, ref):
    g, r = got.astype(np.float64), ref.astype(np.float64)
    return float(np.linalg.norm(g - r) / np.linalg.norm(r))


def draws(seed, n, *ranges):
    rng = np.random.default_rng(seed)
    return [tuple(int(rng.integers(lo, hi + 1)) for lo, hi in ranges) for _ in range(n)]


@pytest.mark.parametrize("M,N,K", draws(11, 10, (1, 600), (1, 600), (1, 700)) + [(257, 255, 33), (512, 768, 96)])
def test_f16_gemm_random(gpu, M, N, K):
    A, B = f16_inputs(M, N, K, 7000 + M + N + K)
    C = gemm_gpu(gpu, A, B, "fp16", "TN")
    R = O.gemm_f16q(A, B, True)
    assert frob(O.f16_to_f32(C), R) <= 1e-3


@pytest.mark.parametrize("layout", ["NT", "TN"])
@pytest.mark.parametrize("M,N,K", draws(12, 6, (1, 300), (1, 300), (1, 400)) + [(128, 192, 64), (65, 64, 64)])
def test_f32_gemm_random(gpu, layout, M, N, K):
    A = O.uniform(M * K, 7100 + M, -1.0, 1.0).reshape(M, K)
    B = O.uniform(N * K, 7200 + N, -1.0, 1.0).reshape((N, K) if layout == "TN" else (K, N))
    C = gemm_gpu(gpu, A, B, "fp32", layout)
    assert frob(C, O.gemm_f32(A, B, layout == "TN")) <= 1e-5


@pytest.mark.parametrize("layout", ["NT", "TN"])
@pytest.mark.parametrize("M,N,K", [(64 * m, 64 * n, 64 * k) for m, n, k in draws(16, 6, (1, 24), (1, 24), (1, 24))])
def test_f32_gemm_random_tiled(gpu, layout, M, N, K):
    # 64-multiples: the solver routes these to the direct-to-LDS tiled kernel.
    assert gpu.solve(gpu.make_desc("gemm", [M, N, K], dtype="fp32", layout=layout)).key == "gemm_f32:64x64x64,w8"
    A = O.uniform(M * K, 7400 + M, -1.0, 1.0).reshape(M, K)
    B = O.uniform(N * K, 7500 + N, -1.0, 1.0).reshape((N, K) if layout == "TN" else (K, N))
    C = gemm_gpu(gpu, A, B, "fp32", layout)
    assert frob(C, O.gemm_f32(A, B, layout == "TN")) <= 1e-5


@pytest.mark.parametrize("N,C,H,W,Oc,Kh,Kw,pad,stride",
                         [(n, c, h, w, oc, k, k, p, s)
                          for (n, c, h, w, oc, k, p, s) in draws(13, 8, (1, 3), (1, 24), (3, 40), (3, 40), (1, 70),
                                                                 (1, 3), (0, 1), (1, 2))
                          if h + 2 * p >= k and w + 2 * p >= k])
def test_conv_random(gpu, N, C, H, W, Oc, Kh, Kw, pad, stride):
    d = gpu.make_desc("conv", [H, W, C, Kh, Kw, Oc], layout="NCHW", batch=N, pad=pad, stride=stride,
                      epilogue="channelscale")
    gap = gpu.support_gap(d)
    if gap:
        pytest.skip(f"refused by the capability gate: {gap}")
    x, w, s = rand_conv(N, C, H, W, Oc, Kh, Kw, 7300 + N + C + H)
    y = conv_nchw_gpu(gpu, x, w, s, pad, stride)
    assert frob(y, O.conv_nchw(x, w, s, pad, stride)) <= 1e-5


@pytest.mark.parametrize("M,N,kp", draws(14, 8, (1, 24), (1, 400), (1, 40)))
def test_q8_0_random(gpu, M, N, kp):
    K = 64 * kp
    blocks, _, _ = make_weights(N, K, 7400 + M + N)
    Xh = O.f16_bits(O.normal(M * K, 7500 + kp, 0.0, 1.0)).reshape(M, K)
    assert frob(q8_gpu(gpu, Xh, blocks, N), O.q8_0_gemm(Xh, blocks, N)) <= 1e-5


@pytest.mark.parametrize("N,kq", draws(16, 10, (1, 3000), (1, 40)))
def test_q8_0_decode_row_random(gpu, N, kq):
    # One activation row, K a multiple of 256 up to 10240: the solver routes K <= 4096 to the
    # one-row-per-wavefront kernel and longer K to the tile kernels.
    K = 256 * kq
    blocks, _, _ = make_weights(N, K, 7700 + N + kq)
    Xh = O.f16_bits(O.normal(K, 7800 + N, 0.0, 1.0)).reshape(1, K)
    assert frob(q8_gpu(gpu, Xh, blocks, N), O.q8_0_gemm(Xh, blocks, N)) <= 1e-5


@pytest.mark.parametrize("L,C", draws(15, 8, (1, 300), (1, 6000)) + [(5, 4097), (9, 16384), (1, 1)])
def test_rows_random(gpu, L, C):
    X = O.normal(L * C, 7600 + L, 0.0, 1.0).reshape(L, C)
    W = O.normal(C, 7700 + C, 1.0, 0.1)
    check_rowsum(X, run_op(gpu, "reduce", X))
    assert max_rel(run_op(gpu, "rmsnorm", X, W), rmsnorm64(X, W)) <= 1e-5
    X8 = (X * np.float32(8.0)).astype(np.float32)
    assert max_rel(run_op(gpu, "softmax", X8), softmax64(X8)) <= 1e-5
