"""Exact algebraic properties of the kernels at the full BASELINE sizes.

Negation and multiplication by a power of two commute with every f32 and f16 rounding (barring
overflow and underflow), so a kernel whose summation order is
fixed must satisfy, value for value, f(-x) = -f(x) and f(2x) = 2 f(x) in an argument the op is
linear in. The oracle comparisons in the other GPU tests check the same kernels against the
reference's loops; these add whole-output identities at the BASELINE sizes, which a wrong index,
a lane that reads stale data or a run-dependent summation order would break anywhere in the
output. Values are compared as floats (a sum that cancels to +0.0 does so on both sides).

One exception is the hardware's, not the kernels': v_mfma_f32_16x16x32_f16 is not odd. A
one-wavefront probe on this part (random A, B in [-1, 1]) found D(-A, B) one ulp below -D(A, B) at
0.2% of outputs and never above, while D(2A, B) = 2 D(A, B) everywhere and v_mfma_f32_16x16x4f32
is odd and exact under doubling. So its internal sum rounds toward -infinity somewhere. Every
later step of the f16 GEMM and Q8_0 kernels (accumulation, f16 rounding, positive block scales
applied by fma) is monotonic, so for those kernels f(-x) <= -f(x) holds everywhere, with equality
almost everywhere, and doubling is exact.
"""
import numpy as np
import pytest

import _oracle as O
from test_gpu_conv import conv_nchw_gpu, rand_conv
from test_gpu_gemm import f16_inputs, gemm_gpu
from test_gpu_q8_0 import make_weights, q8_gpu
from test_gpu_rows import run_op

pytestmark = pytest.mark.gpu

SEED = 20261202


def f16_scaled(bits, factor):
    """binary16 bit patterns times an exact factor (a power of two or -1)."""
    return (bits.view(np.float16) * np.float16(factor)).view(np.uint16)


def test_conv_baseline_sign_and_scale(gpu):
    # 8 x 64 x 56 x 56 -> 64, 3x3, pad 1, fused channelscale.
    x, w, s = rand_conv(8, 64, 56, 56, 64, 3, 3, SEED)
    y = conv_nchw_gpu(gpu, x, w, s, pad=1)
    assert np.all(np.isfinite(y))
    assert np.array_equal(conv_nchw_gpu(gpu, -x, w, s, pad=1), -y)
    assert np.array_equal(conv_nchw_gpu(gpu, x, w, 2.0 * s, pad=1), 2.0 * y)


def test_gemm_f16_baseline_sign_and_scale(gpu):
    # 4096^3, A row-major, B column-major, f16 out. |C| <= K, so 2 C stays finite.
    # (Subnormal f16 outputs: see the doubling check below.)
    A, B = f16_inputs(4096, 4096, 4096, SEED + 1)
    C = gemm_gpu(gpu, A, B, "fp16", "TN").view(np.float16)
    assert np.all(np.isfinite(C))
    Cn = gemm_gpu(gpu, f16_scaled(A, -1), B, "fp16", "TN").view(np.float16)
    assert np.all(Cn <= -C) and np.mean(Cn != -C) < 0.05
    # Doubling commutes with rounding to a normal binary16 only: below 2^-14 the output grid is
    # fixed (steps of 2^-24), so a subnormal output of 2A may sit one step from twice C's.
    C2 = gemm_gpu(gpu, f16_scaled(A, 2), B, "fp16", "TN").view(np.float16)
    normal = np.abs(C) >= np.float16(2.0 ** -14)
    assert np.array_equal(C2[normal], C[normal] * np.float16(2))
    sub = ~normal
    assert np.all(np.abs(C2[sub].astype(np.float64) - 2.0 * C[sub].astype(np.float64)) <= 2.0 ** -24)


def test_gemm_f32_baseline_sign_and_scale(gpu):
    # f32 1024^3, A and B row-major (the reference's layout). The f32 MFMA is odd.
    A = O.uniform(1024 * 1024, SEED + 6, -1.0, 1.0).reshape(1024, 1024)
    B = O.uniform(1024 * 1024, SEED + 7, -1.0, 1.0).reshape(1024, 1024)
    C = gemm_gpu(gpu, A, B, "fp32", "NT")
    assert np.all(np.isfinite(C))
    assert np.array_equal(gemm_gpu(gpu, -A, B, "fp32", "NT"), -C)
    assert np.array_equal(gemm_gpu(gpu, 2.0 * A, B, "fp32", "NT"), 2.0 * C)


@pytest.mark.parametrize("M", [1, 16])
@pytest.mark.parametrize("N", [4096, 11008])
def test_q8_0_baseline_sign_and_scale(gpu, M, N):
    # configs[4] shapes at M = 1 (the one-row-per-wavefront kernel on v_dot2_f32_f16) and M = 16
    # (the one- and three-tile MFMA kernels). Both instructions' sums are one-sided under negation
    # (measured: -X gives outputs <= -Y, 0.5-0.7% of them below it for the dot products), so the
    # negated result is bounded on one side and mostly equal.
    K = 4096
    blocks, _, _ = make_weights(N, K, SEED + N)
    Xh = O.f16_bits(O.normal(M * K, SEED + M, 0.0, 1.0)).reshape(M, K)
    Y = q8_gpu(gpu, Xh, blocks, N)
    assert np.all(np.isfinite(Y))
    Yn = q8_gpu(gpu, f16_scaled(Xh, -1), blocks, N)
    assert np.all(Yn <= -Y) and np.mean(Yn != -Y) < 0.05
    assert np.array_equal(q8_gpu(gpu, f16_scaled(Xh, 2), blocks, N), 2.0 * Y)


def test_rows_baseline_sign(gpu):
    # 4096 x 4096 f32. Row-sum and RMSNorm are odd in X (RMSNorm's statistic is even).
    L = C = 4096
    X = O.normal(L * C, SEED + 3, 0.0, 1.0).reshape(L, C)
    W = O.normal(C, SEED + 4, 1.0, 0.1)
    s = run_op(gpu, "reduce", X)
    assert np.array_equal(run_op(gpu, "reduce", -X), -s)
    y = run_op(gpu, "rmsnorm", X, W)
    assert np.array_equal(run_op(gpu, "rmsnorm", -X, W), -y)
    assert np.array_equal(run_op(gpu, "rmsnorm", X, 2.0 * W), 2.0 * y)


def test_softmax_baseline_rows_are_distributions(gpu):
    # configs[1]'s softmax input (N(0,1) x 8): every output in [0, 1], every row summing to 1
    # within 4096 roundings of the row's values, and the row maximum's own term at least 1/4096.
    L = C = 4096
    X = (O.normal(L * C, SEED + 5, 0.0, 1.0) * np.float32(8.0)).reshape(L, C)
    Y = run_op(gpu, "softmax", X)
    assert np.all((Y >= 0.0) & (Y <= 1.0))
    assert np.max(np.abs(Y.astype(np.float64).sum(axis=1) - 1.0)) <= C * 2.0 ** -24
    assert np.all(Y[np.arange(L), np.argmax(X, axis=1)] >= 1.0 / C)
