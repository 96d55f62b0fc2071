"""Parity of the Q8_0 skinny GEMM (in-kernel dequant, f16 MFMA, f32 accumulate).

The reference has no Q8_0 path (src/codegen_hip.cpp:87-88 refuses int8), so the oracle is the
block definition itself (GGUF type 8: binary16 d, int8 q[32]; value d*q) with a binary64 dot.
Gates: ||y - r||_F / ||r||_F <= 1e-5 against the binary64 oracle; dequantisation and indexing
bit-exact (one-hot activations select single dequantised weights; exact-arithmetic inputs give
bit-identical outputs).
"""
import numpy as np
import pytest

import _oracle as O

pytestmark = pytest.mark.gpu


def make_weights(N, K, seed, exact=False):
    if exact:
        q = (np.arange(N * K) % 255 - 127).astype(np.int8).reshape(N, K)
        e = (np.arange(N * (K // 32)) % 7).astype(np.float32)
        d = O.f16_bits(np.ldexp(np.float32(1.0), -(e.astype(np.int32) + 4)).astype(np.float32))
    else:
        u = O.uniform(N * K, seed, 0.0, 1.0)
        q = ((u * 255.0).astype(np.int32) - 127).astype(np.int8).reshape(N, K)
        d = O.f16_bits(O.uniform(N * (K // 32), seed + 1, 1e-3, 1e-2))
    return O.q8_0_pack(q, d.reshape(N, K // 32)), q, d


def q8_gpu(uk, Xh, blocks, N, plan=None):
    M, K = Xh.shape
    d = uk.make_desc("gemm", [M, N, K], dtype="q8_0", layout="TN")
    xb, wb = uk.DeviceBuffer.from_array(Xh), uk.DeviceBuffer.from_array(blocks)
    yb = uk.DeviceBuffer(M * N * 4)
    yb.fill(0xFF)
    uk.launch(d, [xb, wb], yb, plan=plan)
    return yb.download(np.float32, (M, N))


def frob(y, r):
    return float(np.linalg.norm(y.astype(np.float64) - r) / np.linalg.norm(r))


@pytest.mark.parametrize("M", [1, 8, 16])
@pytest.mark.parametrize("N", [4096, 11008])
def test_llama7b_decode_shapes(gpu, M, N):
    K = 4096
    blocks, _, _ = make_weights(N, K, 20261201 + 41)
    Xh = O.f16_bits(O.normal(M * K, 20261201 + 40, 0.0, 1.0)).reshape(M, K)
    y = q8_gpu(gpu, Xh, blocks, N)
    r = O.q8_0_gemm(Xh, blocks, N)
    assert frob(y, r) <= 1e-5
    # every output individually within 1e-5 of its row's scale
    assert np.all(np.abs(y - r) <= 1e-5 * np.linalg.norm(r, axis=1, keepdims=True) / np.sqrt(N) * 10)


@pytest.mark.parametrize("M", [16, 5, 1])
def test_dequant_bit_exact_one_hot(gpu, M):
    # Row m of X is one-hot at column k_m: y[m][n] = d[n][k_m/32] * q[n][k_m] exactly, so the
    # kernel's dequantisation and its block/lane indexing are checked value by value. M = 16
    # takes the whole-line activation loads, M = 5 and M = 1 the activations copied into LDS.
    N, K = 96, 512
    blocks, _, _ = make_weights(N, K, 77)
    deq = O.q8_0_dequant(blocks, N, K)
    for start in range(0, K, 16 * 7):
        ks = [(start + 7 * j) % K for j in range(M)]
        X = np.zeros((M, K), np.float32)
        X[np.arange(M), ks] = 1.0
        y = q8_gpu(gpu, O.f16_bits(X), blocks, N)
        want = deq[:, ks].T
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("M", [16, 5, 1])
def test_exact_arithmetic_bit_exact(gpu, M):
    # Power-of-two scales and small-integer activations: every product and partial sum is exact,
    # so the f32 result equals the binary64 oracle rounded once (i.e. exactly).
    N, K = 256, 1024
    blocks, _, _ = make_weights(N, K, 0, exact=True)
    X = ((np.arange(M * K) % 5) - 2).astype(np.float32).reshape(M, K)
    y = q8_gpu(gpu, O.f16_bits(X), blocks, N)
    r = O.q8_0_gemm(O.f16_bits(X), blocks, N)
    assert np.array_equal(y, r.astype(np.float32))


@pytest.mark.parametrize("M,N,K", [(3, 17, 64), (20, 100, 128), (1, 1, 64), (16, 4097, 256), (5, 48, 4096)])
def test_ragged_shapes(gpu, M, N, K):
    blocks, _, _ = make_weights(N, K, M + N)
    Xh = O.f16_bits(O.normal(M * K, K, 0.0, 1.0)).reshape(M, K)
    assert frob(q8_gpu(gpu, Xh, blocks, N), O.q8_0_gemm(Xh, blocks, N)) <= 1e-5


@pytest.mark.parametrize("vi", range(10))  # the tile kernels; the M = 1 kernel is tested below
@pytest.mark.parametrize("K", [2048, 4608])
@pytest.mark.parametrize("M", [1, 5, 8, 13])
def test_every_variant(gpu, vi, K, M):
    # K = 4608 (72 block pairs) leaves a partial last round for every variant; N = 300 leaves a
    # partial last weight tile for the 64-row workgroups. M = 13 takes the whole-line activation
    # loads (M > 8) with rows 13-15 past M; M = 1, 5 and 8 the activations copied into LDS where
    # the variant has room for them (M = 5: the last copy's upper half masked).
    p = gpu.Plan()
    p.family, p.variant = 8, vi
    N = 300
    blocks, _, _ = make_weights(N, K, 5 + vi)
    Xh = O.f16_bits(O.normal(M * K, 6 + vi, 0.0, 1.0)).reshape(M, K)
    assert frob(q8_gpu(gpu, Xh, blocks, N, plan=p), O.q8_0_gemm(Xh, blocks, N)) <= 1e-5


GEMV_VARIANT = 10  # the kQ8Variants entry of the M = 1 kernel


def gemv_plan(gpu, vi):
    p = gpu.Plan()
    p.family, p.variant = 8, vi
    return p


@pytest.mark.parametrize("K", [256, 768, 2048, 3840, 4096])
@pytest.mark.parametrize("N", [1, 5, 300, 4097])
def test_gemv(gpu, K, N):
    # One weight row per wavefront: N = 1, 5 and 4097 leave wavefronts past N (clamped rows, not
    # stored); K < 4096 runs the general instantiation (K = 256: 4 of the 64 lanes busy), K = 4096
    # the one with constant counts.
    blocks, _, _ = make_weights(N, K, 31 + K + N)
    Xh = O.f16_bits(O.normal(K, 32 + N, 0.0, 1.0)).reshape(1, K)
    y = q8_gpu(gpu, Xh, blocks, N, plan=gemv_plan(gpu, GEMV_VARIANT))
    assert frob(y, O.q8_0_gemm(Xh, blocks, N)) <= 1e-5


@pytest.mark.parametrize("K", [1280, 4096])
def test_gemv_dequant_bit_exact_one_hot(gpu, K):
    # A one-hot activation row selects one dequantised weight per row: every block, lane and
    # activation-chunk rotation is checked value by value (y[n] = d[n][k/32] * q[n][k]).
    N = 40
    blocks, _, _ = make_weights(N, K, 5 + K)
    deq = O.q8_0_dequant(blocks, N, K)
    for k in list(range(0, 64)) + list(range(64, K, 61)) + [K - 1]:
        X = np.zeros((1, K), np.float32)
        X[0, k] = 1.0
        y = q8_gpu(gpu, O.f16_bits(X), blocks, N, plan=gemv_plan(gpu, GEMV_VARIANT))
        assert np.array_equal(y[0].view(np.uint32), deq[:, k].view(np.uint32)), k


@pytest.mark.parametrize("K", [1024, 4096])
def test_gemv_exact_arithmetic_bit_exact(gpu, K):
    N = 256
    blocks, _, _ = make_weights(N, K, 0, exact=True)
    X = ((np.arange(K) % 5) - 2).astype(np.float32).reshape(1, K)
    y = q8_gpu(gpu, O.f16_bits(X), blocks, N, plan=gemv_plan(gpu, GEMV_VARIANT))
    assert np.array_equal(y, O.q8_0_gemm(O.f16_bits(X), blocks, N).astype(np.float32))


def test_gemv_refuses_what_it_cannot_run(gpu):
    blocks, _, _ = make_weights(8, 512, 9)
    with pytest.raises(gpu.UnikernError):  # two activation rows
        q8_gpu(gpu, O.f16_bits(O.normal(2 * 512, 1, 0.0, 1.0)).reshape(2, 512), blocks, 8, plan=gemv_plan(gpu, GEMV_VARIANT))
    blocks, _, _ = make_weights(8, 192, 9)
    with pytest.raises(gpu.UnikernError):  # K not a multiple of 256
        q8_gpu(gpu, O.f16_bits(O.normal(192, 1, 0.0, 1.0)).reshape(1, 192), blocks, 8, plan=gemv_plan(gpu, GEMV_VARIANT))
    blocks, _, _ = make_weights(8, 4352, 9)
    with pytest.raises(gpu.UnikernError):  # more than 64 block pairs (one per lane)
        q8_gpu(gpu, O.f16_bits(O.normal(4352, 1, 0.0, 1.0)).reshape(1, 4352), blocks, 8, plan=gemv_plan(gpu, GEMV_VARIANT))


def test_decode_row_picks_gemv(gpu):
    # The solver's M = 1 pick at the BASELINE shapes is the one-row-per-wavefront kernel.
    for N in (4096, 11008):
        assert gpu.solve(gpu.make_desc("gemm", [1, N, 4096], dtype="q8_0", layout="TN")).key.startswith("q8_0:gemv")


def test_k_not_whole_block_pairs_is_refused(gpu):
    d = gpu.make_desc("gemm", [4, 16, 96], dtype="q8_0", layout="TN")
    assert "K divisible by 64" in gpu.support_gap(d)


def test_sixteen_byte_copies_need_aligned_segments(gpu):
    # variant 0 copies 16-byte units: K must be a multiple of 64 * pairs (256); K = 192 is not
    p = gpu.Plan()
    p.family, p.variant = 8, 0
    blocks, _, _ = make_weights(17, 192, 3)
    Xh = O.f16_bits(O.normal(3 * 192, 4, 0.0, 1.0)).reshape(3, 192)
    with pytest.raises(gpu.UnikernError):
        q8_gpu(gpu, Xh, blocks, 17, plan=p)
    # the solver never picks it for such K
    assert gpu.solve(gpu.make_desc("gemm", [3, 17, 192], dtype="q8_0", layout="TN")).key.endswith("vec=1")
