"""uk_launch_noalloc, the entry point that allocates nothing, against uk_launch through the C ABI.

The two share their kernels; only the 1-D reduce needs scratch (its pass-1 partials), which each
takes from a static device array of its own (uk_launch orders its reduces through an event,
uk_launch_noalloc leaves ordering to the caller). Results must
be bit-identical to uk_launch's, on two calls in a row with the second on a smaller input (the
array keeps the first call's partials; nothing in it may leak into the second result).
"""
import ctypes as C

import numpy as np
import pytest

import _oracle as O

pytestmark = pytest.mark.gpu


def _launch(uk, fn, d, ins, out, stream=None):
    arr = (C.c_void_p * len(ins))(*[b.ptr for b in ins])
    rc = fn(C.byref(d), None, arr, len(ins), out.ptr, stream)
    assert rc == uk.UK_OK, uk.last_error()
    uk.synchronize()


def _reduce_both(uk, x, stream=None):
    d = uk.make_desc("reduce", [x.size])
    xb = uk.DeviceBuffer.from_array(x)
    got = []
    for fn in (uk.lib.uk_launch, uk.lib.uk_launch_noalloc):
        yb = uk.DeviceBuffer(4)
        yb.fill(0xFF)
        _launch(uk, fn, d, [xb], yb, stream)
        got.append(yb.download(np.float32, (1,))[0])
    return got


def test_noalloc_reduce_two_calls_second_smaller(gpu):
    big = O.normal(12_345_679, 901, 0.0, 1.0)
    small = O.normal(3001, 902, 0.0, 1.0)
    for x in (big, small):
        ref, noalloc = _reduce_both(gpu, x)
        assert noalloc.view(np.uint32) == ref.view(np.uint32)
        gate = 1e-5 * float(np.sum(np.abs(x.astype(np.float64))))
        assert abs(float(noalloc) - float(O.reduce_blocked(x))) <= gate
    # n = 1 after a full array: a single partial, the other 2047 slots hold stale values that
    # the fold must not read.
    ref, noalloc = _reduce_both(gpu, np.array([3.25], np.float32))
    assert noalloc == np.float32(3.25) and ref == np.float32(3.25)


def test_noalloc_reduce_on_a_new_stream(gpu):
    x = O.normal(1 << 20, 903, 0.0, 1.0)
    with gpu.Stream() as s:
        ref, noalloc = _reduce_both(gpu, x, s.ptr)
    assert noalloc.view(np.uint32) == ref.view(np.uint32)


@pytest.mark.parametrize("op,L,C", [("rmsnorm", 512, 4096), ("rmsnorm", 64, 1024), ("softmax", 300, 2048)])
def test_noalloc_rows_match_launch(gpu, op, L, C):
    X = O.normal(L * C, 904 + C, 0.0, 1.0).reshape(L, C)
    ins = [gpu.DeviceBuffer.from_array(X)]
    if op == "rmsnorm":
        ins.append(gpu.DeviceBuffer.from_array(O.normal(C, 905, 1.0, 0.1)))
    d = gpu.make_desc(op, [L, C])
    outs = []
    for fn in (gpu.lib.uk_launch, gpu.lib.uk_launch_noalloc):
        yb = gpu.DeviceBuffer(L * C * 4)
        yb.fill(0xFF)
        _launch(gpu, fn, d, ins, yb)
        outs.append(yb.download(np.float32, (L, C)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_noalloc_gemm_f16_matches_launch(gpu):
    M, N, K = 512, 512, 256
    A = O.f16_bits(O.uniform(M * K, 906, -1.0, 1.0)).reshape(M, K)
    B = O.f16_bits(O.uniform(N * K, 907, -1.0, 1.0)).reshape(N, K)
    d = gpu.make_desc("gemm", [M, N, K], dtype="fp16", layout="TN")
    ins = [gpu.DeviceBuffer.from_array(A), gpu.DeviceBuffer.from_array(B)]
    outs = []
    for fn in (gpu.lib.uk_launch, gpu.lib.uk_launch_noalloc):
        cb = gpu.DeviceBuffer(M * N * 2)
        _launch(gpu, fn, d, ins, cb)
        outs.append(cb.download(np.uint16, (M, N)))
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("M", [1, 16])
def test_noalloc_q8_0_matches_launch(gpu, M):
    # M = 1: the one-row-per-wavefront kernel; M = 16: the tile kernel. Neither needs scratch.
    from test_gpu_q8_0 import make_weights

    N, K = 1000, 4096
    blocks, _, _ = make_weights(N, K, 908 + M)
    Xh = O.f16_bits(O.normal(M * K, 909 + M, 0.0, 1.0)).reshape(M, K)
    d = gpu.make_desc("gemm", [M, N, K], dtype="q8_0", layout="TN")
    ins = [gpu.DeviceBuffer.from_array(Xh), gpu.DeviceBuffer.from_array(blocks)]
    outs = []
    for fn in (gpu.lib.uk_launch, gpu.lib.uk_launch_noalloc):
        yb = gpu.DeviceBuffer(M * N * 4)
        yb.fill(0xFF)
        _launch(gpu, fn, d, ins, yb)
        outs.append(yb.download(np.float32, (M, N)))
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert np.linalg.norm(outs[0] - O.q8_0_gemm(Xh, blocks, N)) <= 1e-5 * np.linalg.norm(O.q8_0_gemm(Xh, blocks, N))
