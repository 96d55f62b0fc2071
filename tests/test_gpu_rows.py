"""Parity of the row family (row-sum, RMSNorm, softmax), standalone channelscale and the 1-D
reduce on the MI355X against the CPU oracle, through the C ABI.

Gates (stated here, from the north star): row-sum |y - r| <= 1e-5 * sum|x| per row;
RMSNorm and softmax max |y - r| / max(|r|, 1e-6) <= 1e-5 (the reference's metric,
src/codegen_hip.cpp:1410-1416, at the north-star tolerance); channelscale bit-exact (one
correctly rounded multiply); sawtooth ("exact mode") row sums bit-exact.
"""
import numpy as np
import pytest

import _oracle as O

pytestmark = pytest.mark.gpu

# (threads per row, float4 per thread) of every compiled rows variant, in table order; from the
# seventeenth on they carry the non-temporal hint, the twenty-third and twenty-fourth walk two rows
# per workgroup, and the last stores its workgroup's four rows after one barrier (gain in LDS).
ROWS_VARIANTS = [(64, 1), (64, 2), (64, 4), (64, 8), (64, 16), (128, 4), (128, 8), (256, 1), (256, 2), (256, 4),
                 (256, 8), (512, 2), (512, 4), (1024, 1), (1024, 2), (1024, 4), (256, 4), (512, 2), (1024, 1),
                 (512, 4), (1024, 2), (128, 8), (256, 4), (512, 2), (64, 16)]


def run_op(uk, op, X, W=None, plan=None, eps=1e-6):
    L, C = X.shape
    d = uk.make_desc(op, [L, C], eps=eps)
    xb = uk.DeviceBuffer.from_array(X)
    ins = [xb]
    if W is not None:
        ins.append(uk.DeviceBuffer.from_array(W))
    out_shape = (L,) if op == "reduce" else (L, C)
    yb = uk.DeviceBuffer(int(np.prod(out_shape)) * 4)
    yb.fill(0xFF)  # NaN pattern: an output the kernel does not write fails the comparison
    uk.launch(d, ins, yb, plan=plan)
    return yb.download(np.float32, out_shape)


def rows_plan(uk, variant):
    p = uk.Plan()
    p.family = 1
    p.variant = variant
    return p


def check_rowsum(X, Y):
    r, a = O.rowsum_f64(X)
    ref_order = O.rowsum_blocked(X)  # the reference's own basis (width 1024)
    assert np.all(np.abs(Y.astype(np.float64) - r) <= 1e-5 * a), "row-sum gate vs binary64"
    assert np.all(np.abs(Y.astype(np.float64) - ref_order.astype(np.float64)) <= 1e-5 * a), "vs reference order"


def max_rel(y, r):
    r64 = r.astype(np.float64)
    return float(np.max(np.abs(y.astype(np.float64) - r64) / np.maximum(np.abs(r64), 1e-6)))


def softmax64(X):
    x = X.astype(np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def rmsnorm64(X, W, eps=1e-6):
    x = X.astype(np.float64)
    return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * W.astype(np.float64)


def check_rows_op(Y, ref_order, exact64, C):
    """North-star gate against binary64; against the reference-order loops (a sequential f32 sum
    whose own error grows with the row length) the bound is widened by C * 2^-24."""
    assert max_rel(Y, exact64) <= 1e-5
    assert max_rel(Y, ref_order) <= max(1e-5, C * 2.0 ** -24)


SHAPES = [(4096, 4096), (64, 256), (3, 4096), (1, 4), (7, 1000), (2, 16384), (130, 512), (65536, 256)]


@pytest.mark.parametrize("L,C", SHAPES)
def test_rowsum_solver_plan(gpu, L, C):
    X = O.normal(L * C, 20261201 + 10 + L + C, 0.0, 1.0).reshape(L, C)
    check_rowsum(X, run_op(gpu, "reduce", X))


@pytest.mark.parametrize("L,C", SHAPES)
def test_rmsnorm_solver_plan(gpu, L, C):
    X = O.normal(L * C, 20261201 + 10 + L, 0.0, 1.0).reshape(L, C)
    W = O.normal(C, 20261201 + 11, 1.0, 0.1)
    Y = run_op(gpu, "rmsnorm", X, W)
    check_rows_op(Y, O.rmsnorm(X, W), rmsnorm64(X, W), C)


@pytest.mark.parametrize("L,C", SHAPES)
def test_softmax_solver_plan(gpu, L, C):
    X = O.normal(L * C, 20261201 + 12 + L, 0.0, 8.0).reshape(L, C)
    Y = run_op(gpu, "softmax", X)
    check_rows_op(Y, O.softmax(X), softmax64(X), C)
    assert np.allclose(Y.astype(np.float64).sum(axis=1), 1.0, atol=1e-4)


@pytest.mark.parametrize("vi", range(len(ROWS_VARIANTS)))
def test_every_rows_variant(gpu, vi):
    tpr, nv = ROWS_VARIANTS[vi]
    cap = tpr * nv * 4
    for C in sorted({cap, max(4, cap // 2 + 4), max(4, cap - 4)}):
        L = 37
        X = O.normal(L * C, 7 + C, 0.0, 2.0).reshape(L, C)
        W = O.normal(C, 8 + C, 1.0, 0.1)
        plan = rows_plan(gpu, vi)
        check_rowsum(X, run_op(gpu, "reduce", X, plan=plan))
        check_rows_op(run_op(gpu, "rmsnorm", X, W, plan=plan), O.rmsnorm(X, W), rmsnorm64(X, W), C)
        check_rows_op(run_op(gpu, "softmax", X * 4, plan=plan), O.softmax(X * 4), softmax64(X * 4), C)


@pytest.mark.parametrize("L,C", [(5, 1001), (3, 3), (2, 70001), (1, 1)])
def test_stream_fallback_any_length(gpu, L, C):
    sol = gpu.solve(gpu.make_desc("softmax", [L, C]))
    assert sol.family == "rows_stream"
    X = O.normal(L * C, 99 + C, 0.0, 3.0).reshape(L, C)
    W = O.normal(C, 98 + C, 1.0, 0.1)
    check_rowsum(X, run_op(gpu, "reduce", X))
    check_rows_op(run_op(gpu, "rmsnorm", X, W), O.rmsnorm(X, W), rmsnorm64(X, W), C)
    check_rows_op(run_op(gpu, "softmax", X), O.softmax(X), softmax64(X), C)


def test_rowsum_exact_mode_bit_exact(gpu):
    # Sawtooth rows in 2^-4 units (the reference's initX): every partial sum is exact, so the
    # GPU must equal the reference-order CPU sum bit for bit.
    L, C = 1024, 4096
    X = O.sawtooth(L * C, 17, 8).reshape(L, C)
    Y = run_op(gpu, "reduce", X)
    assert np.array_equal(Y.view(np.uint32), O.rowsum_blocked(X).view(np.uint32))


def test_constant_rows_closed_forms(gpu):
    # softmax of a constant row is 1/C exactly; rmsnorm of a constant row v with unit gain is
    # v / sqrt(v^2 + eps) (one rounding each for the divide, sqrt and multiplies).
    L, C = 8, 4096
    X = np.full((L, C), 0.75, np.float32)
    Y = run_op(gpu, "softmax", X)
    assert np.all(Y == np.float32(1.0 / C))
    W = np.ones(C, np.float32)
    Yr = run_op(gpu, "rmsnorm", X, W)
    assert np.array_equal(Yr, O.rmsnorm(X, W))


def test_softmax_large_magnitudes_need_max_subtraction(gpu):
    # exp(x) overflows binary32 above 88.7: without max subtraction these rows become inf/nan.
    L, C = 16, 2048
    X = O.normal(L * C, 5, 0.0, 40.0).reshape(L, C) + 100.0
    Y = run_op(gpu, "softmax", X)
    assert np.all(np.isfinite(Y))
    check_rows_op(Y, O.softmax(X), softmax64(X), C)


@pytest.mark.parametrize("vi", [11, 17, 24])
def test_softmax_huge_maxima(gpu, vi):
    # The numerators are 2^((x - max) log2 e): x - max is exact wherever x is within a factor of
    # two of the maximum, so their error does not grow with the maximum's magnitude. Rows with
    # maxima from 0 to 1e30 (where max log2 e rounded to binary32 is off by up to 2^76) share one
    # launch; variant 24 is the grouped-store form.
    L, C = 12, 4096
    X = O.normal(L * C, 77, 0.0, 8.0).reshape(L, C)
    offsets = np.array([0, 1e4, -1e6, 1.1e7, 1.17e7, -1.17e7, 1e8, -3e9, 1e20, -1e30, 250.0, 0], np.float32)
    X = (X + offsets[:, None]).astype(np.float32)
    Y = run_op(gpu, "softmax", X, plan=rows_plan(gpu, vi))
    assert np.all(np.isfinite(Y))
    check_rows_op(Y, O.softmax(X), softmax64(X), C)


@pytest.mark.parametrize("vi", [None, 11, 17, 24])
def test_softmax_non_finite_rows(gpu, vi):
    # The reference's loop (src/codegen_hip.cpp:1999-2009) on non-finite inputs: a -inf element
    # under a finite maximum gives exactly 0, a row holding +inf or only -inf gives NaN
    # throughout (inf - inf), and a row with one finite element gives exactly 1 there.
    L, C = 6, 4096
    X = O.normal(L * C, 91, 0.0, 8.0).reshape(L, C).copy()
    X[1, ::7] = -np.inf
    X[2, 100] = np.inf
    X[3, :] = -np.inf
    X[4, :] = -np.inf
    X[4, 4095] = 3.0
    Y = run_op(gpu, "softmax", X, plan=None if vi is None else rows_plan(gpu, vi))
    R = O.softmax(X)
    assert np.array_equal(np.isnan(Y), np.isnan(R)) and np.isnan(Y[2]).all() and np.isnan(Y[3]).all()
    assert np.all(Y[1, ::7] == 0.0) and Y[4, 4095] == 1.0 and np.all(Y[4, :4095] == 0.0)
    ok = ~np.isnan(R)
    assert np.all(np.abs(Y[ok] - R[ok]) <= 1e-5 * np.maximum(np.abs(R[ok]), 1e-6))


@pytest.mark.parametrize("L,C", [(4096, 4096), (65536, 256), (3, 7), (1, 1), (5, 12), (37, 4096), (6, 2052),
                                 (5, 3000), (2, 2048), (3, 4100)])
def test_channelscale_bit_exact(gpu, L, C):
    # (37, 4096), (6, 2052) and (5, 3000) take the row form (rows beyond L masked in the last
    # workgroup); (2, 2048) and (3, 4100) fall on either side of it.
    X = O.normal(L * C, 31 + C, 0.0, 1.0).reshape(L, C)
    S = O.uniform(C, 32, 0.5, 1.5)
    Y = run_op(gpu, "channelscale", X, S)
    assert np.array_equal(Y.view(np.uint32), O.channelscale(X, S).view(np.uint32))


@pytest.mark.parametrize("n", [1, 3, 1000, 1 << 20, 4194304, 12345679])
def test_reduce1d(gpu, n):
    x = O.normal(n, 40 + n, 0.0, 1.0)
    d = gpu.make_desc("reduce", [n])
    xb = gpu.DeviceBuffer.from_array(x)
    yb = gpu.DeviceBuffer(4)
    gpu.launch(d, [xb], yb)
    y = float(yb.download(np.float32, (1,))[0])
    exact = float(np.sum(x.astype(np.float64)))
    assert abs(y - exact) <= 1e-5 * float(np.sum(np.abs(x.astype(np.float64))))
    assert abs(y - float(O.reduce_blocked(x))) <= 1e-5 * float(np.sum(np.abs(x.astype(np.float64))))


def test_reduce1d_interleaved_on_two_streams(gpu):
    # uk_launch's 1-D reduces share one partials array per GPU and are ordered through one event:
    # reduces enqueued alternately on two streams, with no synchronisation between them, each
    # give the result the same reduce gives alone.
    xs = [O.normal(n, 41 + n, 0.0, 1.0) for n in (12_345_679, 4_000_037)]
    d = [gpu.make_desc("reduce", [x.size]) for x in xs]
    xb = [gpu.DeviceBuffer.from_array(x) for x in xs]
    solo = []
    for k in range(2):
        yb = gpu.DeviceBuffer(4)
        gpu.launch(d[k], [xb[k]], yb)
        solo.append(yb.download(np.float32, (1,))[0])
    outs = [[gpu.DeviceBuffer(4) for _ in range(6)] for _ in range(2)]
    with gpu.Stream() as s0, gpu.Stream() as s1:
        for i in range(6):
            for k, st in enumerate((s0, s1)):
                gpu.launch(d[k], [xb[k]], outs[k][i], stream=st.ptr, sync=False)
        s0.synchronize()
        s1.synchronize()
    for k in range(2):
        for yb in outs[k]:
            assert yb.download(np.float32, (1,))[0].view(np.uint32) == solo[k].view(np.uint32)


def test_reduce1d_reference_verify_instance(gpu):
    # The reference's own device verify (src/codegen_hip.cpp:916-941): 2^20 values of 2^-6 sum to
    # exactly 16384 in any binary32 order.
    x = np.full(1 << 20, 0.015625, np.float32)
    d = gpu.make_desc("reduce", [x.size])
    xb = gpu.DeviceBuffer.from_array(x)
    yb = gpu.DeviceBuffer(4)
    gpu.launch(d, [xb], yb)
    assert yb.download(np.float32, (1,))[0] == np.float32(16384.0)


def test_reduce1d_two_streams(gpu):
    # Two 1-D reduces enqueued back to back on two streams run concurrently; each stream has its
    # own pass-1 partials, so both sums come out as they do alone (bit for bit: the fold order
    # is fixed).
    n = 1 << 24
    xs = [O.normal(n, 77 + i, 0.0, 1.0) for i in range(2)]
    d = gpu.make_desc("reduce", [n])
    alone = []
    for x in xs:
        xb, yb = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4)
        gpu.launch(d, [xb], yb)
        alone.append(yb.download(np.float32, (1,))[0])
    with gpu.Stream() as s0, gpu.Stream() as s1:
        bufs = [(gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4)) for x in xs]
        for _ in range(20):
            for (xb, yb), s in zip(bufs, (s0, s1)):
                gpu.launch(d, [xb], yb, stream=s.ptr, sync=False)
        s0.synchronize()
        s1.synchronize()
        got = [yb.download(np.float32, (1,))[0] for _, yb in bufs]
    for x, g, a in zip(xs, got, alone):
        assert g.view(np.uint32) == a.view(np.uint32)
        assert abs(float(g) - float(np.sum(x.astype(np.float64)))) <= 1e-5 * float(np.sum(np.abs(x.astype(np.float64))))
