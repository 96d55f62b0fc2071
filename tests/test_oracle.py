"""Pins the CPU oracle (oracle/liboracle.so) before any GPU result is judged by it.

Each restated function is checked against (1) the reference's own outputs — golden vectors that
tests/golden/make_golden.py wrote from the reference sources compiled in this container, (2) the
reference's hand-computed cases (tests/acceptance.cpp:1318-1357), (3) closed forms and (4) a
binary64 brute force on small inputs, chosen so that a plausible mistake (a dropped term, a
transposed operand, a wrong index or order) fails at least one of them. When oracle/_ref is
built (this container only), the restatement is also compared with the live reference build.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import _oracle as O

G = np.load(Path(__file__).resolve().parent / "golden" / "numerics.npz")


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ---------------------------------------------------------------------------------------------
# PRNG and binary16 conversion


def test_splitmix64_published_sequence():
    # SplitMix64 (Steele, Lea, Flood 2014; Vigna's reference C) from state 0.
    st = C.c_uint64(0)
    got = [O.oracle().or_splitmix64(C.byref(st)) for _ in range(3)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_uniform_stream_definition():
    # uniform = lo + (hi - lo) * (top 24 bits of the SplitMix64 word) * 2^-24, rounded to f32
    st = C.c_uint64(12345)
    words = [O.oracle().or_splitmix64(C.byref(st)) for _ in range(8)]
    want = np.array([-2.0 + 5.0 * ((w >> 40) * 2.0 ** -24) for w in words], np.float32)
    assert np.array_equal(O.uniform(8, 12345, -2.0, 3.0), want)


def test_f16_to_f32_exhaustive():
    h = np.arange(1 << 16, dtype=np.uint16)
    got = O.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got[~nan]), bits(want[~nan]))


def test_f32_to_f16_round_to_nearest_even():
    x = np.concatenate([G["f2h_x"], O.normal(1 << 16, 99, 0.0, 3e4), O.uniform(1 << 16, 98, -7e-5, 7e-5),
                        np.array([65519.996, 65520.0, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -24 * 1.5],
                                 np.float32)]).astype(np.float32)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f16_bits(x), want)


def test_f32_to_f16_matches_reference_float2half():
    # the conversion the reference's f16 GEMM program applies to its inputs (hip_fp16.h)
    assert np.array_equal(O.f16_bits(G["f2h_x"]), G["f2h_h"])


# ---------------------------------------------------------------------------------------------
# reduce (src/reference.cpp:24-48)


@pytest.mark.parametrize("n", [0, 1, 3, 1023, 1024, 1025, 4097, 20011])
def test_reduce_matches_reference_vectors(n):
    x = G[f"reduce_x_{n}"]
    assert O.reduce_blocked(x, 1024) == G[f"reduce_blocked_y_{n}"][0] or (
        bits(O.reduce_blocked(x, 1024)) == bits(G[f"reduce_blocked_y_{n}"][0]))
    y = np.zeros(1, np.float32)
    O.oracle().or_cpu_reduce(O.ptr(x), O.ptr(y), n)
    assert bits(y) == bits(G[f"reduce_y_{n}"])


def test_reduce_closed_forms():
    # tests/acceptance.cpp:1348-1355: 2^20 values of 2^-6 sum to 16384; empty range is 0
    for n, want in ((1 << 20, 16384.0), (1 << 24, 262144.0)):
        v = np.full(n, 0.015625, np.float32)
        y = np.zeros(1, np.float32)
        O.oracle().or_cpu_reduce(O.ptr(v), O.ptr(y), n)
        assert y[0] == want
        assert O.reduce_blocked(v, 1024) == want
    y = np.ones(1, np.float32)
    O.oracle().or_cpu_reduce(O.ptr(np.zeros(1, np.float32)), O.ptr(y), 0)
    assert y[0] == 0.0


def test_reduce_blocked_order():
    # width-1024 blocking: partial p sums x[p], x[p+1024], ... ascending, partials folded in
    # index order; 1 + 2^-24 patterns make a sequential sum differ from the blocked one.
    n = 4096
    x = np.full(n, 2.0 ** -24, np.float32)
    x[0] = 1.0
    want = np.float32(0)
    parts = [np.float32(0)] * 1024
    for i in range(n):
        parts[i % 1024] = np.float32(parts[i % 1024] + x[i])
    for p in parts:
        want = np.float32(want + p)
    assert O.reduce_blocked(x, 1024) == want
    seq = np.zeros(1, np.float32)
    O.oracle().or_cpu_reduce(O.ptr(x), O.ptr(seq), n)
    assert seq[0] == 1.0 and want != 1.0  # the two orders are distinguishable on this input


def test_rowsum_is_blocked_reduce_per_row():
    X = np.stack([G["reduce_x_4097"][:4096], G["reduce_x_20011"][:4096], -G["reduce_x_4097"][1:]])
    got = O.rowsum_blocked(X, 1024)
    for i in range(3):
        assert bits(got[i]) == bits(O.reduce_blocked(X[i], 1024))


# ---------------------------------------------------------------------------------------------
# conv (src/reference.cpp:6-22) and the NCHW restatement used for the BASELINE conv


def test_cpu_conv_hand_cases():
    # tests/acceptance.cpp:1322-1346
    y = O.cpu_conv(np.array([1, 2, 3, 4], np.float32), np.array([0.5], np.float32), 2, 2, 1, 1, 1, 1)
    assert list(y.ravel()) == [0.5, 1.0, 1.5, 2.0]
    y = O.cpu_conv(np.arange(1, 10, dtype=np.float32), np.eye(3, dtype=np.float32).ravel(), 3, 3, 1, 3, 3, 1)
    assert list(y.ravel()) == [15.0]
    y = O.cpu_conv(np.array([1, 2, 3, 4], np.float32), np.array([1, 10, -1, 1], np.float32), 1, 2, 2, 1, 1, 2)
    assert list(y.ravel()) == [21.0, 43.0, 1.0, 1.0]


@pytest.mark.parametrize("i", range(5))
def test_cpu_conv_matches_reference_vectors(i):
    H, W, Cc, Kh, Kw, Oc = (int(v) for v in G[f"conv_{i}_shape"])
    y = O.cpu_conv(G[f"conv_{i}_x"], G[f"conv_{i}_w"], H, W, Cc, Kh, Kw, Oc)
    assert np.array_equal(bits(y.ravel()), bits(G[f"conv_{i}_y"]))


def _conv_f64(x, w, pad, stride):
    N, Cc, H, W = x.shape
    Oc, _, Kh, Kw = w.shape
    Ho, Wo = (H + 2 * pad - Kh) // stride + 1, (W + 2 * pad - Kw) // stride + 1
    xp = np.zeros((N, Cc, H + 2 * pad, W + 2 * pad))
    xp[:, :, pad:pad + H, pad:pad + W] = x
    y = np.zeros((N, Oc, Ho, Wo))
    for kh in range(Kh):
        for kw in range(Kw):
            patch = xp[:, :, kh:kh + stride * Ho:stride, kw:kw + stride * Wo:stride]
            y += np.einsum("nchw,oc->nohw", patch, w[:, :, kh, kw].astype(np.float64))
    return y


@pytest.mark.parametrize("shape", [(1, 3, 5, 6, 4, 3, 3, 1, 1), (2, 5, 7, 7, 6, 3, 3, 1, 2), (1, 2, 4, 9, 3, 1, 1, 0, 1),
                                   (3, 4, 6, 5, 2, 5, 3, 2, 1), (1, 1, 1, 1, 1, 3, 3, 1, 1)])
def test_conv_nchw_against_binary64(shape):
    N, Cc, H, W, Oc, Kh, Kw, pad, stride = shape
    x = O.normal(N * Cc * H * W, 11, 0.0, 1.0).reshape(N, Cc, H, W)
    w = O.normal(Oc * Cc * Kh * Kw, 12, 0.0, 0.5).reshape(Oc, Cc, Kh, Kw)
    s = O.uniform(Oc, 13, 0.5, 1.5)
    y = O.conv_nchw(x, w, s, pad, stride)
    r = _conv_f64(x, w, pad, stride) * s.astype(np.float64)[None, :, None, None]
    assert y.shape == r.shape
    k = Cc * Kh * Kw
    bound = (k + 1) * 2.0 ** -24 * (_conv_f64(np.abs(x), np.abs(w), pad, stride) *
                                      s.astype(np.float64)[None, :, None, None]) + 1e-30
    assert np.all(np.abs(y - r) <= bound)


def test_conv_nchw_equals_reference_conv_on_its_layout():
    # N=1, pad 0, stride 1: the NCHW restatement and the reference's HWC conv accumulate in the
    # same c -> kh -> kw order, so the results agree bit for bit after the layout transposes.
    H, W, Cc, Kh, Kw, Oc = 9, 7, 8, 3, 3, 5
    x_hwc = O.normal(H * W * Cc, 21, 0.0, 1.0).reshape(H, W, Cc)
    w_ohwc = O.normal(Oc * Kh * Kw * Cc, 22, 0.0, 0.3).reshape(Oc, Kh, Kw, Cc)
    ref = O.cpu_conv(x_hwc.ravel(), w_ohwc.ravel(), H, W, Cc, Kh, Kw, Oc)
    y = O.conv_nchw(np.ascontiguousarray(x_hwc.transpose(2, 0, 1))[None],
                    np.ascontiguousarray(w_ohwc.transpose(0, 3, 1, 2)), None, 0, 1)
    assert np.array_equal(bits(y.ravel()), bits(ref.ravel()))


# ---------------------------------------------------------------------------------------------
# emitted-program CPU references (src/codegen_hip.cpp)


@pytest.mark.parametrize("i", range(4))
def test_softmax_rmsnorm_channelscale_match_reference_vectors(i):
    L, Cc = (int(v) for v in G[f"softmax_{i}_shape"])
    x = G[f"softmax_{i}_x"].reshape(L, Cc)
    assert np.array_equal(bits(O.softmax(x)), bits(G[f"softmax_{i}_y"].reshape(L, Cc)))
    x = G[f"rmsnorm_{i}_x"].reshape(L, Cc)
    assert np.array_equal(bits(O.rmsnorm(x, G[f"rmsnorm_{i}_w"])), bits(G[f"rmsnorm_{i}_y"].reshape(L, Cc)))
    assert np.array_equal(bits(O.channelscale(x, G[f"channelscale_{i}_s"])),
                          bits(G[f"channelscale_{i}_y"].reshape(L, Cc)))


def test_softmax_closed_forms():
    # constant row -> 1/C; a shifted row gives the same result (max subtraction), and a row at
    # +-1000 must not overflow
    x = np.full((2, 64), 3.25, np.float32)
    assert np.all(O.softmax(x) == np.float32(1.0) / np.float32(64))
    r = np.array([[1000.0, 999.0, 998.0, -1000.0]], np.float32)
    e = np.exp(r.astype(np.float64) - 1000.0)
    want = e / e.sum()
    got = O.softmax(r)
    assert np.all(np.isfinite(got)) and np.allclose(got, want, rtol=1e-6, atol=0)
    assert np.array_equal(O.softmax(r), O.softmax(r - 1000.0))


def test_rmsnorm_closed_forms():
    # y = x * (1/sqrt(sum x^2 / C + eps)) * W; with x = 1e-3 the eps term doubles the mean square
    for v, Cc in ((1e-3, 64), (0.5, 256), (-2.0, 1000)):
        x = np.full((1, Cc), v, np.float32)
        W = O.normal(Cc, 5, 1.0, 0.1)
        ms = float(np.float32(v)) ** 2
        want = float(np.float32(v)) / np.sqrt(ms + 1e-6) * W.astype(np.float64)
        assert np.allclose(O.rmsnorm(x, W)[0], want, rtol=2e-6, atol=0)


@pytest.mark.parametrize("i", range(4))
def test_gemm_matches_reference_vectors(i):
    M, N, K = (int(v) for v in G[f"gemm_{i}_shape"])
    a, b = G[f"gemm_{i}_a"].reshape(M, K), G[f"gemm_{i}_b"].reshape(K, N)
    assert np.array_equal(bits(O.gemm_f32(a, b, b_colmajor=False).ravel()), bits(G[f"gemm_{i}_c_f32"]))
    # f16 program: inputs rounded to binary16 first, then the same f32 loop
    ah, bh = O.f16_bits(a), O.f16_bits(b)
    assert np.array_equal(bits(O.gemm_f16q(ah, bh, b_colmajor=False).ravel()), bits(G[f"gemm_{i}_c_f16"]))
    # column-major B (the BASELINE f16 layout) is the same product
    bt = np.ascontiguousarray(bh.reshape(K, N).T)
    assert np.array_equal(bits(O.gemm_f16q(ah, bt, b_colmajor=True).ravel()), bits(G[f"gemm_{i}_c_f16"]))


def test_gemm_against_binary64_and_transposition():
    M, N, K = 33, 17, 65
    a = O.uniform(M * K, 31, -1.0, 1.0).reshape(M, K)
    b = O.uniform(K * N, 32, -1.0, 1.0).reshape(K, N)
    c = O.gemm_f32(a, b, b_colmajor=False)
    r = a.astype(np.float64) @ b.astype(np.float64)
    bound = K * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert np.all(np.abs(c - r) <= bound)
    # a transposed operand must fail the same check
    wrong = a.astype(np.float64) @ np.ascontiguousarray(b.T.reshape(K, N)).astype(np.float64)
    assert not np.all(np.abs(c - wrong) <= bound)


def test_sawtooth_inputs_and_exact_products():
    # initA ((i % 17) - 8) / 16, initB ((i % 13) - 6) / 16 (src/codegen_hip.cpp:1122-1123)
    i = np.arange(4096)
    assert np.array_equal(G["saw_a"], (((i % 17) - 8) / 16).astype(np.float32))
    assert np.array_equal(G["saw_b"], (((i % 13) - 6) / 16).astype(np.float32))
    assert np.array_equal(O.sawtooth(4096, 17, 8), G["saw_a"])
    # every partial sum of a K <= 2^12 product of these is a multiple of 2^-8 below 2^16:
    # exact in f32, so any order equals the binary64 result
    M = N = K = 64
    a = O.sawtooth(M * K, 17, 8).reshape(M, K)
    b = O.sawtooth(K * N, 13, 6).reshape(K, N)
    assert np.array_equal(O.gemm_f32(a, b, b_colmajor=False), (a.astype(np.float64) @ b).astype(np.float32))


def test_tolerance_table_and_verify_metrics():
    # src/runtime.cpp:182-189 via the golden table: fp32 2^-5, fp16 2^-4, int8 0
    assert list(G["tolerance_for"]) == [0.03125, 0.0625, 0.0]
    # src/runtime.cpp:191-213 verify_fp32: binary64 |g - r| / max(1e-9, |r|), stops at the first
    # element above the tolerance and reports that element's error
    g, r = G["verify_got"].astype(np.float64), G["verify_ref"].astype(np.float64)
    ok, mr = G["verify_result"]
    e = np.abs(g - r) / np.maximum(1e-9, np.abs(r))
    bad = np.nonzero(e > 0.03125)[0]
    assert not ok and bad.size and mr == e[bad[0]]
    ok_part = slice(1, 97)  # a stretch without zero reference values
    # the emitted programs' metric (src/codegen_hip.cpp:1410-1416), in binary32 with a 1e-6 floor
    gf, rf = G["verify_got"][ok_part], G["verify_ref"][ok_part]
    with np.errstate(divide="ignore"):
        want = np.max(np.abs(gf - rf) / np.maximum(np.abs(rf), np.float32(1e-6)))
    assert O.oracle().or_max_rel(O.ptr(np.ascontiguousarray(gf)), O.ptr(np.ascontiguousarray(rf)), gf.size,
                                 1e-6) == pytest.approx(float(want), rel=1e-6)


# ---------------------------------------------------------------------------------------------
# Q8_0 (GGUF type 8): the reference has no Q8_0 path; the block definition is the oracle


def test_q8_0_pack_layout_and_dequant():
    N, K = 3, 128
    q = ((np.arange(N * K) * 37) % 255 - 127).astype(np.int8).reshape(N, K)
    d = O.f16_bits(O.uniform(N * K // 32, 3, 1e-3, 1e-2)).reshape(N, K // 32)
    blk = O.q8_0_pack(q, d)
    assert blk.dtype == np.uint8 and blk.size == N * (K // 32) * 34
    raw = blk.reshape(N, K // 32, 34)
    assert np.array_equal(raw[:, :, :2].copy().view(np.uint16)[..., 0], d)  # little-endian binary16 first
    assert np.array_equal(raw[:, :, 2:].view(np.int8).reshape(N, K), q)
    deq = O.q8_0_dequant(blk, N, K)
    want = (O.f16_to_f32(d.ravel()).reshape(N, K // 32).repeat(32, axis=1).astype(np.float64) * q)
    assert np.array_equal(deq.astype(np.float64), want)  # d*q is exact in binary32


def test_q8_0_gemm_binary64():
    M, N, K = 5, 7, 256
    q = ((np.arange(N * K) * 29) % 255 - 127).astype(np.int8).reshape(N, K)
    d = O.f16_bits(O.uniform(N * K // 32, 4, 1e-3, 1e-2)).reshape(N, K // 32)
    blk = O.q8_0_pack(q, d)
    Xh = O.f16_bits(O.normal(M * K, 5, 0.0, 1.0)).reshape(M, K)
    y = O.q8_0_gemm(Xh, blk, N)
    want = O.f16_to_f32(Xh).astype(np.float64) @ O.q8_0_dequant(blk, N, K).astype(np.float64).T
    assert np.allclose(y, want, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------------------------
# Live comparison with the reference build (this container only)


@pytest.mark.ref
def test_live_reference_matches_oracle(ref):
    x = O.normal(100003, 1, 0.0, 1.0)
    y1, y2 = np.zeros(1, np.float32), np.zeros(1, np.float32)
    ref.ref_cpu_reduce_blocked(O.ptr(x), O.ptr(y1), x.size, 1024)
    assert bits(y1) == bits(O.reduce_blocked(x, 1024))
    ref.ref_cpu_reduce(O.ptr(x), O.ptr(y2), x.size)
    y3 = np.zeros(1, np.float32)
    O.oracle().or_cpu_reduce(O.ptr(x), O.ptr(y3), x.size)
    assert bits(y2) == bits(y3)
    L, Cc = 16, 777
    X = O.normal(L * Cc, 2, 0.0, 8.0).reshape(L, Cc)
    r = np.zeros_like(X)
    ref.ref_emit_softmax(O.ptr(X), O.ptr(r), L, Cc)
    assert np.array_equal(bits(r), bits(O.softmax(X)))
    W = O.normal(Cc, 3, 1.0, 0.1)
    ref.ref_emit_rmsnorm(O.ptr(X), O.ptr(W), O.ptr(r), L, Cc)
    assert np.array_equal(bits(r), bits(O.rmsnorm(X, W)))
    M, N, K = 40, 24, 300
    a, b = O.uniform(M * K, 4, -1, 1).reshape(M, K), O.uniform(K * N, 5, -1, 1).reshape(K, N)
    c = np.zeros((M, N), np.float32)
    ref.ref_emit_gemm_f16(O.ptr(a), O.ptr(b), O.ptr(c), M, N, K)
    assert np.array_equal(bits(c), bits(O.gemm_f16q(O.f16_bits(a), O.f16_bits(b), b_colmajor=False)))
    H, Wd, Ci, Oc = 12, 11, 7, 6
    x = O.normal(H * Wd * Ci, 6, 0, 1)
    w = O.normal(Oc * 9 * Ci, 7, 0, 1)
    yr = np.zeros(Oc * (H - 2) * (Wd - 2), np.float32)
    ref.ref_cpu_conv(O.ptr(x), O.ptr(w), O.ptr(yr), H, Wd, Ci, 3, 3, Oc)
    assert np.array_equal(bits(yr), bits(O.cpu_conv(x, w, H, Wd, Ci, 3, 3, Oc).ravel()))
