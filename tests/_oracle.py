"""ctypes bindings of the CPU oracle (oracle/liboracle.so) and of the reference build
(oracle/_ref/libukref.so) — test infrastructure only. The oracle is the checker of the HIP path;
nothing here is part of the product.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libukref.so"

_P = C.c_void_p
_i, _f, _d, _sz, _u64, _i64 = C.c_int, C.c_float, C.c_double, C.c_size_t, C.c_uint64, C.c_int64

_ORACLE_SIG = {
    "or_f32_to_f16": ([_f], C.c_uint16),
    "or_f16_to_f32": ([C.c_uint16], _f),
    "or_f32_to_f16_n": ([_P, _P, _sz], None),
    "or_f16_to_f32_n": ([_P, _P, _sz], None),
    "or_splitmix64": ([C.POINTER(_u64)], _u64),
    "or_fill_uniform": ([_P, _sz, _u64, _f, _f], None),
    "or_fill_normal": ([_P, _sz, _u64, _f, _f], None),
    "or_fill_sawtooth": ([_P, _sz, _i, _i, _f, _f], None),
    "or_cpu_conv": ([_P, _P, _P] + [_i] * 6, None),
    "or_cpu_reduce": ([_P, _P, _i64], None),
    "or_cpu_reduce_blocked": ([_P, _P, _i64, _i], None),
    "or_gemm_f32": ([_P, _P, _P, _i, _i, _i, _i], None),
    "or_gemm_f16q": ([_P, _P, _P, _i, _i, _i, _i], None),
    "or_softmax": ([_P, _P, _i, _i], None),
    "or_rmsnorm": ([_P, _P, _P, _i, _i, _f], None),
    "or_channelscale": ([_P, _P, _P, _i, _i], None),
    "or_rowsum_blocked": ([_P, _P, _i, _i, _i], None),
    "or_rowsum_f64": ([_P, _P, _P, _i, _i], None),
    "or_conv_nchw": ([_P, _P, _P, _P] + [_i] * 9, None),
    "or_q8_0_dequant": ([_P, _P, _i, _i], None),
    "or_q8_0_gemm_f64": ([_P, _P, _P, _i, _i, _i], None),
    "or_q8_0_pack": ([_P, _P, _P, _i, _i], None),
    "or_max_rel": ([_P, _P, _sz, _d], _d),
    "or_frobenius_rel": ([_P, _P, _sz], _d),
    "or_softmax_mt": ([_P, _P, _i, _i, _i], None),
    "or_rmsnorm_mt": ([_P, _P, _P, _i, _i, _f, _i], None),
    "or_rowsum_blocked_mt": ([_P, _P, _i, _i, _i, _i], None),
    "or_gemm_f16q_mt": ([_P, _P, _P, _i, _i, _i, _i, _i], None),
    "or_gemm_f32_mt": ([_P, _P, _P, _i, _i, _i, _i, _i], None),
    "or_conv_nchw_mt": ([_P, _P, _P, _P] + [_i] * 10, None),
    "or_q8_0_gemm_f64_mt": ([_P, _P, _P, _i, _i, _i, _i], None),
}

_REF_SIG = {
    "ref_cpu_conv": ([_P, _P, _P] + [_i] * 6, None),
    "ref_cpu_reduce": ([_P, _P, C.c_longlong], None),
    "ref_cpu_reduce_blocked": ([_P, _P, C.c_longlong, _i], None),
    "ref_kref_reduce_width": ([], _i),
    "ref_kml_import": ([C.c_char_p, C.POINTER(_i), C.POINTER(_i), C.POINTER(_i), C.POINTER(_i), C.POINTER(_i),
                        C.c_char_p, _i, C.POINTER(_i), C.c_char_p, _i], _i),
    "ref_kml_canonical": ([C.c_char_p, C.c_char_p, _i], _i),
    "ref_kml_signature": ([C.c_char_p, C.c_char_p, _i], _i),
    "ref_kml_export": ([C.c_char_p, C.c_char_p, _i], _i),
    "ref_kml_tree_hash": ([C.c_char_p, C.c_char_p, _i], _i),
    "ref_workload": ([C.c_char_p, C.POINTER(C.c_longlong), C.POINTER(C.c_longlong)], _i),
    "ref_fnv1a": ([C.c_char_p, C.c_char_p, _i], _i),
    "ref_hcs_fingerprint": ([C.c_char_p, C.c_char_p, _i], _i),
    "ref_hcs_export": ([C.c_char_p, C.c_char_p, _i], _i),
    "ref_solve": ([C.c_char_p, C.c_char_p, C.POINTER(_i), C.POINTER(_i), C.POINTER(_i), C.POINTER(_d),
                   C.POINTER(_i)], _i),
    "ref_tolerance_for": ([_i], _d),
    "ref_verify_fp32": ([_P, _P, _i, _d, C.POINTER(_d)], _i),
    "ref_op_support_gap": ([C.c_char_p, C.c_char_p, _i], _i),
    "ref_emit_softmax": ([_P, _P, _i, _i], None),
    "ref_emit_rmsnorm": ([_P, _P, _P, _i, _i], None),
    "ref_emit_channelscale": ([_P, _P, _P, _i, _i], None),
    "ref_emit_gemm_f32": ([_P, _P, _P, _i, _i, _i], None),
    "ref_emit_gemm_f16": ([_P, _P, _P, _i, _i, _i], None),
    "ref_emit_float2half": ([_P, _P, C.c_longlong], None),
    "ref_emit_sawtooth_ab": ([_P, _P, _i], None),
}


def _bind(path: Path, sig: dict):
    lib = C.CDLL(str(path))
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


_oracle = None
_ref = None


def oracle():
    global _oracle
    if _oracle is None:
        if not ORACLE_SO.exists():
            raise RuntimeError(f"{ORACLE_SO} missing: run `make -C oracle` (or __graft_entry__.build())")
        _oracle = _bind(ORACLE_SO, _ORACLE_SIG)
    return _oracle


def ref_available() -> bool:
    return REF_SO.exists()


def ref():
    global _ref
    if _ref is None:
        _ref = _bind(REF_SO, _REF_SIG)
    return _ref


def ptr(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(C.c_void_p)


# ---- numpy conveniences over the oracle ----
def f16_bits(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, np.uint16)
    oracle().or_f32_to_f16_n(ptr(a), ptr(out), a.size)
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    oracle().or_f16_to_f32_n(ptr(h), ptr(out), h.size)
    return out


def uniform(n: int, seed: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    oracle().or_fill_uniform(ptr(out), n, seed, lo, hi)
    return out


def normal(n: int, seed: int, mu: float, sigma: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    oracle().or_fill_normal(ptr(out), n, seed, mu, sigma)
    return out


def sawtooth(n: int, period: int, offset: int, unit: float = 0.0625, bias: float = 0.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    oracle().or_fill_sawtooth(ptr(out), n, period, offset, unit, bias)
    return out


def softmax(X: np.ndarray, threads: int = 8) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    Y = np.empty_like(X)
    oracle().or_softmax_mt(ptr(X), ptr(Y), X.shape[0], X.shape[1], threads)
    return Y


def rmsnorm(X: np.ndarray, W: np.ndarray, eps: float = 1e-6, threads: int = 8) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    Y = np.empty_like(X)
    oracle().or_rmsnorm_mt(ptr(X), ptr(W), ptr(Y), X.shape[0], X.shape[1], eps, threads)
    return Y


def rowsum_blocked(X: np.ndarray, width: int = 1024, threads: int = 8) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    Y = np.empty(X.shape[0], np.float32)
    oracle().or_rowsum_blocked_mt(ptr(X), ptr(Y), X.shape[0], X.shape[1], width, threads)
    return Y


def rowsum_f64(X: np.ndarray):
    X = np.ascontiguousarray(X, np.float32)
    Y = np.empty(X.shape[0], np.float64)
    A = np.empty(X.shape[0], np.float64)
    oracle().or_rowsum_f64(ptr(X), ptr(Y), ptr(A), X.shape[0], X.shape[1])
    return Y, A


def channelscale(X: np.ndarray, S: np.ndarray) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    S = np.ascontiguousarray(S, np.float32)
    Y = np.empty_like(X)
    oracle().or_channelscale(ptr(X), ptr(S), ptr(Y), X.shape[0], X.shape[1])
    return Y


def reduce_blocked(x: np.ndarray, width: int = 1024) -> np.float32:
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(1, np.float32)
    oracle().or_cpu_reduce_blocked(ptr(x), ptr(y), x.size, width)
    return y[0]


def gemm_f16q(Ah: np.ndarray, Bh: np.ndarray, b_colmajor: bool, threads: int = 8) -> np.ndarray:
    """Ah [M][K] f16 bits; Bh [N][K] (b_colmajor) or [K][N] f16 bits -> f32 [M][N]."""
    Ah = np.ascontiguousarray(Ah, np.uint16)
    Bh = np.ascontiguousarray(Bh, np.uint16)
    M, K = Ah.shape
    N = Bh.shape[0] if b_colmajor else Bh.shape[1]
    Cm = np.empty((M, N), np.float32)
    oracle().or_gemm_f16q_mt(ptr(Ah), ptr(Bh), ptr(Cm), M, N, K, int(b_colmajor), threads)
    return Cm


def gemm_f32(A: np.ndarray, B: np.ndarray, b_colmajor: bool, threads: int = 8) -> np.ndarray:
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    M, K = A.shape
    N = B.shape[0] if b_colmajor else B.shape[1]
    Cm = np.empty((M, N), np.float32)
    oracle().or_gemm_f32_mt(ptr(A), ptr(B), ptr(Cm), M, N, K, int(b_colmajor), threads)
    return Cm


def conv_nchw(x, w, scale, pad: int, stride: int = 1, threads: int = 8) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    N, Cin, H, W = x.shape
    Oc, _, Kh, Kw = w.shape
    Ho, Wo = (H + 2 * pad - Kh) // stride + 1, (W + 2 * pad - Kw) // stride + 1
    y = np.empty((N, Oc, Ho, Wo), np.float32)
    sp = None if scale is None else ptr(np.ascontiguousarray(scale, np.float32))
    s_keep = scale
    oracle().or_conv_nchw_mt(ptr(x), ptr(w), sp, ptr(y), N, Cin, H, W, Oc, Kh, Kw, pad, stride, threads)
    del s_keep
    return y


def cpu_conv(x, wt, H, W, Cc, Kh, Kw, Oc) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    wt = np.ascontiguousarray(wt, np.float32)
    y = np.empty((Oc, H - Kh + 1, W - Kw + 1), np.float32)
    oracle().or_cpu_conv(ptr(x), ptr(wt), ptr(y), H, W, Cc, Kh, Kw, Oc)
    return y


def q8_0_pack(q: np.ndarray, d_bits: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, np.int8)
    d_bits = np.ascontiguousarray(d_bits, np.uint16)
    N, K = q.shape
    blocks = np.empty(N * (K // 32) * 34, np.uint8)
    oracle().or_q8_0_pack(ptr(q), ptr(d_bits), ptr(blocks), N, K)
    return blocks


def q8_0_dequant(blocks: np.ndarray, N: int, K: int) -> np.ndarray:
    out = np.empty((N, K), np.float32)
    oracle().or_q8_0_dequant(ptr(np.ascontiguousarray(blocks)), ptr(out), N, K)
    return out


def q8_0_gemm(Xh: np.ndarray, blocks: np.ndarray, N: int, threads: int = 8) -> np.ndarray:
    Xh = np.ascontiguousarray(Xh, np.uint16)
    M, K = Xh.shape
    Y = np.empty((M, N), np.float64)
    oracle().or_q8_0_gemm_f64_mt(ptr(Xh), ptr(np.ascontiguousarray(blocks)), ptr(Y), M, N, K, threads)
    return Y
