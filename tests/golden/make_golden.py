"""Writes the golden fixtures of this directory from the reference's own code.

Run in a container that holds the reference tree, after `make -C oracle ref` has compiled the
reference sources into oracle/_ref/libukref.so:

    python tests/golden/make_golden.py

Outputs (data only — inputs and the reference's outputs):
  numerics.npz  reference CPU functions (src/reference.cpp:6-48) and the CPU sections of its
                emitted programs (src/codegen_hip.cpp:1124-1132, :1854-1862, :1999-2009,
                :2168-2178, :2339-2344) on small seeded inputs, plus tolerance_for and verify_fp32
                (src/runtime.cpp:182-213).
  front.json    the reference front end on KML and HCS texts: kml_import verdicts and messages,
                canonical_form, fnv1a tree hash, op_signature, kml_export, workload_of and
                op_support_gap (src/kml_front.cpp, src/kml.cpp:57-177, src/codegen_hip.cpp:81-130),
                hcs_fingerprint / hcs_export (src/hcs.cpp:52-115) and solve's tile pick
                (src/solver.cpp:141-186) for the reference's sample HCS files.
Inputs are generated with the oracle's SplitMix64 streams and stored in the fixture, so the
tests need neither the reference nor the generator to replay them.
"""
from __future__ import annotations

import ctypes as C
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
import _oracle as O  # noqa: E402

REF_SAMPLES = Path("/root/reference/samples")


def _s(fn, text: str, cap: int = 1 << 16):
    buf = C.create_string_buffer(cap)
    n = fn(text.encode(), buf, cap)
    return None if n < 0 else buf.value.decode()


def numerics(R) -> dict:
    out = {}
    # cpu_reduce / cpu_reduce_blocked (src/reference.cpp:24-48)
    for n in (0, 1, 3, 1023, 1024, 1025, 4097, 20011):
        x = O.normal(n, 7000 + n, 0.0, 1.0) if n else np.zeros(0, np.float32)
        y = np.zeros(1, np.float32)
        R.ref_cpu_reduce(O.ptr(x), O.ptr(y), n)
        yb = np.zeros(1, np.float32)
        R.ref_cpu_reduce_blocked(O.ptr(x), O.ptr(yb), n, 1024)
        out[f"reduce_x_{n}"] = x
        out[f"reduce_y_{n}"] = y
        out[f"reduce_blocked_y_{n}"] = yb
    # cpu_conv (src/reference.cpp:6-22): X[H][W][C], Wt[Oc][Kh][Kw][C], Y[Oc][Ho][Wo]
    for i, (H, W, Cc, Kh, Kw, Oc) in enumerate([(5, 6, 3, 3, 3, 4), (9, 7, 8, 3, 3, 5), (4, 4, 2, 1, 1, 3),
                                                 (8, 10, 6, 5, 3, 2), (6, 6, 17, 3, 3, 9)]):
        x = O.normal(H * W * Cc, 7100 + i, 0.0, 1.0)
        w = O.normal(Oc * Kh * Kw * Cc, 7200 + i, 0.0, 0.3)
        y = np.zeros(Oc * (H - Kh + 1) * (W - Kw + 1), np.float32)
        R.ref_cpu_conv(O.ptr(x), O.ptr(w), O.ptr(y), H, W, Cc, Kh, Kw, Oc)
        out[f"conv_{i}_shape"] = np.array([H, W, Cc, Kh, Kw, Oc], np.int32)
        out[f"conv_{i}_x"], out[f"conv_{i}_w"], out[f"conv_{i}_y"] = x, w, y
    # emitted CPU references
    for i, (L, Cc) in enumerate([(3, 5), (7, 256), (4, 1000), (1, 4096)]):
        x = O.normal(L * Cc, 7300 + i, 0.0, 8.0)
        y = np.zeros_like(x)
        R.ref_emit_softmax(O.ptr(x), O.ptr(y), L, Cc)
        out[f"softmax_{i}_shape"] = np.array([L, Cc], np.int32)
        out[f"softmax_{i}_x"], out[f"softmax_{i}_y"] = x, y
        x = O.normal(L * Cc, 7400 + i, 0.0, 1.0)
        w = O.normal(Cc, 7500 + i, 1.0, 0.1)
        y = np.zeros_like(x)
        R.ref_emit_rmsnorm(O.ptr(x), O.ptr(w), O.ptr(y), L, Cc)
        out[f"rmsnorm_{i}_shape"] = np.array([L, Cc], np.int32)
        out[f"rmsnorm_{i}_x"], out[f"rmsnorm_{i}_w"], out[f"rmsnorm_{i}_y"] = x, w, y
        s = O.uniform(Cc, 7600 + i, 0.5, 1.5)
        y = np.zeros_like(x)
        R.ref_emit_channelscale(O.ptr(x), O.ptr(s), O.ptr(y), L, Cc)
        out[f"channelscale_{i}_s"], out[f"channelscale_{i}_y"] = s, y
    for i, (M, N, K) in enumerate([(1, 1, 1), (5, 7, 3), (17, 33, 65), (64, 48, 128)]):
        a = O.uniform(M * K, 7700 + i, -1.0, 1.0)
        b = O.uniform(K * N, 7800 + i, -1.0, 1.0)
        c = np.zeros(M * N, np.float32)
        R.ref_emit_gemm_f32(O.ptr(a), O.ptr(b), O.ptr(c), M, N, K)
        ch = np.zeros(M * N, np.float32)
        R.ref_emit_gemm_f16(O.ptr(a), O.ptr(b), O.ptr(ch), M, N, K)
        out[f"gemm_{i}_shape"] = np.array([M, N, K], np.int32)
        out[f"gemm_{i}_a"], out[f"gemm_{i}_b"] = a, b
        out[f"gemm_{i}_c_f32"], out[f"gemm_{i}_c_f16"] = c, ch
    # __float2half of the emitted f16 program on special and random values
    v = np.concatenate([np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65520.0, 65519.99, 1e-8, 5.96e-8, 2.98e-8,
                                  2.9802322e-8, 6.1035156e-5, np.inf, -np.inf, 1.0009765625, 1.00048828125,
                                  1.000732421875, 3.0e-5, -7.0e4], np.float32),
                        O.normal(2048, 7900, 0.0, 100.0), O.uniform(2048, 7901, -1e-4, 1e-4)]).astype(np.float32)
    h = np.zeros(v.size, np.uint16)
    R.ref_emit_float2half(O.ptr(v), O.ptr(h), v.size)
    out["f2h_x"], out["f2h_h"] = v, h
    # reference sawtooth inputs of the emitted gemm (initA/initB)
    a = np.zeros(4096, np.float32)
    b = np.zeros(4096, np.float32)
    R.ref_emit_sawtooth_ab(O.ptr(a), O.ptr(b), 4096)
    out["saw_a"], out["saw_b"] = a, b
    # tolerance table and verify metric
    out["tolerance_for"] = np.array([R.ref_tolerance_for(d) for d in range(3)], np.float64)
    g = O.normal(1000, 8000, 0.0, 1.0)
    r = (g * (1 + O.uniform(1000, 8001, -0.04, 0.04))).astype(np.float32)
    r[::97] = 0.0
    mr = C.c_double()
    ok = R.ref_verify_fp32(O.ptr(g), O.ptr(r), 1000, 0.03125, C.byref(mr))
    out["verify_got"], out["verify_ref"] = g, r
    out["verify_result"] = np.array([ok, mr.value], np.float64)
    return out


def kml_cases() -> list[str]:
    cases = []
    for p in sorted(REF_SAMPLES.glob("kml_*.json")) + sorted(REF_SAMPLES.glob("*.kml")):
        cases.append(p.read_text())
    one = lambda **kv: json.dumps(kv)  # noqa: E731
    cases += [
        one(op="gemm", dtype="fp32", dims=[4096, 4096, 4096]),
        one(op="gemm", dtype="fp16", dims=[4096, 4096, 4096], layout="NT"),
        one(op="gemm", dtype="int8", dims=[64, 64, 64]),
        one(op="gemm", dtype="fp32", dims=[1, 2, 3], tile_m=32, tile_n=96),
        one(op="reduce", dtype="fp32", dims=[1024]),
        one(op="reduce", dtype="fp16", dims=[1024]),
        one(op="softmax", dtype="fp32", dims=[4096, 4096]),
        one(op="rmsnorm", dtype="fp32", dims=[4096, 4096]),
        one(op="channelscale", dtype="fp32", dims=[8, 64]),
        one(op="conv", dtype="fp32", dims=[56, 56, 64, 3, 3, 64]),
        one(op="conv", dtype="fp16", dims=[8, 8, 4, 3, 3, 4]),
        # rejections
        one(dtype="fp32", dims=[4]),
        one(op="matmul", dtype="fp32", dims=[4, 4, 4]),
        one(op="gemm", dtype="bf16", dims=[4, 4, 4]),
        one(op="gemm", dtype="fp32", dims=[4, 4]),
        one(op="gemm", dtype="fp32", dims=[4, -4, 4]),
        one(op="gemm", dtype="fp32", dims=[4, 0, 4]),
        one(op="reduce", dtype="fp32", dims=[2147483648]),
        one(op="reduce", dtype="fp32", dims=[2147483647]),
        one(op="reduce", dtype="fp32", dims=[1048576], tile_m=99999999999),
        one(op="gemm", dtype="fp32", dims=[4, 4, 4], layout="TN"),
        one(op="gemm", dtype="fp32", dims=[4, 4, 4], colour="red"),
        one(op="softmax", dtype="fp32", dims=[4]),
        one(op="conv", dtype="fp32", dims=[2, 2, 1, 3, 3, 1]),
        one(op="gemm", dtype="fp32", dims=[4, 4, 4], tile_m=-8),
        '{"op": "gemm", "dtype": "fp32", "dims": [4, 4, 4]',
        "[]",
        "",
        # children: commutative normalisation and path-prefixed errors
        one(op="gemm", dtype="fp32", dims=[8, 8, 8],
            children=[dict(op="reduce", dtype="fp32", dims=[64]), dict(op="softmax", dtype="fp32", dims=[4, 8])]),
        one(op="gemm", dtype="fp32", dims=[8, 8, 8],
            children=[dict(op="softmax", dtype="fp32", dims=[4, 8]), dict(op="reduce", dtype="fp32", dims=[64])]),
        one(op="gemm", dtype="fp32", dims=[8, 8, 8], children=[dict(op="reduce", dtype="fp99", dims=[64])]),
        one(op="gemm", dtype="fp32", dims=[8, 8, 8], children=[dict(dtype="fp32", dims=[64, 2, 2])]),
    ]
    return cases


def front(R) -> dict:
    kml = []
    for text in kml_cases():
        op, dt, nch, tm, tn = (C.c_int() for _ in range(5))
        dims = (C.c_int * 6)()
        lay = C.create_string_buffer(64)
        err = C.create_string_buffer(1 << 16)
        ok = R.ref_kml_import(text.encode(), C.byref(op), C.byref(dt), dims, C.byref(tm), C.byref(tn), lay, 64,
                              C.byref(nch), err, 1 << 16)
        rec = {"text": text, "accepted": bool(ok)}
        if ok:
            ops, nbytes = C.c_longlong(), C.c_longlong()
            R.ref_workload(text.encode(), C.byref(ops), C.byref(nbytes))
            rec.update(op=op.value, dtype=dt.value, dims=list(dims), tile_m=tm.value, tile_n=tn.value,
                       layout=lay.value.decode(), n_children=nch.value,
                       canonical=_s(R.ref_kml_canonical, text), signature=_s(R.ref_kml_signature, text),
                       export=_s(R.ref_kml_export, text), tree_hash=_s(R.ref_kml_tree_hash, text),
                       ops=ops.value, bytes=nbytes.value, support_gap=_s(R.ref_op_support_gap, text))
        else:
            rec["error"] = err.value.decode()
        kml.append(rec)
    hcs = []
    hcs_texts = [p.read_text() for p in sorted(REF_SAMPLES.glob("hcs_*.json"))]
    hcs_texts += ['{"vendor":"amd"}', '{"vendor": "amd", "device": "x", "unified_memory": false}', "not json"]
    for text in hcs_texts:
        fp = C.create_string_buffer(1 << 16)
        ok = R.ref_hcs_fingerprint(text.encode(), fp, 1 << 16)
        rec = {"text": text, "accepted": bool(ok)}
        if ok:
            rec.update(fingerprint=fp.value.decode(), export=_s(R.ref_hcs_export, text))
            picks = []
            for k in kml:
                if not k["accepted"]:
                    continue
                tm, tn, path, fc = C.c_int(), C.c_int(), C.c_int(), C.c_int()
                cms = C.c_double()
                if R.ref_solve(text.encode(), k["text"].encode(), C.byref(tm), C.byref(tn), C.byref(path),
                               C.byref(cms), C.byref(fc)):
                    picks.append({"kml": k["text"], "tile_m": tm.value, "tile_n": tn.value, "path": path.value,
                                  "c_ms": cms.value, "feasible": fc.value})
            rec["solve"] = picks
        else:
            rec["error"] = fp.value.decode()
        hcs.append(rec)
    fnv = {s: _s(R.ref_fnv1a, s) for s in ["", "a", "foobar", "unikern", "gemm:fp32:4096x4096x4096"]}
    return {"kml": kml, "hcs": hcs, "fnv1a": fnv, "kref_reduce_width": R.ref_kref_reduce_width()}


def main():
    if not O.ref_available():
        sys.exit("oracle/_ref/libukref.so is missing: run `make -C oracle ref` in a container with the reference")
    R = O.ref()
    np.savez_compressed(HERE / "numerics.npz", **numerics(R))
    (HERE / "front.json").write_text(json.dumps(front(R), indent=1, ensure_ascii=False) + "\n")
    print("wrote", HERE / "numerics.npz", HERE / "front.json")


if __name__ == "__main__":
    main()
