"""unikern_amd — UNIKERN's kernel hot path, native to one MI355X (gfx950).

Python face of libunikern_hip.so (include/unikern_hip.h). It mirrors the reference's C++
interface for the path (include/unikern/components.hpp, include/unikern/codegen.hpp):

    kml_import / kml_export / canonical_form / op_signature / workload_of   (src/kml_front.cpp, src/kml.cpp)
    hcs_fingerprint / hcs_export                                           (src/hcs.cpp)
    solve                                                                  (src/solver.cpp)
    run -> RunOutcome                                                      (run_hip, src/runner.cpp:146-238)
    launch                                                                 (raw operator on device buffers)

There is no CPU fallback: importing fails when the library is missing, and every execution
entry point runs the HIP kernels.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from . import _capi
from ._capi import (DTYPES, FAMILIES, LAYOUTS, OPS, UK_BAD_INVOCATION, UK_HIP_FAILURE, UK_INFEASIBLE, UK_OK,
                    UK_RESIDENCY, UK_VERIFY_FAIL, MfmaProbe, OpDesc, Plan, Result)

lib = _capi.load()
CLI = Path(__file__).resolve().parent / "unikern"  # the command-line front door (built with the library)

SEED = 20261201
ROOT = Path(__file__).resolve().parent.parent
SAMPLES = ROOT / "samples"


class KmlError(ValueError):
    """A rejected KML declaration; the message lists every violation."""


class UnikernError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


def last_error() -> str:
    e = lib.uk_last_error()
    return e.decode() if e else ""


def _buf(n: int = 1 << 16):
    return C.create_string_buffer(n)


def _text(json_text: str | bytes) -> bytes:
    return json_text.encode() if isinstance(json_text, str) else json_text


# ---------------------------------------------------------------------------------------
# KML front end
# ---------------------------------------------------------------------------------------
def kml_import(text: str) -> OpDesc:
    d = OpDesc()
    err = _buf()
    rc = lib.uk_kml_import(_text(text), C.byref(d), err, len(err))
    if rc != UK_OK:
        raise KmlError(err.value.decode())
    return d


def kml_load(path: str | Path) -> OpDesc:
    return kml_import(Path(path).read_text())


def _str_call(fn, text) -> str:
    out = _buf()
    n = fn(_text(text), out, len(out))
    if n < 0:
        raise KmlError(last_error())
    return out.value.decode()


def kml_export(text: str) -> str:
    return _str_call(lib.uk_kml_export, text)


def canonical_form(text: str) -> str:
    return _str_call(lib.uk_kml_canonical, text)


def tree_hash(text: str) -> str:
    return _str_call(lib.uk_kml_tree_hash, text)


def op_signature(d: OpDesc) -> str:
    out = _buf(256)
    if lib.uk_op_signature(C.byref(d), out, len(out)) < 0:
        raise KmlError(last_error())
    return out.value.decode()


def workload_of(d: OpDesc) -> dict:
    ops, nbytes, wbytes = C.c_int64(), C.c_int64(), C.c_int64()
    rc = lib.uk_workload(C.byref(d), C.byref(ops), C.byref(nbytes), C.byref(wbytes))
    if rc != UK_OK:
        raise KmlError(last_error())
    return {"ops": ops.value, "bytes": nbytes.value, "weight_bytes": wbytes.value}


def support_gap(d: OpDesc) -> str:
    out = _buf(1024)
    lib.uk_support_gap(C.byref(d), out, len(out))
    return out.value.decode()


def make_desc(op: str, dims, dtype: str = "fp32", layout: str = "NT", *, batch: int = 1, pad: int = 0,
              stride: int = 1, epilogue: str = "none", eps: float = 1e-6, tile_m: int = 64,
              tile_n: int = 128) -> OpDesc:
    """Build a descriptor directly (same meaning as a KML declaration)."""
    d = OpDesc()
    d.op, d.dtype, d.layout = OPS[op], DTYPES[dtype], LAYOUTS[layout]
    d.epilogue = 1 if epilogue == "channelscale" else 0
    d.ndims = len(dims)
    for i, v in enumerate(dims):
        d.dims[i] = int(v)
    d.tile_m, d.tile_n = tile_m, tile_n
    d.batch, d.pad, d.stride, d.eps = batch, pad, stride, eps
    return d


# ---------------------------------------------------------------------------------------
# HCS + solver
# ---------------------------------------------------------------------------------------
def hcs_fingerprint(hcs_json: str | None = None) -> str:
    out = _buf(256)
    rc = lib.uk_hcs_fingerprint(None if hcs_json is None else _text(hcs_json), out, len(out))
    if rc != UK_OK:
        raise ValueError(out.value.decode())
    return out.value.decode()


def hcs_export(hcs_json: str | None = None) -> str:
    out = _buf()
    n = lib.uk_hcs_export(None if hcs_json is None else _text(hcs_json), out, len(out))
    if n < 0:
        raise ValueError(last_error())
    return out.value.decode()


@dataclass
class Solution:
    plan: Plan
    family: str
    key: str
    predicted_us: float
    feasible: int
    log: str


def solve(d: OpDesc, hcs_json: str | None = None) -> Solution:
    p = Plan()
    log = _buf()
    rc = lib.uk_solve(None if hcs_json is None else _text(hcs_json), C.byref(d), C.byref(p), log, len(log))
    if rc != UK_OK:
        raise UnikernError(rc, log.value.decode() or last_error())
    return Solution(p, FAMILIES.get(p.family, "?"), p.key.decode(), p.predicted_us, p.feasible, log.value.decode())


# ---------------------------------------------------------------------------------------
# Execution
# ---------------------------------------------------------------------------------------
@dataclass
class RunOutcome:
    """Mirror of the reference's RunOutcome (include/unikern/codegen.hpp:49-83) plus roofline."""
    built: bool
    ran: bool
    verified: bool
    exit_code: int
    max_rel: float
    err_metric: float
    tol: float
    kernel_ms: float
    measured_ms: float
    achieved: float
    peak: float
    frac: float
    bound: str
    migrations: int
    checks: int
    vram_free: int
    vram_total: int
    plan_key: str
    family: str
    sets: int
    log: str
    line: str
    cpu_ms: float = -1.0      # the run's own CPU reference pass (binary64, over the outputs it checks)
    cpu_cores: int = -1       # host threads that pass ran on
    cpu_outputs: int = -1     # outputs it computed (all, or the sampled rows/images)
    stream_path: str = ""     # a streamed run's data path for A: "pinned" or "mmap"
    raw: Result = field(repr=False, default=None)


def run(d: OpDesc, *, seed: int = SEED, exact: bool = False, iters: int = 50, plan: Plan | None = None,
        hcs_json: str | None = None) -> RunOutcome:
    r = Result()
    log = _buf(1 << 16)
    rc = lib.uk_run(None if hcs_json is None else _text(hcs_json), C.byref(d),
                    None if plan is None else C.byref(plan), seed, 1 if exact else 0, iters, C.byref(r), log,
                    len(log))
    return _outcome(r, rc, log.value.decode())


def _outcome(r: Result, rc: int, log: str) -> RunOutcome:
    line = _buf(2048)
    lib.uk_format_result(C.byref(r), line, len(line))
    return RunOutcome(bool(r.built), bool(r.ran), bool(r.verified), rc, r.max_rel, r.err_metric, r.tol, r.kernel_ms,
                      r.measured_ms, r.achieved, r.peak, r.frac, "mfma" if r.bound == 1 else "hbm", r.migrations,
                      r.checks, r.vram_free, r.vram_total, r.plan.key.decode(), FAMILIES.get(r.plan.family, "?"),
                      r.sets, log, line.value.decode(), r.cpu_ms, r.cpu_cores, r.cpu_outputs,
                      r.stream_path.decode(), r)


def parse_result(program_output: str, exit_code: int) -> RunOutcome:
    """A program's output parsed as the reference's run_hip parses it (src/runner.cpp:195-237)."""
    r = Result()
    _check(lib.uk_parse_result(program_output.encode(), exit_code, C.byref(r)))
    return _outcome(r, exit_code, program_output)


def migration_alarm(migrations: int, checks: int, threshold: float) -> tuple[bool, float]:
    """(violation, rate) of a residency report (reference migration_rate_violation,
    src/runner.cpp:240-255)."""
    rate = C.c_double(-1.0)
    v = lib.uk_migration_alarm(migrations, checks, threshold, C.byref(rate))
    return bool(v), rate.value


def residency_class(probe_status: int, memory_type: int) -> int:
    """Exit class (0, 4 or 5) of one allocation's residency probe (src/codegen_hip.cpp:256-280)."""
    return lib.uk_residency_class(probe_status, memory_type)


def device_check() -> str:
    arch = _buf(128)
    rc = lib.uk_device_check(arch, len(arch))
    if rc != UK_OK:
        raise UnikernError(rc, last_error())
    return arch.value.decode()


def device_props() -> dict:
    cus, lds, clk = C.c_int32(), C.c_int32(), C.c_int32()
    tot = C.c_uint64()
    rc = lib.uk_device_props(C.byref(cus), C.byref(lds), C.byref(clk), C.byref(tot))
    if rc != UK_OK:
        raise UnikernError(rc, last_error())
    return {"compute_units": cus.value, "lds_per_block": lds.value, "clock_khz": clk.value,
            "total_bytes": tot.value}


def probe_mfma() -> dict:
    """Matrix-core ceiling of the device (uk_probe_mfma): sustained f16 MFMA TFLOP/s, the shader
    clock under that load and the issue cycles per MFMA, for v_mfma_f32_16x16x32_f16 and (keys
    ending in _32x32) v_mfma_f32_32x32x16_f16."""
    r = MfmaProbe()
    rc = lib.uk_probe_mfma(C.byref(r))
    if rc != UK_OK:
        raise UnikernError(rc, last_error())
    return {"tflops": r.tflops, "clock_ghz": r.clock_ghz, "cycles_per_mfma": r.cycles_per_mfma,
            "ms_per_launch": r.ms_per_launch, "workgroups": r.workgroups, "mfmas_per_wave": r.mfmas_per_wave,
            "tflops_32x32": r.tflops_32x32, "clock_ghz_32x32": r.clock_ghz_32x32,
            "cycles_per_mfma_32x32": r.cycles_per_mfma_32x32}


def _check(rc: int):
    if rc != UK_OK:
        raise UnikernError(rc, last_error())


class DeviceBuffer:
    """Device allocation owned by Python; copies to/from numpy arrays."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        _check(lib.uk_malloc(C.byref(p), self.nbytes))
        self.ptr = p

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        _check(lib.uk_memcpy_htod(self.ptr, a.ctypes.data_as(C.c_void_p), a.nbytes))

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        _check(lib.uk_memcpy_dtoh(out.ctypes.data_as(C.c_void_p), self.ptr, out.nbytes))
        return out

    def fill(self, value: int):
        _check(lib.uk_memset(self.ptr, value, self.nbytes))

    def free(self):
        if self.ptr:
            lib.uk_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def launch(d: OpDesc, ins, out: DeviceBuffer, plan: Plan | None = None, stream=None, sync: bool = True):
    arr = (C.c_void_p * len(ins))(*[b.ptr for b in ins])
    rc = lib.uk_launch(C.byref(d), None if plan is None else C.byref(plan), arr, len(ins), out.ptr, stream)
    _check(rc)
    if sync:
        _check(lib.uk_synchronize())


def synchronize():
    _check(lib.uk_synchronize())


def stream_gemm(d: OpDesc, A: np.ndarray, B: np.ndarray, plan: Plan | None = None,
                hcs_json: str | None = None) -> tuple[np.ndarray, float]:
    """Scenario-B GEMM on host operands (uk_stream_gemm): (C, pass_ms). A [M][K], B as the layout
    says ([K][N] NT, [N][K] TN), both f16 bits (uint16) or f32 as the descriptor's dtype says; C
    comes back in the same element type. The library copies rows straight out of the arrays, so
    their shapes and element type are checked against the descriptor first."""
    if d.op != OPS["gemm"] or d.ndims != 3:
        raise UnikernError(UK_BAD_INVOCATION, "stream_gemm: the descriptor is not a gemm [M, N, K]")
    M, N, K = (int(d.dims[i]) for i in range(3))
    want = {DTYPES["fp16"]: np.uint16, DTYPES["fp32"]: np.float32}.get(int(d.dtype))
    if want is None:
        raise UnikernError(UK_BAD_INVOCATION, "stream_gemm: only fp16 and fp32 GEMMs stream")
    b_shape = (N, K) if d.layout == LAYOUTS["TN"] else (K, N)
    for name, arr, shape in (("A", A, (M, K)), ("B", B, b_shape)):
        if arr.dtype != want or tuple(arr.shape) != shape:
            raise UnikernError(UK_BAD_INVOCATION, f"stream_gemm: {name} is {arr.dtype}{tuple(arr.shape)}, the "
                                                  f"descriptor needs {np.dtype(want)}{shape}")
    A = np.ascontiguousarray(A)
    B = np.ascontiguousarray(B)
    Cm = np.empty((M, N), dtype=want)
    ms = C.c_double()
    _check(lib.uk_stream_gemm(None if hcs_json is None else _text(hcs_json), C.byref(d),
                              None if plan is None else C.byref(plan), A.ctypes.data_as(C.c_void_p),
                              B.ctypes.data_as(C.c_void_p), Cm.ctypes.data_as(C.c_void_p), C.byref(ms)))
    return Cm, ms.value


def stream_gemm_file(d: OpDesc, a_path: str | Path, B: np.ndarray, plan: Plan | None = None,
                     hcs_json: str | None = None) -> tuple[np.ndarray, float]:
    """Scenario B's mapped path (uk_stream_gemm_file): (C, pass_ms) with A [M][K] read from the file
    at a_path (raw elements of the descriptor's dtype, row-major) shard by shard into host-mapped
    staging that the kernel reads directly; B as for stream_gemm. The library refuses a file
    shorter than M K elements."""
    if d.op != OPS["gemm"] or d.ndims != 3:
        raise UnikernError(UK_BAD_INVOCATION, "stream_gemm_file: the descriptor is not a gemm [M, N, K]")
    M, N, K = (int(d.dims[i]) for i in range(3))
    want = {DTYPES["fp16"]: np.uint16, DTYPES["fp32"]: np.float32}.get(int(d.dtype))
    if want is None:
        raise UnikernError(UK_BAD_INVOCATION, "stream_gemm_file: only fp16 and fp32 GEMMs stream")
    b_shape = (N, K) if d.layout == LAYOUTS["TN"] else (K, N)
    if B.dtype != want or tuple(B.shape) != b_shape:
        raise UnikernError(UK_BAD_INVOCATION, f"stream_gemm_file: B is {B.dtype}{tuple(B.shape)}, the descriptor "
                                              f"needs {np.dtype(want)}{b_shape}")
    B = np.ascontiguousarray(B)
    Cm = np.empty((M, N), dtype=want)
    ms = C.c_double()
    _check(lib.uk_stream_gemm_file(None if hcs_json is None else _text(hcs_json), C.byref(d),
                                   None if plan is None else C.byref(plan), str(a_path).encode(),
                                   B.ctypes.data_as(C.c_void_p), Cm.ctypes.data_as(C.c_void_p), C.byref(ms)))
    return Cm, ms.value


class Stream:
    """A HIP stream at the default priority (uk_stream_create); pass .ptr as launch(stream=...)."""

    def __init__(self):
        p = C.c_void_p()
        _check(lib.uk_stream_create(C.byref(p)))
        self.ptr = p

    def synchronize(self):
        _check(lib.uk_stream_synchronize(self.ptr))

    def destroy(self):
        if self.ptr:
            self.synchronize()
            _check(lib.uk_stream_destroy(self.ptr))
            self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.destroy()


# ---------------------------------------------------------------------------------------
# Solution ledger (reference ILedger: include/unikern/components.hpp:83-125)
# ---------------------------------------------------------------------------------------
@dataclass
class LedgerHit:
    plan: Plan
    c_ms: float
    measured_ms: float
    kernel_ms: float


class Ledger:
    """A ".jsonl" path opens the text ledger, any other path SQLite (the reference's schema)."""

    def __init__(self, path: str | Path):
        h = C.c_void_p()
        _check(lib.uk_ledger_open(str(path).encode(), C.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            lib.uk_ledger_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def key(kml_text: str, hcs_json: str | None = None) -> str:
        out = _buf(4096)
        if lib.uk_ledger_key(None if hcs_json is None else _text(hcs_json), _text(kml_text), out, len(out)) < 0:
            raise UnikernError(UK_BAD_INVOCATION, last_error())
        return out.value.decode()

    def lookup(self, kml_text: str, hcs_json: str | None = None) -> LedgerHit | None:
        p, c, m, k, hit = Plan(), C.c_double(), C.c_double(), C.c_double(), C.c_int32()
        _check(lib.uk_ledger_lookup(self._h, None if hcs_json is None else _text(hcs_json), _text(kml_text),
                                    C.byref(p), C.byref(c), C.byref(m), C.byref(k), C.byref(hit)))
        return LedgerHit(p, c.value, m.value, k.value) if hit.value else None

    def commit(self, kml_text: str, plan: Plan, measured_ms: float = 0.0, kernel_ms: float = 0.0,
               hcs_json: str | None = None, replayed: bool = False):
        _check(lib.uk_ledger_commit(self._h, None if hcs_json is None else _text(hcs_json), _text(kml_text),
                                    C.byref(plan), measured_ms, kernel_ms, 1 if replayed else 0))

    def record_violation(self, kml_text: str, rate: float, threshold: float, migrations: int, checks: int,
                         vram_free: int, hcs_json: str | None = None):
        _check(lib.uk_ledger_record_violation(self._h, None if hcs_json is None else _text(hcs_json),
                                              _text(kml_text), rate, threshold, migrations, checks, vram_free))

    def size(self) -> tuple[int, int]:
        s, v = C.c_int32(), C.c_int32()
        _check(lib.uk_ledger_size(self._h, C.byref(s), C.byref(v)))
        return s.value, v.value

    def measured(self, hcs_fp: str) -> list[tuple[float, float, float]]:
        n = lib.uk_ledger_measured(self._h, hcs_fp.encode(), None, 0)
        if n < 0:
            raise UnikernError(UK_BAD_INVOCATION, last_error())
        rows = (C.c_double * (3 * max(n, 1)))()
        lib.uk_ledger_measured(self._h, hcs_fp.encode(), rows, n)
        return [(rows[3 * i], rows[3 * i + 1], rows[3 * i + 2]) for i in range(n)]

    def calibrate(self, hcs_json: str | None = None, probe: dict | None = None) -> tuple[str, str]:
        """(calibrated HCS text, detail): hbm_bw_gbps, clock_mhz and link_bw_gbps refitted from this
        ledger's measured rows (and the matrix-core probe's clock when no MFMA-bound row exists)."""
        out, detail = _buf(1 << 16), _buf(1 << 16)
        pr = None
        if probe is not None:
            pr = MfmaProbe()
            pr.clock_ghz = float(probe["clock_ghz"])
            pr.tflops = float(probe.get("tflops", 0.0))
        rc = lib.uk_calibrate(None if hcs_json is None else _text(hcs_json), self._h,
                              None if pr is None else C.byref(pr), out, len(out), detail, len(detail))
        if rc != UK_OK:
            raise UnikernError(rc, detail.value.decode())
        return out.value.decode(), detail.value.decode()


def hcs_with_capacity(hcs_json: str | None, nbytes: int) -> str:
    out = _buf(1 << 16)
    _check(lib.uk_hcs_with_capacity(None if hcs_json is None else _text(hcs_json), nbytes, out, len(out)))
    return out.value.decode()


# ---------------------------------------------------------------------------------------
# GGUF weights
# ---------------------------------------------------------------------------------------
GGML_TYPES = {0: "f32", 1: "f16", 8: "q8_0", 30: "bf16"}


@dataclass
class GgufTensor:
    index: int
    name: str
    ggml_type: int
    ne: tuple
    offset: int
    nbytes: int

    @property
    def type_name(self) -> str:
        return GGML_TYPES.get(self.ggml_type, f"type{self.ggml_type}")


class Gguf:
    """Header, metadata and tensor directory of a GGUF file; tensor bytes to host or device."""

    def __init__(self, path: str | Path):
        h = C.c_void_p()
        _check(lib.uk_gguf_open(str(path).encode(), C.byref(h)))
        self._h = h

    def close(self):
        if self._h:
            lib.uk_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return lib.uk_gguf_tensor_count(self._h)

    def tensor(self, key: int | str) -> GgufTensor:
        idx = key if isinstance(key, int) else lib.uk_gguf_find(self._h, key.encode())
        if idx < 0:
            raise KeyError(key)
        name = _buf(4096)
        t, nd = C.c_int32(), C.c_int32()
        ne = (C.c_int64 * 4)()
        off, nb = C.c_uint64(), C.c_uint64()
        _check(lib.uk_gguf_tensor_info(self._h, idx, name, len(name), C.byref(t), C.byref(nd), ne, C.byref(off),
                                       C.byref(nb)))
        return GgufTensor(idx, name.value.decode(), t.value, tuple(ne[: nd.value]), off.value, nb.value)

    def tensors(self) -> list[GgufTensor]:
        return [self.tensor(i) for i in range(len(self))]

    def metadata(self, key: str) -> str | None:
        out = _buf(1 << 16)
        n = lib.uk_gguf_metadata(self._h, key.encode(), out, len(out))
        return None if n < 0 else out.value.decode()

    def read(self, key: int | str) -> np.ndarray:
        t = self.tensor(key)
        out = np.empty(t.nbytes, np.uint8)
        _check(lib.uk_gguf_read(self._h, t.index, out.ctypes.data_as(C.c_void_p), out.nbytes))
        return out

    def upload(self, key: int | str) -> "DeviceBuffer":
        t = self.tensor(key)
        buf = DeviceBuffer(t.nbytes)
        _check(lib.uk_gguf_upload(self._h, t.index, buf.ptr, t.nbytes))
        return buf

    def q8_0_desc(self, key: int | str, M: int) -> OpDesc:
        d = OpDesc()
        _check(lib.uk_gguf_q8_0_desc(self._h, self.tensor(key).index, M, C.byref(d)))
        return d
