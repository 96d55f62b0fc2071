"""ctypes declarations of include/unikern_hip.h.

Loading fails loudly when libunikern_hip.so is missing: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libunikern_hip.so"
ABI_VERSION = 4  # UK_ABI_VERSION of the header these declarations mirror

UK_OK, UK_VERIFY_FAIL, UK_BAD_INVOCATION, UK_INFEASIBLE, UK_HIP_FAILURE, UK_RESIDENCY = range(6)
OPS = {"gemm": 0, "conv": 1, "reduce": 2, "softmax": 3, "rmsnorm": 4, "channelscale": 5}
DTYPES = {"fp32": 0, "fp16": 1, "int8": 2, "q8_0": 3}
LAYOUTS = {"NT": 0, "TN": 1, "NCHW": 2}
FAMILIES = {0: "none", 1: "rows", 2: "rows_stream", 3: "channelscale", 4: "reduce1d", 5: "gemm_f16_mfma",
            6: "gemm_generic_mfma", 7: "conv_igemm_mfma", 8: "q8_0_gemm"}


class OpDesc(C.Structure):
    _fields_ = [("op", C.c_int32), ("dtype", C.c_int32), ("layout", C.c_int32), ("epilogue", C.c_int32),
                ("ndims", C.c_int32), ("dims", C.c_int32 * 6), ("tile_m", C.c_int32), ("tile_n", C.c_int32),
                ("batch", C.c_int32), ("pad", C.c_int32), ("stride", C.c_int32), ("eps", C.c_float),
                ("n_children", C.c_int32)]


class Plan(C.Structure):
    _fields_ = [("family", C.c_int32), ("variant", C.c_int32), ("tile_m", C.c_int32), ("tile_n", C.c_int32),
                ("tile_k", C.c_int32), ("threads", C.c_int32), ("tpr", C.c_int32), ("vec", C.c_int32),
                ("split_k", C.c_int32), ("stages", C.c_int32), ("grid", C.c_int64), ("predicted_us", C.c_double),
                ("feasible", C.c_int32), ("shard_rows", C.c_int32), ("stream_path", C.c_int32), ("key", C.c_char * 64)]


class Result(C.Structure):
    _fields_ = [("built", C.c_int32), ("ran", C.c_int32), ("verified", C.c_int32), ("exit_code", C.c_int32),
                ("max_rel", C.c_double), ("err_metric", C.c_double), ("tol", C.c_double), ("tol_kind", C.c_int32),
                ("kernel_ms", C.c_double), ("measured_ms", C.c_double), ("achieved", C.c_double),
                ("peak", C.c_double), ("frac", C.c_double), ("bound", C.c_int32), ("migrations", C.c_int32),
                ("checks", C.c_int32), ("vram_free", C.c_uint64), ("vram_total", C.c_uint64),
                ("algo_bytes", C.c_int64), ("algo_flops", C.c_int64), ("weight_bytes", C.c_int64),
                ("launches", C.c_int32), ("repeats", C.c_int32), ("sets", C.c_int32), ("plan", Plan),
                ("mode", C.c_char * 16), ("dtype", C.c_char * 8), ("perf", C.c_char * 48),
                ("cpu_ms", C.c_double), ("cpu_cores", C.c_int32), ("cpu_outputs", C.c_int64),
                ("stream_path", C.c_char * 8)]


class MfmaProbe(C.Structure):
    _fields_ = [("tflops", C.c_double), ("clock_ghz", C.c_double), ("cycles_per_mfma", C.c_double),
                ("ms_per_launch", C.c_double), ("workgroups", C.c_int32), ("mfmas_per_wave", C.c_int32),
                ("tflops_32x32", C.c_double), ("clock_ghz_32x32", C.c_double), ("cycles_per_mfma_32x32", C.c_double)]


_P = C.c_void_p
_SIG = {
    "uk_abi_version": ([], C.c_int),
    "uk_device_check": ([C.c_char_p, C.c_size_t], C.c_int),
    "uk_device_props": ([C.POINTER(C.c_int32)] * 3 + [C.POINTER(C.c_uint64)], C.c_int),
    "uk_probe_mfma": ([C.POINTER(MfmaProbe)], C.c_int),
    "uk_last_error": ([], C.c_char_p),
    "uk_kml_import": ([C.c_char_p, C.POINTER(OpDesc), C.c_char_p, C.c_size_t], C.c_int),
    "uk_kml_export": ([C.c_char_p, C.c_char_p, C.c_size_t], C.c_int),
    "uk_kml_canonical": ([C.c_char_p, C.c_char_p, C.c_size_t], C.c_int),
    "uk_kml_tree_hash": ([C.c_char_p, C.c_char_p, C.c_size_t], C.c_int),
    "uk_op_signature": ([C.POINTER(OpDesc), C.c_char_p, C.c_size_t], C.c_int),
    "uk_workload": ([C.POINTER(OpDesc), C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.POINTER(C.c_int64)], C.c_int),
    "uk_support_gap": ([C.POINTER(OpDesc), C.c_char_p, C.c_size_t], C.c_int),
    "uk_hcs_fingerprint": ([C.c_char_p, C.c_char_p, C.c_size_t], C.c_int),
    "uk_hcs_export": ([C.c_char_p, C.c_char_p, C.c_size_t], C.c_int),
    "uk_solve": ([C.c_char_p, C.POINTER(OpDesc), C.POINTER(Plan), C.c_char_p, C.c_size_t], C.c_int),
    "uk_launch": ([C.POINTER(OpDesc), C.POINTER(Plan), C.POINTER(_P), C.c_int32, _P, _P], C.c_int),
    "uk_launch_noalloc": ([C.POINTER(OpDesc), C.POINTER(Plan), C.POINTER(_P), C.c_int32, _P, _P], C.c_int),
    "uk_launch_n": ([C.POINTER(OpDesc), C.POINTER(Plan), C.POINTER(_P), C.c_int32, C.POINTER(_P), C.c_int32,
                     C.c_int32, _P], C.c_int),
    "uk_run": ([C.c_char_p, C.POINTER(OpDesc), C.POINTER(Plan), C.c_uint64, C.c_int32, C.c_int32, C.POINTER(Result),
                C.c_char_p, C.c_size_t], C.c_int),
    "uk_format_result": ([C.POINTER(Result), C.c_char_p, C.c_size_t], C.c_int),
    "uk_stream_gemm": ([C.c_char_p, C.POINTER(OpDesc), C.POINTER(Plan), _P, _P, _P, C.POINTER(C.c_double)], C.c_int),
    "uk_stream_gemm_file": ([C.c_char_p, C.POINTER(OpDesc), C.POINTER(Plan), C.c_char_p, _P, _P,
                             C.POINTER(C.c_double)], C.c_int),
    "uk_parse_result": ([C.c_char_p, C.c_int32, C.POINTER(Result)], C.c_int),
    "uk_migration_alarm": ([C.c_int32, C.c_int32, C.c_double, C.POINTER(C.c_double)], C.c_int),
    "uk_residency_class": ([C.c_int32, C.c_int32], C.c_int),
    "uk_fill_uniform": ([_P, C.c_size_t, C.c_uint64, C.c_float, C.c_float], C.c_int),
    "uk_fill_normal": ([_P, C.c_size_t, C.c_uint64, C.c_float, C.c_float], C.c_int),
    "uk_f32_to_f16": ([_P, _P, C.c_size_t], C.c_int),
    "uk_f16_to_f32": ([_P, _P, C.c_size_t], C.c_int),
    "uk_q8_0_pack": ([_P, _P, _P, C.c_int32, C.c_int32], C.c_int),
    "uk_ledger_open": ([C.c_char_p, C.POINTER(_P)], C.c_int),
    "uk_ledger_close": ([_P], C.c_int),
    "uk_ledger_key": ([C.c_char_p, C.c_char_p, C.c_char_p, C.c_size_t], C.c_int),
    "uk_ledger_lookup": ([_P, C.c_char_p, C.c_char_p, C.POINTER(Plan), C.POINTER(C.c_double), C.POINTER(C.c_double),
                          C.POINTER(C.c_double), C.POINTER(C.c_int32)], C.c_int),
    "uk_ledger_commit": ([_P, C.c_char_p, C.c_char_p, C.POINTER(Plan), C.c_double, C.c_double, C.c_int32], C.c_int),
    "uk_ledger_record_violation": ([_P, C.c_char_p, C.c_char_p, C.c_double, C.c_double, C.c_int32, C.c_int32,
                                    C.c_uint64], C.c_int),
    "uk_ledger_size": ([_P, C.POINTER(C.c_int32), C.POINTER(C.c_int32)], C.c_int),
    "uk_ledger_measured": ([_P, C.c_char_p, C.POINTER(C.c_double), C.c_int32], C.c_int),
    "uk_calibrate": ([C.c_char_p, _P, C.POINTER(MfmaProbe), C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t],
                     C.c_int),
    "uk_hcs_with_capacity": ([C.c_char_p, C.c_uint64, C.c_char_p, C.c_size_t], C.c_int),
    "uk_gguf_open": ([C.c_char_p, C.POINTER(_P)], C.c_int),
    "uk_gguf_close": ([_P], C.c_int),
    "uk_gguf_tensor_count": ([_P], C.c_int32),
    "uk_gguf_find": ([_P, C.c_char_p], C.c_int32),
    "uk_gguf_tensor_info": ([_P, C.c_int32, C.c_char_p, C.c_size_t, C.POINTER(C.c_int32), C.POINTER(C.c_int32),
                             C.POINTER(C.c_int64), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)], C.c_int),
    "uk_gguf_metadata": ([_P, C.c_char_p, C.c_char_p, C.c_size_t], C.c_int),
    "uk_gguf_read": ([_P, C.c_int32, _P, C.c_uint64], C.c_int),
    "uk_gguf_upload": ([_P, C.c_int32, _P, C.c_uint64], C.c_int),
    "uk_gguf_q8_0_desc": ([_P, C.c_int32, C.c_int32, C.POINTER(OpDesc)], C.c_int),
    "uk_malloc": ([C.POINTER(_P), C.c_size_t], C.c_int),
    "uk_free": ([_P], C.c_int),
    "uk_memcpy_htod": ([_P, _P, C.c_size_t], C.c_int),
    "uk_memcpy_dtoh": ([_P, _P, C.c_size_t], C.c_int),
    "uk_memset": ([_P, C.c_int, C.c_size_t], C.c_int),
    "uk_synchronize": ([], C.c_int),
    "uk_stream_create": ([C.POINTER(_P)], C.c_int),
    "uk_stream_destroy": ([_P], C.c_int),
    "uk_stream_synchronize": ([_P], C.c_int),
    "uk_event_create": ([C.POINTER(_P)], C.c_int),
    "uk_event_destroy": ([_P], C.c_int),
    "uk_event_record": ([_P, _P], C.c_int),
    "uk_event_elapsed_ms": ([_P, _P, C.POINTER(C.c_float)], C.c_int),
}

EXPORTED = tuple(_SIG)


def load(path: Path | str = LIB_PATH) -> C.CDLL:
    p = Path(path)
    if not p.exists():
        raise ImportError(
            f"{p} is missing: build it with `python3 unikern_amd/build.py` (or __graft_entry__.build()); "
            "the MI355X kernels have no fallback path")
    lib = C.CDLL(str(p))
    for name, (args, res) in _SIG.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if lib.uk_abi_version() != ABI_VERSION:
        raise ImportError(f"{p} reports ABI {lib.uk_abi_version()}, these declarations are ABI {ABI_VERSION}: "
                          "rebuild it with `python3 unikern_amd/build.py`")
    return lib
