"""HBM traffic per kernel launch from two rocprofv3 counter passes.

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d DIR_F -- python3 bench.py --no-cpu-baseline
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d DIR_W -- python3 bench.py --no-cpu-baseline
    python3 -m unikern_amd.traffic --fetch DIR_F --write DIR_W --out profiles/traffic.json

FETCH_SIZE and WRITE_SIZE are the TCC (L2) counters of bytes read from and written to memory,
reported in KiB per dispatch. They are calibrated against a kernel whose memory traffic is known
exactly: channelscale over X[4096][4096] f32 streams every input byte once and writes every output
byte once (2 * 64 MiB + 16 KiB), and bench.py launches it over rotating buffers so no launch hits
in the 256 MiB MALL. The calibration factor (algorithmic bytes / counter bytes) of that launch
scales the counter readings of every other kernel; traffic well above a kernel's algorithmic bytes
means re-reads.
"""
from __future__ import annotations

import argparse
import csv
import json
import re
from collections import defaultdict
from pathlib import Path

# Name patterns (demangled or mangled, as rocprofv3 prints them) of the kernels bench.py launches;
# rows_kernel<TPR, NV, op, ...> with op 0 row-sum, 1 RMSNorm, 2 softmax.
KERNELS = {
    "rowsum": re.compile(r"rows_kernel<\d+, \d+, 0[,>]"),
    "rmsnorm": re.compile(r"rows_kernel<\d+, \d+, 1[,>]"),
    "softmax": re.compile(r"rows_kernel<\d+, \d+, 2[,>]"),
    "copy": re.compile(r"rows_kernel<64, 16, 3[,>]"),
    "gemm_f16": re.compile(r"gemm_f16_(tn|pp|w4|w4s|w4k|w4k16)_kernel"),
    "gemm_f32": re.compile(r"gemm_f32_kernel"),
    "gemm_generic": re.compile(r"gemm_generic_kernel"),
    "conv": re.compile(r"conv_igemm_kernel|conv_tile_kernel|conv_lds_kernel|conv_lds16_kernel"),
    "q8_0": re.compile(r"q8_0_gemm_kernel|q8_0_gemv_kernel"),
}
COPY_BYTES_READ = 4096 * 4096 * 4 + 4096 * 4
COPY_BYTES_WRITTEN = 4096 * 4096 * 4


def read_counter(directory: Path, counter: str) -> dict[str, list[float]]:
    """Per kernel family: counter value (bytes) of every dispatch found in the pass's CSV files.
    A family launched with several grid sizes is split into "family@grid" entries."""
    out: dict[str, list[float]] = defaultdict(list)
    files = sorted(directory.rglob("*counter_collection.csv"))
    if not files:
        raise FileNotFoundError(f"no *counter_collection.csv under {directory}")
    for f in files:
        with open(f, newline="") as fh:
            for row in csv.DictReader(fh):
                if row["Counter_Name"] != counter:
                    continue
                for name, pat in KERNELS.items():
                    if pat.search(row["Kernel_Name"]):
                        v = float(row["Counter_Value"]) * 1024.0  # KiB -> bytes
                        out[name].append(v)
                        out[f"{name}@{row['Grid_Size']}"].append(v)
    # keep the per-grid split only where a family ran with more than one grid
    for name in KERNELS:
        grids = [k for k in out if k.startswith(name + "@")]
        if len(grids) == 1:
            del out[grids[0]]
        elif grids:
            del out[name]
    return out


def summarize(fetch_dir: Path, write_dir: Path) -> dict:
    fetch = read_counter(fetch_dir, "FETCH_SIZE")
    write = read_counter(write_dir, "WRITE_SIZE")
    if not fetch.get("copy") or not write.get("copy"):
        raise RuntimeError("the channelscale calibration launches are missing from the counter passes")
    # the calibration launches are the steady-state ones (the first touches cold pages)
    med = lambda v: sorted(v)[len(v) // 2]  # noqa: E731
    f_factor = COPY_BYTES_READ / med(fetch["copy"])
    w_factor = COPY_BYTES_WRITTEN / med(write["copy"])
    res = {"_calibration": {"kernel": "channelscale (row form) 4096x4096 f32", "algorithmic_read": COPY_BYTES_READ,
                            "algorithmic_written": COPY_BYTES_WRITTEN, "fetch_factor": round(f_factor, 4),
                            "write_factor": round(w_factor, 4), "dispatches": [len(fetch["copy"]), len(write["copy"])]}}
    for name in sorted(fetch):
        if name.startswith("copy") or not write.get(name):
            continue
        rd, wr = med(fetch[name]) * f_factor, med(write[name]) * w_factor
        res[name] = {"read_bytes": int(rd), "written_bytes": int(wr), "bytes": int(rd + wr),
                     "dispatches": [len(fetch[name]), len(write[name])]}
    return res


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--fetch", type=Path, required=True)
    ap.add_argument("--write", type=Path, required=True)
    ap.add_argument("--out", type=Path, required=True)
    a = ap.parse_args()
    res = summarize(a.fetch, a.write)
    a.out.write_text(json.dumps(res, indent=1) + "\n")
    print(json.dumps(res))


if __name__ == "__main__":
    main()
